"""Function-level drop-ins for the reference's fused kernels
(src/triton_id_matmul.py), backed by libwal2026_amd.so.

Same signatures and argument checks (ValueError for device, rank, stage and
feature mismatches).  The tuning keyword arguments of the Triton versions
(``autotuned``, ``block_m``, ``block_n``, ``block_k``) are accepted and
ignored: tile shapes are fixed by the HIP kernels.
"""
from __future__ import annotations

import torch

from . import _lib


def rvq_group_linear_matmul(
    x: torch.Tensor,
    stage_ids: torch.Tensor,
    codebooks: torch.Tensor,
    row_scale: torch.Tensor,
    *,
    autotuned: bool = True,
    block_m: int = 32,
    block_n: int = 32,
) -> torch.Tensor:
    """out[..., n] = (sum_k x[..., k] * x_dtype(sum_s cb[s, ids[s, n, k // d], k % d])) * rho[n]
    (src/triton_id_matmul.py:220-306).  Any block size and 8/16/32-bit ids."""
    del autotuned, block_m, block_n
    if not x.is_cuda or not stage_ids.is_cuda or not codebooks.is_cuda or not row_scale.is_cuda:
        raise ValueError("rvq_group_linear_matmul expects CUDA tensors")
    if stage_ids.ndim != 3:
        raise ValueError(f"expected stage_ids to have shape [stages, rows, blocks], got {tuple(stage_ids.shape)}")
    if codebooks.ndim != 3:
        raise ValueError(f"expected codebooks to have shape [stages, codebook, block], got {tuple(codebooks.shape)}")
    if stage_ids.shape[0] != codebooks.shape[0]:
        raise ValueError(f"stage mismatch: {stage_ids.shape[0]} != {codebooks.shape[0]}")
    dev = _lib.require_rocm(x, stage_ids, codebooks, row_scale)
    orig = x.shape
    x2 = x.reshape(-1, orig[-1]).contiguous()
    ids = stage_ids.contiguous()
    cbs = codebooks.contiguous()
    rho = row_scale.reshape(-1).contiguous()
    m, k = x2.shape
    S, n, bpr = ids.shape
    d = int(cbs.shape[2])
    if bpr * d != k:
        raise ValueError(f"Feature mismatch: expected {bpr * d}, got {k}")
    if rho.numel() != n:
        raise ValueError(f"Row-scale mismatch: {n} != {rho.numel()}")
    if ids.numel():
        lo, hi = _lib.id_range(ids)
        if lo < 0 or hi >= cbs.shape[1]:
            raise IndexError(f"stage_ids hold index range [{lo}, {hi}] outside [0, {cbs.shape[1]})")
    out = torch.empty(m, n, dtype=x.dtype, device=dev)
    _lib.check(_lib.lib().wal_rvq_group_linear_matmul(
        x2.data_ptr(), m, k, _lib.float_tag(x2.dtype), ids.data_ptr(), _lib.id_tag(ids.dtype), S, n, bpr,
        cbs.data_ptr(), _lib.float_tag(cbs.dtype), cbs.shape[1], d, rho.data_ptr(), _lib.float_tag(rho.dtype),
        out.data_ptr(), _lib.float_tag(out.dtype), _lib.stream_ptr(dev)))
    return out.reshape(*orig[:-1], n)


def id_route_linear_matmul(
    x: torch.Tensor,
    ids: torch.Tensor,
    codebook_sum: torch.Tensor,
    row_scale: torch.Tensor,
    *,
    autotuned: bool = True,
    block_m: int = 32,
    block_n: int = 32,
    block_k: int = 32,
) -> torch.Tensor:
    """out = x @ (x_dtype(lut[ids]) * x_dtype(rho))^T, accumulated in fp32 and
    stored in x dtype (src/triton_id_matmul.py:70-140)."""
    del autotuned, block_m, block_n, block_k
    if not x.is_cuda or not ids.is_cuda or not codebook_sum.is_cuda or not row_scale.is_cuda:
        raise ValueError("id_route_linear_matmul expects CUDA tensors")
    if x.shape[-1] != ids.shape[1]:
        raise ValueError(f"Feature mismatch: {x.shape[-1]} != {ids.shape[1]}")
    if ids.shape[0] != row_scale.numel():
        raise ValueError(f"Row-scale mismatch: {ids.shape[0]} != {row_scale.numel()}")
    dev = _lib.require_rocm(x, ids, codebook_sum, row_scale)
    orig = x.shape
    x2 = x.reshape(-1, orig[-1]).contiguous()
    ids2 = ids.contiguous()
    lut = codebook_sum.contiguous()
    rho = row_scale.reshape(-1).contiguous()
    if rho.dtype != lut.dtype:
        raise ValueError(f"row_scale dtype {rho.dtype} must match codebook_sum dtype {lut.dtype}")
    n, k = ids2.shape
    if ids2.numel():
        lo, hi = _lib.id_range(ids2)
        if lo < 0 or hi >= lut.numel():
            raise IndexError(f"ids hold index range [{lo}, {hi}] outside [0, {lut.numel()})")
    out = torch.empty(x2.shape[0], n, dtype=x.dtype, device=dev)
    _lib.check(_lib.lib().wal_id_route_linear(
        x2.data_ptr(), x2.shape[0], k, _lib.float_tag(x2.dtype), ids2.data_ptr(), _lib.id_tag(ids2.dtype), n,
        lut.data_ptr(), lut.numel(), _lib.float_tag(lut.dtype), rho.data_ptr(), None, _lib.F32, 1,
        out.data_ptr(), _lib.float_tag(out.dtype), _lib.stream_ptr(dev)))
    return out.reshape(*orig[:-1], n)
