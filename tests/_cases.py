"""Shared builders for the parity tests: seeded random encodings (CPU) in every
layout the library accepts, and the oracle's weight / contraction for them."""
from __future__ import annotations

import torch

from oracle import c_oracle
from wal2026_amd.block_vq import BlockRVQEncoding, GroupedBlockRVQEncoding, _id_storage_dtype


def make_encoding(out_features: int, in_features: int, *, d: int = 8, S: int = 2, K: int = 256,
                  id_dtype: torch.dtype | None = None, group_rows: int | None = None,
                  cb_dtype: torch.dtype = torch.float16, stage_scales: bool = False, block_scale: bool = False,
                  stages_per_split: tuple[int, ...] | None = None, product_splits: int = 1,
                  special: bool = False, seed: int = 0, scale_dtype: torch.dtype = torch.float16,
                  scale_run: int | None = None) -> GroupedBlockRVQEncoding:
    """scale_run: rows of a group share their row scale in aligned runs of
    that many rows (a per-row-group scale expanded to rows)."""
    g = torch.Generator().manual_seed(seed)
    id_dtype = id_dtype or _id_storage_dtype(K)
    B = -(-in_features // d)
    group_rows = group_rows or out_features
    slices = [(r0, min(r0 + group_rows, out_features)) for r0 in range(0, out_features, group_rows)]
    groups = []
    for r0, r1 in slices:
        rows = r1 - r0
        cbs = []
        for _ in range(S):
            cb = torch.randn(K, d, generator=g) * 0.02
            if special:
                # fp16 subnormals, signed zeros, tiny and large values, exact ties
                flat = cb.view(-1)
                n = flat.numel()
                pick = torch.randperm(n, generator=g)
                q = max(n // 16, 1)
                flat[pick[:q]] = torch.randint(1, 1024, (q,), generator=g).float() * 2.0 ** -24
                flat[pick[q:2 * q]] = 0.0
                flat[pick[2 * q:3 * q]] = -0.0
                flat[pick[3 * q:4 * q]] = (torch.rand(q, generator=g) - 0.5) * 1000.0
                flat[pick[4 * q:5 * q]] = torch.randint(-64, 64, (q,), generator=g).float() * 2.0 ** -9
            cbs.append(cb.to(cb_dtype))
        if id_dtype == torch.uint16:
            ids = [torch.randint(0, K, (rows, B), generator=g, dtype=torch.int32).to(torch.uint16) for _ in range(S)]
        else:
            ids = [torch.randint(0, K, (rows, B), generator=g).to(id_dtype) for _ in range(S)]
        rs = (torch.rand(rows, 1, generator=g) + 0.5)
        if special:
            rs[: max(rows // 8, 1)] = torch.randint(1, 64, (max(rows // 8, 1), 1), generator=g).float() * 2.0 ** -6
        if scale_run:
            rs = rs[::scale_run].repeat_interleave(scale_run, dim=0)[:rows]
        rs = rs.to(scale_dtype)
        ss = (torch.rand(S, generator=g) + 0.5).to(scale_dtype) if stage_scales else None
        bs = (torch.rand(rows, B, generator=g) + 0.5).to(scale_dtype) if block_scale else None
        spl = stages_per_split or (S,)
        groups.append(BlockRVQEncoding(
            stage_ids=tuple(ids), codebooks=tuple(cbs), stage_value_dims=(d,) * S, stages_per_split=spl,
            stage_scales=ss, residual_correction="none", residual_signs=None, residual_scale=None,
            row_scale=rs, block_scale=bs, transform_kind="none", transform_matrix=None, transform_bias=None,
            product_splits=product_splits, original_shape=(rows, in_features), padded_cols=B * d, block_size=d,
            sample_rel_mse=0.0))
    return GroupedBlockRVQEncoding(groups=tuple(groups), row_slices=tuple(slices),
                                   original_shape=(out_features, in_features))


def oracle_group(group_enc: BlockRVQEncoding) -> c_oracle.OracleGroup:
    return c_oracle.OracleGroup(group_enc.stage_ids, [c.to(torch.float16) if c.dtype == torch.float16 else c
                                                      for c in group_enc.codebooks],
                                group_enc.row_scale, in_features=group_enc.original_shape[1],
                                block_size=group_enc.block_size, stage_scales=group_enc.stage_scales,
                                block_scale=group_enc.block_scale)


def oracle_weight(enc: GroupedBlockRVQEncoding, out_dtype: torch.dtype, active=None) -> torch.Tensor:
    """Reference dequantisation of every group, concatenated (CPU)."""
    parts = []
    for g in enc.groups:
        og = oracle_group(g)
        if active is None:
            parts.append(c_oracle.reconstruct_weight(og, out_dtype))
        else:
            parts.append(c_oracle.reconstruct_weight_fast(og, active, out_dtype))
    return torch.cat(parts, 0)


def module_buffers_as_encoding(module) -> GroupedBlockRVQEncoding:
    """The module's (fp16-converted) buffers back as an encoding on the CPU, so
    the oracle sees exactly what the kernels read."""
    groups = []
    for grp in module.groups:
        S = grp.num_stages
        groups.append(BlockRVQEncoding(
            stage_ids=tuple(getattr(grp, f"stage_ids_{i}").cpu() for i in range(S)),
            codebooks=tuple(getattr(grp, f"codebook_{i}").cpu() for i in range(S)),
            stage_value_dims=(grp.block_size,) * S, stages_per_split=grp.stages_per_split,
            stage_scales=None if grp.stage_scales is None else grp.stage_scales.cpu(),
            residual_correction="none", residual_signs=None, residual_scale=None,
            row_scale=grp.row_scale.cpu(), block_scale=None if grp.block_scale is None else grp.block_scale.cpu(),
            transform_kind="none", transform_matrix=None, transform_bias=None, product_splits=grp.product_splits,
            original_shape=(grp.out_features, grp.in_features), padded_cols=grp.padded_cols,
            block_size=grp.block_size, sample_rel_mse=0.0))
    return GroupedBlockRVQEncoding(groups=tuple(groups), row_slices=module.row_slices,
                                   original_shape=(module.out_features, module.in_features))


def rel_err(y: torch.Tensor, ref: torch.Tensor) -> float:
    """max|y - ref| / max|ref|, the parity metric (tolerance 2e-3)."""
    y = y.double().cpu()
    ref = ref.double().cpu()
    return float((y - ref).abs().max() / ref.abs().max().clamp_min(1e-30))


def bits(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous().cpu()
    if t.dtype == torch.float32:
        return t.view(torch.int32)
    return t.view(torch.int16)
