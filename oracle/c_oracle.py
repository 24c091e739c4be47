"""ctypes binding of the C oracle (rvq_oracle.c).  TEST INFRASTRUCTURE ONLY.

Takes CPU torch tensors (torch is plumbing here: it carries fp16/bf16 bits and
owns the memory).  Builds ``oracle/_build/librvq_oracle.so`` with ``make`` on
first use if it is missing.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import torch

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "_build" / "librvq_oracle.so"

OR_U8, OR_I16, OR_U16, OR_I32 = 0, 1, 2, 3
OR_F16, OR_BF16, OR_F32 = 10, 11, 12
MAX_STAGES = 8

_FLOAT_TAG = {torch.float16: OR_F16, torch.bfloat16: OR_BF16, torch.float32: OR_F32}
_ID_TAG = {torch.uint8: OR_U8, torch.int16: OR_I16, torch.uint16: OR_U16, torch.int32: OR_I32}
_TAG_DTYPE = {OR_F16: torch.float16, OR_BF16: torch.bfloat16, OR_F32: torch.float32}


class _Group(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_int32),
        ("in_features", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("blocks_per_row", ctypes.c_int32),
        ("codebook_size", ctypes.c_int32),
        ("num_stages", ctypes.c_int32),
        ("id_dtype", ctypes.c_int32),
        ("cb_dtype", ctypes.c_int32),
        ("rs_dtype", ctypes.c_int32),
        ("ss_dtype", ctypes.c_int32),
        ("bs_dtype", ctypes.c_int32),
        ("scale_rows", ctypes.c_int32),
        ("stage_ids", ctypes.c_void_p * MAX_STAGES),
        ("codebooks", ctypes.c_void_p * MAX_STAGES),
        ("stage_scales", ctypes.c_void_p),
        ("row_scale", ctypes.c_void_p),
        ("block_scale", ctypes.c_void_p),
    ]


_lib = None


def build() -> Path:
    """Compile the oracle with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        L.or_f32_to_bf16.restype = ctypes.c_uint16
        L.or_f32_to_bf16.argtypes = [ctypes.c_float]
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_reconstruct_weight.restype = ctypes.c_int
        L.or_reconstruct_weight.argtypes = [ctypes.POINTER(_Group), ctypes.c_int, ctypes.c_void_p]
        L.or_stagewise_linear.restype = ctypes.c_int
        L.or_stagewise_linear.argtypes = [ctypes.POINTER(_Group), ctypes.c_void_p, ctypes.c_int, ctypes.c_int64,
                                          ctypes.c_void_p]
        L.or_reconstruct_weight_fast.restype = ctypes.c_int
        L.or_reconstruct_weight_fast.argtypes = [ctypes.POINTER(_Group), ctypes.c_uint32, ctypes.c_int, ctypes.c_void_p]
        L.or_linear_f64.restype = None
        L.or_linear_f64.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                    ctypes.c_void_p, ctypes.c_int, ctypes.c_int64,
                                    ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        L.or_triton_rvq_matmul.restype = None
        L.or_triton_rvq_matmul.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                           ctypes.c_void_p, ctypes.c_int, ctypes.c_int32,
                                           ctypes.c_int64, ctypes.c_int64,
                                           ctypes.c_void_p, ctypes.c_int, ctypes.c_int64,
                                           ctypes.c_int32, ctypes.c_void_p, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_void_p]
        L.or_id_route_weight.restype = None
        L.or_id_route_weight.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_int64,
                                         ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
        L.or_centroid_sums.restype = ctypes.c_int
        L.or_centroid_sums.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_int64,
                                       ctypes.c_void_p, ctypes.c_void_p]
        L.or_assign.restype = None
        L.or_assign.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                ctypes.c_void_p, ctypes.c_void_p]
        _lib = L
    return _lib


def _cpu(t: torch.Tensor | None) -> torch.Tensor | None:
    if t is None:
        return None
    return t.detach().to("cpu").contiguous()


class OracleGroup:
    """Host copy of one group's buffers plus the C struct that points at them."""

    def __init__(self, stage_ids, codebooks, row_scale, *, in_features, block_size,
                 stage_scales=None, block_scale=None, scale_rows=1):
        self.ids = [_cpu(t) for t in stage_ids]
        self.cbs = [_cpu(t) for t in codebooks]
        self.rs = _cpu(row_scale).reshape(-1)
        self.ss = _cpu(stage_scales)
        self.bs = _cpu(block_scale)
        if len(self.ids) != len(self.cbs) or not 1 <= len(self.ids) <= MAX_STAGES:
            raise ValueError("stage count mismatch")
        cb_dtypes = {c.dtype for c in self.cbs}
        if len(cb_dtypes) != 1:
            raise ValueError("codebooks must share one dtype")
        rows, bpr = self.ids[0].shape
        g = _Group()
        g.rows = rows
        g.in_features = in_features
        g.block_size = block_size
        g.blocks_per_row = bpr
        g.codebook_size = self.cbs[0].shape[0]
        g.num_stages = len(self.ids)
        g.id_dtype = _ID_TAG[self.ids[0].dtype]
        g.cb_dtype = _FLOAT_TAG[self.cbs[0].dtype]
        g.rs_dtype = _FLOAT_TAG[self.rs.dtype]
        g.ss_dtype = _FLOAT_TAG[self.ss.dtype] if self.ss is not None else OR_F32
        g.bs_dtype = _FLOAT_TAG[self.bs.dtype] if self.bs is not None else OR_F32
        g.scale_rows = scale_rows
        for i, (a, c) in enumerate(zip(self.ids, self.cbs)):
            g.stage_ids[i] = a.data_ptr()
            g.codebooks[i] = c.data_ptr()
        g.stage_scales = self.ss.data_ptr() if self.ss is not None else None
        g.row_scale = self.rs.data_ptr()
        g.block_scale = self.bs.data_ptr() if self.bs is not None else None
        self.struct = g
        self.rows = rows
        self.in_features = in_features

    @classmethod
    def from_module_group(cls, group) -> "OracleGroup":
        """Read the buffers of a PackedBlockRVQGroup-like object."""
        S = group.num_stages
        return cls(
            [getattr(group, f"stage_ids_{i}") for i in range(S)],
            [getattr(group, f"codebook_{i}") for i in range(S)],
            group.row_scale,
            in_features=group.in_features,
            block_size=group.block_size,
            stage_scales=getattr(group, "stage_scales", None),
            block_scale=getattr(group, "block_scale", None),
        )


def reconstruct_weight(g: OracleGroup, out_dtype: torch.dtype) -> torch.Tensor:
    out = torch.empty(g.rows, g.in_features, dtype=out_dtype)
    rc = lib().or_reconstruct_weight(ctypes.byref(g.struct), _FLOAT_TAG[out_dtype], out.data_ptr())
    if rc != 0:
        raise ValueError(f"or_reconstruct_weight failed ({rc})")
    return out


def reconstruct_weight_fast(g: OracleGroup, active_stages, out_dtype: torch.dtype) -> torch.Tensor:
    mask = 0
    for s in active_stages:
        mask |= 1 << int(s)
    out = torch.empty(g.rows, g.in_features, dtype=out_dtype)
    rc = lib().or_reconstruct_weight_fast(ctypes.byref(g.struct), mask, _FLOAT_TAG[out_dtype], out.data_ptr())
    if rc != 0:
        raise ValueError(f"or_reconstruct_weight_fast failed ({rc})")
    return out


def stagewise_linear(g: OracleGroup, x: torch.Tensor) -> torch.Tensor:
    """stagewise_block_matmul of one group (src/runtime.py:878-894), y in x dtype."""
    x = _cpu(x)
    y = torch.empty(x.shape[0], g.rows, dtype=x.dtype)
    rc = lib().or_stagewise_linear(ctypes.byref(g.struct), x.data_ptr(), _FLOAT_TAG[x.dtype], x.shape[0], y.data_ptr())
    if rc != 0:
        raise ValueError(f"or_stagewise_linear failed ({rc})")
    return y


def linear_f64(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """y = x @ w.T (+ bias) in float64 over the exact values of x, w, bias."""
    x = _cpu(x)
    w = _cpu(w)
    b = _cpu(bias)
    m, k = x.shape
    n = w.shape[0]
    y = torch.empty(m, n, dtype=torch.float64)
    lib().or_linear_f64(x.data_ptr(), _FLOAT_TAG[x.dtype], m, k, w.data_ptr(), _FLOAT_TAG[w.dtype], n,
                        b.data_ptr() if b is not None else None,
                        _FLOAT_TAG[b.dtype] if b is not None else OR_F32, y.data_ptr())
    return y


def triton_rvq_matmul(x, stage_ids, codebooks, row_scale, out_dtype=None) -> torch.Tensor:
    """rvq_group_linear_matmul semantics; stage_ids [S, N, B], codebooks [S, K, d]."""
    x = _cpu(x)
    ids = _cpu(stage_ids)
    cbs = _cpu(codebooks)
    rs = _cpu(row_scale).reshape(-1)
    out_dtype = out_dtype or x.dtype
    m, in_features = x.shape
    S, N, B = ids.shape
    out = torch.empty(m, N, dtype=out_dtype)
    lib().or_triton_rvq_matmul(x.data_ptr(), _FLOAT_TAG[x.dtype], m, in_features,
                               ids.data_ptr(), _ID_TAG[ids.dtype], S, N, B,
                               cbs.data_ptr(), _FLOAT_TAG[cbs.dtype], cbs.shape[1], cbs.shape[2],
                               rs.data_ptr(), _FLOAT_TAG[rs.dtype], _FLOAT_TAG[out_dtype], out.data_ptr())
    return out


def id_route_weight(ids, codebook_sum, row_scale, *, mode: int, x_dtype: torch.dtype) -> torch.Tensor:
    """Dense route-codebook weight in x_dtype (mode 0: PackedIDRouteLinear, 1: fused)."""
    ids = _cpu(ids)
    cs = _cpu(codebook_sum)
    rs = _cpu(row_scale).reshape(-1)
    n, k = ids.shape
    out = torch.empty(n, k, dtype=x_dtype)
    lib().or_id_route_weight(ids.data_ptr(), _ID_TAG[ids.dtype], n, k, cs.data_ptr(), _FLOAT_TAG[cs.dtype],
                             rs.data_ptr(), _FLOAT_TAG[rs.dtype], mode, _FLOAT_TAG[x_dtype], out.data_ptr())
    return out


def assign(blocks: torch.Tensor, codebook: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Nearest codeword of every block (or_assign; reference src/block_vq.py:180-196)."""
    b = _cpu(blocks).to(torch.float32).contiguous()
    c = _cpu(codebook).to(torch.float32).contiguous()
    n, d = b.shape
    ids = torch.empty(n, dtype=torch.int64)
    dist = torch.empty(n, dtype=torch.float32)
    lib().or_assign(b.data_ptr(), n, d, c.data_ptr(), c.shape[0], ids.data_ptr(), dist.data_ptr())
    return ids, dist


def centroid_sums(ids: torch.Tensor, blocks: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(sums [k, d] fp32, counts [k] int64) of the k-means update (or_centroid_sums;
    reference src/block_vq.py:216-218)."""
    i = _cpu(ids).to(torch.int64).contiguous()
    b = _cpu(blocks).to(torch.float32).contiguous()
    n, d = b.shape
    sums = torch.empty(k, d, dtype=torch.float32)
    counts = torch.empty(k, dtype=torch.int64)
    if lib().or_centroid_sums(i.data_ptr(), n, b.data_ptr(), d, k, sums.data_ptr(), counts.data_ptr()) != 0:
        raise IndexError("ids outside [0, k)")
    return sums, counts
