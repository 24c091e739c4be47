"""ctypes binding of libwal2026_amd.so (the C ABI declared in include/wal2026_amd.h).

The library is required: every entry point here raises if it is missing or if
the tensors are not on a ROCm device.  There is no CPU or torch fallback.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libwal2026_amd.so"
TORCH_OPS_PATH = Path(__file__).resolve().parent / "_lib" / "libwal2026_amd_torch.so"

MAX_STAGES = 8
ABI_VERSION = 4

# wal_dtype
U8, I16, U16, I32 = 0, 1, 2, 3
F16, BF16, F32 = 10, 11, 12

# wal_rvq_semantics
RECONSTRUCT, RECONSTRUCT_FAST, STAGEWISE = 0, 1, 2

# wal_status
OK, EINVAL, EUNSUPPORTED, EHIP, ESIZE = 0, -1, -2, -3, -4

FLOAT_DTYPES = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}
ID_DTYPES = {torch.uint8: U8, torch.int16: I16, torch.uint16: U16, torch.int32: I32}

# Every symbol include/wal2026_amd.h declares.
EXPORTED_SYMBOLS = (
    "wal_rvq_plan_size",
    "wal_rvq_plan_build",
    "wal_rvq_image_size",
    "wal_rvq_image_build",
    "wal_rvq_reconstruct",
    "wal_rvq_linear",
    "wal_rvq_linear_ws",
    "wal_rvq_linear_noalloc",
    "wal_rvq_linear_workspace_size",
    "wal_rvq_linear_info",
    "wal_rvq_group_linear_matmul",
    "wal_id_route_linear",
    "wal_id_route_reconstruct",
    "wal_rvq_assign",
    "wal_rvq_centroid_sums",
    "wal_read_probe",
    "wal_last_error",
    "wal_abi_version",
)


class WalGroup(ctypes.Structure):
    """struct wal_rvq_group."""

    _fields_ = [
        ("stage_ids", ctypes.c_void_p * MAX_STAGES),
        ("codebooks", ctypes.c_void_p * MAX_STAGES),
        ("stage_scales", ctypes.c_void_p),
        ("row_scale", ctypes.c_void_p),
        ("block_scale", ctypes.c_void_p),
        ("row0", ctypes.c_int32),
        ("rows", ctypes.c_int32),
    ]


class WalLayer(ctypes.Structure):
    """struct wal_rvq_layer."""

    _fields_ = [
        ("in_features", ctypes.c_int32),
        ("out_features", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("blocks_per_row", ctypes.c_int32),
        ("codebook_size", ctypes.c_int32),
        ("num_stages", ctypes.c_int32),
        ("id_dtype", ctypes.c_int32),
        ("codebook_dtype", ctypes.c_int32),
        ("scale_dtype", ctypes.c_int32),
        ("scale_rows", ctypes.c_int32),
        ("n_groups", ctypes.c_int32),
        ("image_tag", ctypes.c_int32),
        ("groups", ctypes.POINTER(WalGroup)),
        ("plan", ctypes.c_void_p),
        ("image", ctypes.c_void_p),
    ]


# wal_rvq_launch_info.kernel / x_mode / tile_shape
KERNEL_NONE, KERNEL_DECODE, KERNEL_PREFILL, KERNEL_GENERIC = 0, 1, 2, 3
XMODE_GLOBAL, XMODE_LDS, XMODE_REG, XMODE_GREG, XMODE_GTR = 0, 1, 2, 3, 4
XMODE_NAMES = {XMODE_GLOBAL: "global", XMODE_LDS: "lds", XMODE_REG: "reg", XMODE_GREG: "greg", XMODE_GTR: "gtr"}
TILE_SHORT, TILE_TALL, TILE_WIDE = 0, 1, 2


class WalLaunchInfo(ctypes.Structure):
    """struct wal_rvq_launch_info."""

    _fields_ = [
        ("kernel", ctypes.c_int32),
        ("x_mode", ctypes.c_int32),
        ("table_slots", ctypes.c_int32),
        ("grid", ctypes.c_int32),
        ("share", ctypes.c_int32),
        ("lds_bytes", ctypes.c_int32),
        ("tile_shape", ctypes.c_int32),
        ("k_splits", ctypes.c_int32),
    ]


def image_tag(semantics: int, x_dtype_tag: int) -> int:
    """WAL_RVQ_IMAGE_TAG(semantics, x_dtype)."""
    return 0x1000 | (semantics & 0xF) | ((x_dtype_tag & 0xFF) << 4)


class WalError(RuntimeError):
    """An error status returned by libwal2026_amd (raised as RuntimeError, the
    type the reference's fused-kernel callers catch, src/runtime.py:1655-1661)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"wal2026_amd error {status}: {message}")
        self.status = status


_lib: ctypes.CDLL | None = None


def _declare(L: ctypes.CDLL) -> None:
    vp, i32, i64, u32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint32, ctypes.c_size_t
    L.wal_last_error.restype = ctypes.c_char_p
    L.wal_last_error.argtypes = []
    L.wal_abi_version.restype = i32
    L.wal_abi_version.argtypes = []
    L.wal_rvq_plan_size.restype = i32
    L.wal_rvq_plan_size.argtypes = [ctypes.POINTER(WalLayer), ctypes.POINTER(sz)]
    L.wal_rvq_plan_build.restype = i32
    L.wal_rvq_plan_build.argtypes = [ctypes.POINTER(WalLayer), vp, sz]
    L.wal_rvq_image_size.restype = i32
    L.wal_rvq_image_size.argtypes = [ctypes.POINTER(WalLayer), i32, i32, ctypes.POINTER(sz)]
    L.wal_rvq_image_build.restype = i32
    L.wal_rvq_image_build.argtypes = [ctypes.POINTER(WalLayer), i32, i32, vp, sz, vp]
    L.wal_rvq_reconstruct.restype = i32
    L.wal_rvq_reconstruct.argtypes = [ctypes.POINTER(WalLayer), i32, u32, vp, i32, vp]
    L.wal_rvq_linear.restype = i32
    L.wal_rvq_linear.argtypes = [ctypes.POINTER(WalLayer), i32, u32, vp, i64, i32, vp, i32, vp, i32, vp]
    L.wal_rvq_linear_ws.restype = i32
    L.wal_rvq_linear_ws.argtypes = [ctypes.POINTER(WalLayer), i32, u32, vp, i64, i32, vp, i32, vp, i32, vp, sz, vp]
    L.wal_rvq_linear_noalloc.restype = i32
    L.wal_rvq_linear_noalloc.argtypes = [ctypes.POINTER(WalLayer), i32, u32, vp, i64, i32, vp, i32, vp, i32, vp]
    L.wal_rvq_linear_workspace_size.restype = i32
    L.wal_rvq_linear_workspace_size.argtypes = [ctypes.POINTER(WalLayer), i32, vp, i64, i32, ctypes.POINTER(sz)]
    L.wal_rvq_linear_info.restype = i32
    L.wal_rvq_linear_info.argtypes = [ctypes.POINTER(WalLayer), i32, vp, i64, i32, ctypes.POINTER(WalLaunchInfo)]
    L.wal_rvq_group_linear_matmul.restype = i32
    L.wal_rvq_group_linear_matmul.argtypes = [vp, i64, i64, i32, vp, i32, ctypes.c_int32, i64, i64, vp, i32, i64,
                                              ctypes.c_int32, vp, i32, vp, i32, vp]
    L.wal_id_route_linear.restype = i32
    L.wal_id_route_linear.argtypes = [vp, i64, i64, i32, vp, i32, i64, vp, i64, i32, vp, vp, i32, i32, vp, i32, vp]
    L.wal_id_route_reconstruct.restype = i32
    L.wal_id_route_reconstruct.argtypes = [vp, i32, i64, i64, vp, i64, i32, vp, i32, i32, vp, vp]
    L.wal_rvq_assign.restype = i32
    L.wal_rvq_assign.argtypes = [vp, i64, i32, vp, i64, vp, vp, vp]
    L.wal_rvq_centroid_sums.restype = i32
    L.wal_rvq_centroid_sums.argtypes = [vp, i64, vp, i32, i64, vp, vp, vp]
    L.wal_read_probe.restype = i32
    L.wal_read_probe.argtypes = [vp, i64, vp, i32, i32, vp]


def lib() -> ctypes.CDLL:
    """Load the library (raises if it was not built)."""
    global _lib
    if _lib is None:
        path = Path(os.environ.get("WAL2026_AMD_LIB", LIB_PATH))
        if not path.exists():
            raise RuntimeError(
                f"wal2026_amd: {path} is missing; build it with `python -m wal2026_amd.build` "
                "(the HIP library is required, there is no fallback path)")
        L = ctypes.CDLL(str(path))
        _declare(L)
        if L.wal_abi_version() != ABI_VERSION:
            raise RuntimeError(f"wal2026_amd: ABI {L.wal_abi_version()} != {ABI_VERSION}")
        _lib = L
    return _lib


_ops = None


def ops():
    """torch.ops.wal2026_amd: the PyTorch-ROCm operators over the C ABI
    (libwal2026_amd_torch.so, built beside the library; raises if missing)."""
    global _ops
    if _ops is None:
        lib()  # the operator library links it: load (and version-check) it first
        path = Path(os.environ.get("WAL2026_AMD_TORCH_LIB", TORCH_OPS_PATH))
        if not path.exists():
            raise RuntimeError(f"wal2026_amd: {path} is missing; build it with `python -m wal2026_amd.build` "
                               "(the HIP library is required, there is no fallback path)")
        torch.ops.load_library(str(path))
        _ops = torch.ops.wal2026_amd
    return _ops


def check(status: int) -> None:
    if status != OK:
        msg = lib().wal_last_error().decode(errors="replace")
        raise WalError(status, msg)


def float_tag(dtype: torch.dtype) -> int:
    try:
        return FLOAT_DTYPES[dtype]
    except KeyError:
        raise TypeError(f"unsupported floating dtype {dtype}") from None


def id_tag(dtype: torch.dtype) -> int:
    try:
        return ID_DTYPES[dtype]
    except KeyError:
        raise TypeError(f"unsupported index dtype {dtype}") from None


def require_rocm(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one ROCm device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "wal2026_amd: tensors must be on a ROCm GPU (got device "
                f"{t.device}); the HIP library is the only compute path")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"wal2026_amd: tensors on different devices ({dev} vs {t.device})")
    if dev is None:
        raise RuntimeError("wal2026_amd: no tensor given")
    if torch.version.hip is None:
        raise RuntimeError("wal2026_amd: this torch build is not a ROCm build")
    return dev


def id_range(*ids: torch.Tensor) -> tuple[int, int]:
    """(min, max) over index tensors of any id dtype, with one host sync.
    uint16 planes are widened through an int16 view (torch has no uint16
    reductions on ROCm devices)."""
    lo, hi = [], []
    for t in ids:
        if t.numel() == 0:
            continue
        w = (t.view(torch.int16).to(torch.int32) & 0xFFFF) if t.dtype == torch.uint16 else t
        lo.append(w.amin().to(torch.int64))
        hi.append(w.amax().to(torch.int64))
    if not lo:
        return 0, -1
    a, b = torch.stack([torch.stack(lo).min(), torch.stack(hi).max()]).tolist()
    return int(a), int(b)


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
