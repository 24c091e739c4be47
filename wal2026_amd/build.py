"""Build libwal2026_amd.so (gfx950) in-tree with hipcc.

``python -m wal2026_amd.build`` compiles every ``csrc/*.hip`` file to an
object under ``wal2026_amd/_build/`` and links ``wal2026_amd/_lib/libwal2026_amd.so``.

Flags that matter for correctness:
* ``-ffp-contract=off``: the kernels reproduce the reference's separately
  rounded fp32 multiplies and adds; no multiply-add may be fused behind their
  back (fused multiply-adds are written explicitly where intended).
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: never emit packed fp32
  VALU instructions (v_pk_add_f32 / v_pk_mul_f32 / v_pk_fma_f32).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = PKG / "_build"
LIBDIR = PKG / "_lib"
LIB = LIBDIR / "libwal2026_amd.so"
ARCH = "gfx950"

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]

SOURCES = sorted(CSRC.glob("*.hip"))
TORCH_OPS_SRC = CSRC / "torch_ops.cpp"
TORCH_OPS_LIB = LIBDIR / "libwal2026_amd_torch.so"
HEADERS = sorted(CSRC.glob("*.h")) + sorted(INCLUDE.glob("*.h"))


def _quiet(stderr: str) -> str:
    # The host pass of hipcc does not know the gfx target feature; drop that notice.
    return "\n".join(l for l in stderr.splitlines() if "is not a recognized feature" not in l)


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{_quiet(r.stderr)}")
    msg = _quiet(r.stderr).strip()
    if msg:
        print(msg, file=sys.stderr)
    return obj


def device_asm(src: Path, out: Path) -> Path:
    """Write the gfx950 assembly of one source (for instruction audits)."""
    cmd = [HIPCC, *COMMON_FLAGS, "--cuda-device-only", "-S", str(src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc -S failed on {src.name}:\n{_quiet(r.stderr)}")
    return out


def _torch_ops_cmd(out: Path) -> list[str]:
    """g++ line of the PyTorch-ROCm operator library (host code only: it
    calls the C ABI, links libwal2026_amd.so beside it)."""
    import torch
    from torch.utils import cpp_extension as ce

    abi = int(torch.compiled_with_cxx11_abi())
    cmd = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-I{INCLUDE}"]
    cmd += [f"-I{p}" for p in ce.include_paths(device_type="cuda")]
    cmd += [str(TORCH_OPS_SRC), "-o", str(out), f"-L{LIBDIR}", "-lwal2026_amd", "-Wl,-rpath,$ORIGIN"]
    for p in ce.library_paths(device_type="cuda"):
        cmd += [f"-L{p}", f"-Wl,-rpath,{p}"]
    cmd += ["-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip", "-ltorch", "-lamdhip64"]
    return cmd


def build_torch_ops() -> Path:
    """Build libwal2026_amd_torch.so (needs libwal2026_amd.so)."""
    tmp = TORCH_OPS_LIB.with_suffix(".so.tmp")
    r = subprocess.run(_torch_ops_cmd(tmp), capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"torch op library failed to build:\n{r.stderr}")
    os.replace(tmp, TORCH_OPS_LIB)
    return TORCH_OPS_LIB


def build(jobs: int | None = None) -> Path:
    """Compile and link the library and its torch operator; always rebuilds."""
    BUILD.mkdir(parents=True, exist_ok=True)
    LIBDIR.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(len(SOURCES), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    build_torch_ops()
    return LIB


if __name__ == "__main__":
    print(build())
