"""wal_rvq_linear_noalloc on the GPU: the entry point that allocates nothing
keeps the split-K partials in the library's per-device scratch array and
returns what wal_rvq_linear_ws returns with a caller workspace, bit for bit
(the same kernels and the same split), on consecutive calls that reuse the
array (the second with fewer rows), and refuses a call whose partials exceed
the array.  Reference: PackedGroupedBlockRVQLinear.forward,
src/runtime.py:1362-1507 (the entry point itself has no counterpart there).
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from _cases import make_encoding, module_buffers_as_encoding, oracle_weight, rel_err
from oracle import c_oracle
from wal2026_amd import PackedGroupedBlockRVQLinear, _lib

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20


@pytest.fixture
def clean_env(monkeypatch):
    for v in ("WAL2026_PREFILL_TILE", "WAL2026_PREFILL_KSPLIT", "WAL2026_PREFILL_TWO_PASS"):
        monkeypatch.delenv(v, raising=False)
    return monkeypatch


def _module(out_f, in_f, device, seed=41, bias=True):
    enc = make_encoding(out_f, in_f, S=2, K=256, seed=seed)
    b = (torch.randn(out_f, generator=torch.Generator().manual_seed(seed)) * 0.5).to(torch.bfloat16) if bias else None
    return PackedGroupedBlockRVQLinear(enc, bias=b, matmul_strategy="hip_block_rvq").to(device)


def _args(mod, x, y):
    addr, sem, mask, _epoch, layer = mod._call_for(x, False)
    b = mod.bias
    return (layer, sem, mask, x.data_ptr(), x.shape[0], _lib.float_tag(x.dtype),
            b.data_ptr() if b is not None else None, _lib.float_tag(b.dtype) if b is not None else _lib.F32,
            y.data_ptr(), _lib.float_tag(y.dtype))


def _noalloc(mod, x, out_dtype):
    y = torch.empty(x.shape[0], mod.out_features, dtype=out_dtype, device=x.device)
    layer, *rest = _args(mod, x, y)
    rc = _lib.lib().wal_rvq_linear_noalloc(ctypes.byref(layer), *rest, _lib.stream_ptr(x.device))
    return rc, y


def _ws(mod, x, out_dtype):
    y = torch.empty(x.shape[0], mod.out_features, dtype=out_dtype, device=x.device)
    layer, sem, mask, xp, m, xt, bp, bt, yp, yt = _args(mod, x, y)
    n = ctypes.c_size_t(0)
    _lib.check(_lib.lib().wal_rvq_linear_workspace_size(ctypes.byref(layer), sem, xp, m, xt, ctypes.byref(n)))
    ws = torch.empty(max(n.value, 16), dtype=torch.uint8, device=x.device)
    _lib.check(_lib.lib().wal_rvq_linear_ws(ctypes.byref(layer), sem, mask, xp, m, xt, bp, bt, yp, yt,
                                            ws.data_ptr(), n.value, _lib.stream_ptr(x.device)))
    return y, n.value


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_noalloc_matches_the_workspace_call(out_dtype, gpu_device, clean_env):
    mod = _module(1024, 4096, gpu_device)
    w = oracle_weight(module_buffers_as_encoding(mod), torch.bfloat16)
    for m, seed in ((96, 1), (40, 2)):  # the second call reuses the array with fewer rows
        x = torch.randn(m, 4096, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16).to(gpu_device)
        info = mod.launch_info(x)
        assert info["kernel"] == "prefill" and info["k_splits"] > 1, info
        rc, y = _noalloc(mod, x, out_dtype)
        assert rc == _lib.OK, _lib.lib().wal_last_error()
        ref, need = _ws(mod, x, out_dtype)
        assert 0 < need <= SCRATCH_BYTES
        assert torch.equal(y.view(torch.int32 if out_dtype == torch.float32 else torch.int16),
                           ref.view(torch.int32 if out_dtype == torch.float32 else torch.int16)), m
        bar = 2e-3 if out_dtype == torch.float32 else 4e-3
        assert rel_err(y, c_oracle.linear_f64(x.cpu(), w) + mod.bias.double().cpu()) <= bar


def test_noalloc_without_a_split_and_over_the_limit(gpu_device, clean_env):
    mod = _module(1024, 4096, gpu_device, bias=False)
    # decode rows: no partials, the plain launch
    x = torch.randn(4, 4096, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(gpu_device)
    rc, y = _noalloc(mod, x, torch.float32)
    assert rc == _lib.OK
    ref, need = _ws(mod, x, torch.float32)
    assert need == 0 and torch.equal(y.view(torch.int32), ref.view(torch.int32))
    # 16 slices of 128 rows x 16384 outputs: 128 MiB of partials, refused before any launch
    big = _module(16384, 4096, gpu_device, bias=False)
    clean_env.setenv("WAL2026_PREFILL_KSPLIT", "16")
    xb = torch.zeros(128, 4096, dtype=torch.bfloat16, device=gpu_device)
    assert big.launch_info(xb)["k_splits"] == 16
    rc, _y = _noalloc(big, xb, torch.float32)
    assert rc == _lib.ESIZE and b"scratch" in _lib.lib().wal_last_error()
