"""Split-K of the 128 x 256 prefill tile on the GPU (wal_rvq_linear_ws): when
a layer's output tiles alone would leave CUs idle, each tile's k-steps are
shared by several workgroups that write fp32 partial sums to the caller's
workspace, and a second launch adds them in slice order.

* parity against the oracle's bit-exact weight contracted in float64
  (max|dy|/max|y| <= 2e-3 for fp32 outputs, 4e-3 for bf16 outputs, which add
  the output's rounding), for the planner's split and a forced one whose
  slices hold unequal numbers of 8-step units (a ragged last unit);
* exactness: one-hot activation rows read the dense weight out bit for bit
  (one nonzero product, every other partial +0);
* determinism (two calls agree bit for bit) and agreement with the unsplit
  launch to fp32 rounding;
* the module forward (torch operator) passes a workspace from torch's
  caching allocator.
Reference: PackedGroupedBlockRVQLinear.forward, src/runtime.py:1362-1507.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from _cases import make_encoding, module_buffers_as_encoding, oracle_weight, rel_err
from oracle import c_oracle
from wal2026_amd import PackedGroupedBlockRVQLinear, _lib

pytestmark = pytest.mark.gpu

LAYOUTS = {
    # name: (out, in, S, K, encoding options, m, forced slices or None, expected slices)
    "s2_u8_m64": (1024, 4096, 2, 256, {}, 64, None, 16),
    "s1_u16_groups_scale128_m40": (768, 2048, 1, 1024, {"group_rows": 256, "scale_run": 128}, 40, None, 8),
    "ragged_units_forced4": (512, 2176, 2, 256, {}, 100, 4, 4),
    "s3_groups_m128": (512, 3584, 3, 256, {"group_rows": 256}, 128, None, 14),
}


@pytest.fixture
def clean_env(monkeypatch):
    for v in ("WAL2026_PREFILL_TILE", "WAL2026_PREFILL_KSPLIT", "WAL2026_PREFILL_TWO_PASS"):
        monkeypatch.delenv(v, raising=False)
    return monkeypatch


def _module(name, device, bias=False, strategy="hip_block_rvq"):
    out_f, in_f, S, K, opts, m, _force, _want = LAYOUTS[name]
    enc = make_encoding(out_f, in_f, S=S, K=K, seed=31, **opts)
    b = (torch.randn(out_f, generator=torch.Generator().manual_seed(5)) * 0.5).to(torch.bfloat16) if bias else None
    return PackedGroupedBlockRVQLinear(enc, bias=b, matmul_strategy=strategy).to(device), b


def _call(mod, x, out_dtype, split=True, fast=False):
    """One call through the C ABI: wal_rvq_linear_ws with the workspace it
    asks for (split=True), or wal_rvq_linear."""
    addr, sem, mask, _epoch, layer = mod._call_for(x, fast)
    lib = _lib.lib()
    m = x.shape[0]
    y = torch.empty(m, mod.out_features, dtype=out_dtype, device=x.device)
    b = mod.bias
    bp, bt = (b.data_ptr(), _lib.float_tag(b.dtype)) if b is not None else (None, _lib.F32)
    st = _lib.stream_ptr(x.device)
    if split:
        n = ctypes.c_size_t(0)
        _lib.check(lib.wal_rvq_linear_workspace_size(ctypes.byref(layer), sem, x.data_ptr(), m,
                                                     _lib.float_tag(x.dtype), ctypes.byref(n)))
        ws = torch.empty(max(n.value, 16), dtype=torch.uint8, device=x.device)
        _lib.check(lib.wal_rvq_linear_ws(ctypes.byref(layer), sem, mask, x.data_ptr(), m, _lib.float_tag(x.dtype),
                                         bp, bt, y.data_ptr(), _lib.float_tag(out_dtype), ws.data_ptr(), n.value, st))
    else:
        _lib.check(lib.wal_rvq_linear(ctypes.byref(layer), sem, mask, x.data_ptr(), m, _lib.float_tag(x.dtype),
                                      bp, bt, y.data_ptr(), _lib.float_tag(out_dtype), st))
    return y


def _x(m, in_f, device, seed=0):
    return torch.randn(m, in_f, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16).to(device)


@pytest.mark.parametrize("name", list(LAYOUTS))
def test_split_k_parity(name, gpu_device, clean_env):
    out_f, in_f, _S, _K, _o, m, force, want = LAYOUTS[name]
    if force:
        clean_env.setenv("WAL2026_PREFILL_KSPLIT", str(force))
    mod, _ = _module(name, gpu_device)
    x = _x(m, in_f, gpu_device, seed=m)
    info = mod.launch_info(x)
    assert info["kernel"] == "prefill" and info["tile_shape"] == "short" and info["k_splits"] == want, info
    y = _call(mod, x, torch.float32)
    w = oracle_weight(module_buffers_as_encoding(mod), torch.bfloat16)
    ref = c_oracle.linear_f64(x.cpu(), w)
    assert rel_err(y, ref) <= 2e-3
    # the unsplit launch: the same products, another fp32 summation order
    y1 = _call(mod, x, torch.float32, split=False)
    assert rel_err(y, y1) <= 1e-5
    # deterministic: the slices are added in a fixed order
    assert torch.equal(_call(mod, x, torch.float32).view(torch.int32), y.view(torch.int32))


def test_split_k_one_hot_readout(gpu_device, clean_env):
    """Row i of x is the unit vector at column c_i: y[i, n] = W[n, c_i]
    exactly, through 16 slices (15 of them add +0)."""
    mod, _ = _module("s2_u8_m64", gpu_device)
    cols = [0, 7, 8, 255, 256, 1023, 1024, 2047, 2048, 3071, 3072, 4095, 13, 500, 2600, 3999]
    x = torch.zeros(64, 4096, dtype=torch.bfloat16)
    for i, c in enumerate(cols * 4):
        x[i, c] = 1.0
    x = x.to(gpu_device)
    assert mod.launch_info(x)["k_splits"] == 16
    y = _call(mod, x, torch.float32).cpu()
    w = oracle_weight(module_buffers_as_encoding(mod), torch.bfloat16).float()
    for i, c in enumerate(cols * 4):
        assert torch.equal(y[i], w[:, c]), (i, c)


def test_split_k_bias_bf16_output_and_fast(gpu_device, clean_env):
    mod, b = _module("s2_u8_m64", gpu_device, bias=True)
    x = _x(64, 4096, gpu_device, seed=3)
    y = _call(mod, x, torch.bfloat16)
    w = oracle_weight(module_buffers_as_encoding(mod), torch.bfloat16)
    ref = c_oracle.linear_f64(x.cpu(), w) + b.double()
    assert rel_err(y, ref) <= 4e-3
    # FAST semantics with one active stage
    fmod, _ = _module("s2_u8_m64", gpu_device, strategy="per_group_fast")
    for g in fmod.groups:
        g.set_effective_stages_per_split(1)
    yf = _call(fmod, x, torch.float32, fast=True)
    wf = oracle_weight(module_buffers_as_encoding(fmod), torch.bfloat16, active=[0])
    assert rel_err(yf, c_oracle.linear_f64(x.cpu(), wf)) <= 2e-3


def test_module_forward_passes_a_workspace(gpu_device, clean_env):
    """The torch operator asks for the workspace and allocates it from torch's
    caching allocator; with the fused kernel kept (WAL2026_PREFILL_TWO_PASS=0)
    the module forward runs the split launch."""
    clean_env.setenv("WAL2026_PREFILL_TWO_PASS", "0")
    mod, _ = _module("s2_u8_m64", gpu_device)
    x = _x(64, 4096, gpu_device, seed=9)
    info = mod.launch_info(x)
    assert info["two_pass"] is False and info["k_splits"] == 16
    y = mod(x)
    assert y.dtype == torch.bfloat16
    w = oracle_weight(module_buffers_as_encoding(mod), torch.bfloat16)
    assert rel_err(y, c_oracle.linear_f64(x.cpu(), w)) <= 4e-3
    # the same bits as the C ABI's split launch
    assert torch.equal(y.view(torch.int16), _call(mod, x, torch.bfloat16).view(torch.int16))


def test_split_k_fp16_activations(gpu_device, clean_env):
    """fp16 x (the weight rounded to fp16, fp16 MFMAs) through 16 slices."""
    mod, _ = _module("s2_u8_m64", gpu_device)
    x = torch.randn(64, 4096, generator=torch.Generator().manual_seed(12)).to(torch.float16).to(gpu_device)
    assert mod.launch_info(x)["k_splits"] == 16
    y = _call(mod, x, torch.float32)
    w = oracle_weight(module_buffers_as_encoding(mod), torch.float16)
    assert rel_err(y, c_oracle.linear_f64(x.cpu(), w)) <= 2e-3
    assert rel_err(y, _call(mod, x, torch.float32, split=False)) <= 1e-5
