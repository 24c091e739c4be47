"""torch.ops.wal2026_amd.rvq_linear_out on the GPU: the module forward's op
writing into a caller's output tensor (the boundary's out= form for code that
keeps its buffers, such as a captured HIP graph).

* the same bits as rvq_linear for the decode kernel (M = 1), the split-K
  fused prefill kernel (M = 64) and the two-pass form (M = 1024), bf16 and
  fp32 outputs;
* shape, device and contiguity errors raise RuntimeError (TORCH_CHECK), the
  exception the reference's fused-kernel callers catch
  (src/runtime.py:1655-1661);
* under HIP graph capture (split-K's workspace and the two-pass weight come
  from the graph's memory pool): every replay, with eager work and a new x
  between replays, equals the eager result.
Reference: PackedGroupedBlockRVQLinear.forward, src/runtime.py:1362-1507.
"""
from __future__ import annotations

import pytest
import torch

from _cases import make_encoding
from wal2026_amd import PackedGroupedBlockRVQLinear, _lib

pytestmark = pytest.mark.gpu


@pytest.fixture
def mod(gpu_device, monkeypatch):
    for v in ("WAL2026_PREFILL_TILE", "WAL2026_PREFILL_KSPLIT", "WAL2026_PREFILL_TWO_PASS"):
        monkeypatch.delenv(v, raising=False)
    enc = make_encoding(1024, 4096, S=2, K=256, seed=61)
    b = (torch.randn(1024, generator=torch.Generator().manual_seed(2)) * 0.5).to(torch.bfloat16)
    return PackedGroupedBlockRVQLinear(enc, bias=b, matmul_strategy="hip_block_rvq").to(gpu_device)


def _x(m, device, seed):
    return torch.randn(m, 4096, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16).to(device)


def _ops(mod, x, out_dtype, out=None):
    c = mod._call_for(x, False)
    ops = _lib.ops()
    if out is None:
        return ops.rvq_linear(x, c[0], c[1], c[2], mod.bias, out_dtype)
    return ops.rvq_linear_out(x, c[0], c[1], c[2], mod.bias, out)


@pytest.mark.parametrize("m,form", [(1, "decode"), (64, "split"), (1024, "two_pass")])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_out_equals_the_allocating_op(m, form, out_dtype, mod, gpu_device, monkeypatch):
    if form == "two_pass":
        monkeypatch.setenv("WAL2026_PREFILL_TWO_PASS", "1")  # (this layer's cost model picks split-K here)
    x = _x(m, gpu_device, seed=m)
    info = mod.launch_info(x)
    if form == "split":
        assert info["k_splits"] > 1, info
    if form == "two_pass" and out_dtype == torch.bfloat16:
        assert info["two_pass"] is True, info
    ref = _ops(mod, x, out_dtype)
    out = torch.full((m, 1024), float("nan"), dtype=out_dtype, device=gpu_device)
    res = _ops(mod, x, out_dtype, out=out)
    assert res.data_ptr() == out.data_ptr()
    view = torch.int16 if out_dtype == torch.bfloat16 else torch.int32
    assert torch.equal(out.view(view), ref.view(view))


def test_out_argument_errors(mod, gpu_device):
    x = _x(4, gpu_device, seed=1)
    with pytest.raises(RuntimeError, match="shape"):
        _ops(mod, x, None, out=torch.empty(4, 1023, dtype=torch.bfloat16, device=gpu_device))
    with pytest.raises(RuntimeError, match="contiguous"):
        _ops(mod, x, None, out=torch.empty(1024, 4, dtype=torch.bfloat16, device=gpu_device).t())
    with pytest.raises(RuntimeError, match="device"):
        _ops(mod, x, None, out=torch.empty(4, 1024, dtype=torch.bfloat16))


@pytest.mark.parametrize("m", [1, 64, 1024])
def test_out_under_graph_capture(m, mod, gpu_device, monkeypatch):
    if m == 1024:
        monkeypatch.setenv("WAL2026_PREFILL_TWO_PASS", "1")  # the two passes under capture
    x = _x(m, gpu_device, seed=100 + m)
    out = torch.empty(m, 1024, dtype=torch.bfloat16, device=gpu_device)
    _ops(mod, x, None, out=out)  # descriptors and images built before capture
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _ops(mod, x, None, out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _ops(mod, x, None, out=out)
    for r in range(3):
        x.copy_(_x(m, gpu_device, seed=200 + r))  # eager work between the replays
        want = _ops(mod, x, None)
        torch.cuda.synchronize()
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), (m, r)
