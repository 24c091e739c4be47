"""The two-pass prefill form of the torch operator, on the GPU: for a
prefill call with an output in x's dtype that its cost model finds faster
than the fused kernel, the module forward writes the dense weight
(wal_rvq_reconstruct, bit-exact) and multiplies with torch's GEMM -- the
reference's own per_group order of work (src/runtime.py:1501-1507).

* when it is taken: launch_info reports it; the cost model's choices at the
  measured crossovers (gate_up's shape fused, with its k-steps split at
  small M, up to 512 rows and two-pass from 768); the switches that keep the
  fused prefill kernel (WAL2026_PREFILL_TWO_PASS=0, a forced tile shape, an
  fp32 output, decode rows) or force the two passes
  (WAL2026_PREFILL_TWO_PASS=1, which the parity tests below use) are
  honoured;
* parity: bf16 outputs against the oracle's bit-exact weight contracted in
  float64, max|dy|/max|y| <= 4e-3: the 2e-3 bar of fp32 accumulation plus the
  output's rounding to bf16 (half an ulp, 2^-9 of max|y|); with the
  reference's bf16 bias inside F.linear; FAST semantics at every stage cap;
* against the fused kernel: the same outputs up to one bf16 ulp per element
  (both accumulate in fp32, in different orders).
"""
from __future__ import annotations

import pytest
import torch

from _cases import make_encoding, module_buffers_as_encoding, oracle_weight, rel_err
from oracle import c_oracle
from wal2026_amd import PackedGroupedBlockRVQLinear

pytestmark = pytest.mark.gpu

BAR_BF16 = 4e-3


def _module(device, strategy="hip_block_rvq", bias=False, S=2, seed=3):
    enc = make_encoding(1024, 2048, S=S, K=256, group_rows=512, seed=seed)
    b = (torch.randn(1024, generator=torch.Generator().manual_seed(seed)) * 0.5).to(torch.bfloat16) if bias else None
    return PackedGroupedBlockRVQLinear(enc, bias=b, matmul_strategy=strategy).to(device), b


def _x(m, device, seed=0):
    return torch.randn(m, 2048, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16).to(device)


@pytest.fixture
def no_overrides(monkeypatch):
    for v in ("WAL2026_PREFILL_TWO_PASS", "WAL2026_PREFILL_TILE", "WAL2026_PREFILL_KSPLIT"):
        monkeypatch.delenv(v, raising=False)
    return monkeypatch


def test_when_the_two_pass_form_is_taken(gpu_device, no_overrides):
    mod, _ = _module(gpu_device)
    assert mod.launch_info(_x(2048, gpu_device))["two_pass"] is True
    assert "two_pass" not in mod.launch_info(_x(16, gpu_device))  # the decode kernel
    no_overrides.setenv("WAL2026_PREFILL_TWO_PASS", "1")
    assert mod.launch_info(_x(17, gpu_device))["two_pass"] is True
    assert "two_pass" not in mod.launch_info(_x(16, gpu_device))
    no_overrides.setenv("WAL2026_PREFILL_TWO_PASS", "0")
    assert mod.launch_info(_x(2048, gpu_device))["two_pass"] is False
    no_overrides.delenv("WAL2026_PREFILL_TWO_PASS")
    no_overrides.setenv("WAL2026_PREFILL_TILE", "tall")
    assert mod.launch_info(_x(2048, gpu_device))["two_pass"] is False


def test_cost_model_at_the_gate_up_shape(gpu_device, no_overrides):
    """c4's fused gate_up shape (28672 x 4096): the fused kernel reads 29 MB of
    indices where the two passes write and read 235 MB of weight, so it is
    chosen up to 512 rows (measured 95-149 us against 131-175), the two
    passes from 768 (232 against 272 us)."""
    from wal2026_amd import synth

    cfg = synth.CONFIGS["c4"]
    enc = synth.make_encoding(28672, 4096, cfg, synth.generator(0, gpu_device), gpu_device)
    mod = PackedGroupedBlockRVQLinear(enc, matmul_strategy="hip_block_rvq").to(gpu_device)
    xb = lambda m: torch.zeros(m, 4096, dtype=torch.bfloat16, device=gpu_device)
    for m, splits in ((64, 2), (256, 1), (512, 1)):
        info = mod.launch_info(xb(m))
        assert info["two_pass"] is False and info["k_splits"] == splits, (m, info)
    for m in (768, 2048):
        assert mod.launch_info(xb(m))["two_pass"] is True, m
    no_overrides.setenv("WAL2026_PREFILL_TWO_PASS", "1")
    assert mod.launch_info(xb(256))["two_pass"] is True


@pytest.mark.parametrize("m", [17, 100, 512, 700])
@pytest.mark.parametrize("bias", [False, True], ids=["nobias", "bias"])
def test_two_pass_parity(m, bias, gpu_device, no_overrides):
    no_overrides.setenv("WAL2026_PREFILL_TWO_PASS", "1")
    mod, b = _module(gpu_device, bias=bias)
    x = _x(m, gpu_device, seed=m)
    assert mod.launch_info(x)["two_pass"] is True
    y = mod(x)
    assert y.dtype == torch.bfloat16 and y.shape == (m, 1024)
    w = oracle_weight(module_buffers_as_encoding(mod), torch.bfloat16)
    ref = c_oracle.linear_f64(x.cpu(), w)
    if b is not None:
        ref = ref + b.double()  # F.linear's bias: added to the accumulator before the rounding
    assert rel_err(y, ref) <= BAR_BF16


@pytest.mark.parametrize("k", [1, 2])
def test_two_pass_fast_semantics(k, gpu_device, no_overrides):
    no_overrides.setenv("WAL2026_PREFILL_TWO_PASS", "1")
    mod, _ = _module(gpu_device, strategy="per_group_fast", S=2, seed=5)
    for g in mod.groups:
        g.set_effective_stages_per_split(k)
    x = _x(640, gpu_device, seed=k)
    assert mod.launch_info(x)["two_pass"] is True
    w = oracle_weight(module_buffers_as_encoding(mod), torch.bfloat16, active=list(range(k)))
    assert rel_err(mod(x), c_oracle.linear_f64(x.cpu(), w)) <= BAR_BF16


@pytest.mark.parametrize("layout", ["f16_x", "groups_u16"])
def test_two_pass_other_layouts(layout, gpu_device, no_overrides):
    """fp16 activations (the weight written in fp16, torch's fp16 GEMM); and
    three row groups with 16-bit ids (K = 1024) and a row scale shared by
    128-row runs."""
    no_overrides.setenv("WAL2026_PREFILL_TWO_PASS", "1")
    if layout == "f16_x":
        enc = make_encoding(1024, 2048, S=2, K=256, group_rows=512, seed=21)
        dt = torch.float16
    else:
        enc = make_encoding(1536, 2048, S=1, K=1024, group_rows=512, scale_run=128, seed=22)
        dt = torch.bfloat16
    mod = PackedGroupedBlockRVQLinear(enc, matmul_strategy="hip_block_rvq").to(gpu_device)
    x = torch.randn(600, 2048, generator=torch.Generator().manual_seed(23)).to(dt).to(gpu_device)
    assert mod.launch_info(x)["two_pass"] is True
    y = mod(x)
    assert y.dtype == dt and y.shape == (600, enc.original_shape[0])
    w = oracle_weight(module_buffers_as_encoding(mod), dt)
    # fp16 output: rounding to fp16 is finer than bf16's, so the bf16 bar bounds it too
    assert rel_err(y, c_oracle.linear_f64(x.cpu(), w)) <= BAR_BF16


def test_two_pass_against_the_fused_kernel(gpu_device, no_overrides):
    mod, _ = _module(gpu_device, bias=True)
    x = _x(1024, gpu_device, seed=11)
    no_overrides.setenv("WAL2026_PREFILL_TWO_PASS", "1")
    assert mod.launch_info(x)["two_pass"] is True
    y2 = mod(x).float().cpu()
    no_overrides.setenv("WAL2026_PREFILL_TWO_PASS", "0")
    # the fused kernel unsplit (a split adds its slices' partial sums in
    # another fp32 order, which near-cancelling outputs show beyond one ulp)
    no_overrides.setenv("WAL2026_PREFILL_KSPLIT", "1")
    assert mod.launch_info(x)["two_pass"] is False
    y1 = mod(x).float().cpu()
    # one bf16 ulp of the larger magnitude bounds every difference
    ulp = torch.maximum(y1.abs(), y2.abs()).clamp_min(1e-30) * 2.0 ** -7
    assert bool(((y1 - y2).abs() <= ulp).all())
    # split 8 ways: one ulp plus 1e-4 of max|y| for the summation order
    no_overrides.setenv("WAL2026_PREFILL_KSPLIT", "8")
    assert mod.launch_info(x)["k_splits"] == 8
    y3 = mod(x).float().cpu()
    bound = torch.maximum(y3.abs(), y2.abs()) * 2.0 ** -7 + 1e-4 * float(y2.abs().max())
    assert bool(((y3 - y2).abs() <= bound).all())


def test_fp32_output_keeps_the_fused_kernel(gpu_device, no_overrides):
    """An fp32 output (the parity tests' form) goes to the fused kernel: the
    two-pass GEMM would round to bf16 first."""
    from wal2026_amd import _lib

    mod, _ = _module(gpu_device)
    x = _x(1024, gpu_device, seed=2)
    c = mod._call_for(x, False)
    y = _lib.ops().rvq_linear(x, c[0], c[1], c[2], None, torch.float32)
    assert y.dtype == torch.float32
    w = oracle_weight(module_buffers_as_encoding(mod), torch.bfloat16)
    assert rel_err(y, c_oracle.linear_f64(x.cpu(), w)) <= 2e-3
