"""GPU: horizontally fused linears (FusedBlockRVQLinears) against the same
linears run one by one.

A fused launch computes every output row with the same kernel and the same
per-row summation order as the linear's own launch, so the bar is bit
equality with the separate forwards (which test_gpu_parity checks against the
oracle), plus the 2e-3 output bar against the oracle directly."""
from __future__ import annotations

import pytest
import torch

from _cases import bits, make_encoding, module_buffers_as_encoding, oracle_weight, rel_err
from oracle import c_oracle
from wal2026_amd import FusedBlockRVQLinears, PackedGroupedBlockRVQLinear

pytestmark = pytest.mark.gpu
TOL = 2e-3

# (name, [(out_features, group_rows)], in_features, S, K, id dtype, extra encoding options)
FUSIONS = [
    ("qkv_s1_k4096_u16_scale128", [(512, None), (128, None), (128, None)], 256, 1, 4096, torch.uint16,
     {"scale_run": 128}),
    ("qkv_s2_u8", [(256, None), (64, None), (64, None)], 256, 2, 256, None, {}),
    ("gate_up_s3_groups", [(600, 256), (600, 256)], 384, 3, 256, None, {}),
    ("mixed_ragged_s1_per_row_scale", [(200, 96), (72, None)], 128, 1, 256, None, {}),
]


def _linears(spec, device, bias: bool):
    name, shapes, in_f, S, K, idt, opts = spec
    mods = []
    for i, (out_f, gr) in enumerate(shapes):
        enc = make_encoding(out_f, in_f, S=S, K=K, id_dtype=idt, group_rows=gr, seed=100 + 7 * i, **opts)
        b = torch.randn(out_f, generator=torch.Generator().manual_seed(i)) if (bias and i != 1) else None
        mods.append(PackedGroupedBlockRVQLinear(enc, b, matmul_strategy="hip_block_rvq").to(device))
    return mods


@pytest.mark.parametrize("spec", FUSIONS, ids=[f[0] for f in FUSIONS])
@pytest.mark.parametrize("m", [1, 4, 16, 40])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float16], ids=["xbf16", "xf16"])
def test_fused_equals_separate(spec, m, x_dtype, gpu_device, monkeypatch):
    # prefill rows (m = 40: 80 rows) on the fused kernel unsplit, whose per-row
    # arithmetic does not depend on the other linears of the launch
    monkeypatch.setenv("WAL2026_PREFILL_TWO_PASS", "0")
    monkeypatch.setenv("WAL2026_PREFILL_KSPLIT", "1")
    mods = _linears(spec, gpu_device, bias=(m == 4))
    fused = FusedBlockRVQLinears(mods)
    x = torch.randn(2, m, spec[2], generator=torch.Generator().manual_seed(m)).to(x_dtype).to(gpu_device)
    outs = fused(x)
    assert len(outs) == len(mods)
    for mod, y in zip(mods, outs):
        ref = mod(x)
        assert y.shape == ref.shape and y.dtype == ref.dtype
        assert torch.equal(bits(y), bits(ref)), f"{spec[0]} m={m}: fused output differs from the separate launch"


@pytest.mark.parametrize("spec", FUSIONS[:2], ids=[f[0] for f in FUSIONS[:2]])
def test_fused_fp32_parity_with_oracle(spec, gpu_device):
    mods = _linears(spec, gpu_device, bias=False)
    fused = FusedBlockRVQLinears(mods)
    x = torch.randn(3, spec[2], generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    outs = fused(x.to(gpu_device))
    for mod, y in zip(mods, outs):
        w_ref = oracle_weight(module_buffers_as_encoding(mod), torch.bfloat16)
        ref = c_oracle.linear_f64(x, w_ref)
        assert rel_err(y.float(), ref) <= 1e-2  # bf16 output: one rounding of y
        y32 = mod._hip_linear(x.to(gpu_device), fast=False, out_dtype=torch.float32)
        assert rel_err(y32, ref) <= TOL


def test_fused_refuses_mixed_strategies(gpu_device):
    enc = make_encoding(64, 128, S=2, seed=1)
    a = PackedGroupedBlockRVQLinear(enc, matmul_strategy="per_group").to(gpu_device)
    b = PackedGroupedBlockRVQLinear(enc, matmul_strategy="per_group_fast").to(gpu_device)
    with pytest.raises(ValueError):
        FusedBlockRVQLinears([a, b])
    c = PackedGroupedBlockRVQLinear(make_encoding(64, 256, S=2, seed=2)).to(gpu_device)
    with pytest.raises(ValueError):
        FusedBlockRVQLinears([a, c])
