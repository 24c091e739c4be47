"""GPU parity: the HIP library against the CPU oracle on the same seeded inputs.

Bar (written in each test):
* dequantised weights: bit-exact with the reference's reconstruct_weight /
  reconstruct_weight_fast (compared as integer bit patterns; NaN is compared
  by NaN-ness because torch's own scalar and vector casts disagree on NaN
  payloads);
* weights seen inside the fused decode / prefill kernels: bit-exact, read out
  through one-hot activations (x = e_k makes y[:, n] = W[n, k] exactly);
* layer outputs in fp32: max|dy| / max|y| <= 2e-3 against float64
  x @ W_ref^T (the observed error is fp32 accumulation order, ~1e-6).
"""
from __future__ import annotations

import zlib

import pytest
import torch

from _cases import bits, make_encoding, module_buffers_as_encoding, oracle_group, oracle_weight, rel_err
from oracle import c_oracle
from wal2026_amd import PackedGroupedBlockRVQLinear

pytestmark = pytest.mark.gpu
TOL = 2e-3

# (name, out, in, d, S, K, id dtype, group_rows, options)
LAYOUTS = [
    ("c1like_s2_u8", 256, 512, 8, 2, 256, None, None, {}),
    ("s1_k4096_i16", 160, 256, 8, 1, 4096, None, None, {}),
    ("s1_k4096_u16", 64, 128, 8, 1, 4096, torch.uint16, None, {}),
    # one stage with row scales shared by aligned runs of rows: the decode
    # kernel stages the codebook already multiplied by the scale
    ("s1_k4096_u16_scale128", 384, 256, 8, 1, 4096, torch.uint16, None, {"scale_run": 128}),
    ("s1_k256_scale16_ragged_groups", 200, 384, 8, 1, 256, None, 96, {"scale_run": 16}),
    ("s3_groups256_ragged", 600, 384, 8, 3, 256, None, 256, {}),
    # four and five row groups in one launch
    ("s1_k4096_groups4_scale32", 256, 256, 8, 1, 4096, torch.uint16, 64, {"scale_run": 32}),
    ("s2_groups5_ragged", 280, 256, 8, 2, 256, None, 64, {}),
    ("s4_u8", 96, 256, 8, 4, 256, None, None, {}),
    ("s2_stage_scales", 128, 256, 8, 2, 256, None, None, {"stage_scales": True}),
    ("s2_bf16_codebooks", 128, 256, 8, 2, 256, None, None, {"cb_dtype": torch.bfloat16}),
    ("s2_special_values", 192, 256, 8, 2, 256, None, 64, {"special": True}),
    ("d32_generic", 100, 320, 32, 2, 256, None, None, {}),
    ("d4_padded_generic", 70, 99, 4, 2, 64, None, 32, {}),
    ("s2_block_scale", 96, 128, 8, 2, 256, None, None, {"block_scale": True}),
    ("s5_generic", 48, 128, 8, 5, 16, None, None, {}),
    ("i32_ids_generic", 40, 64, 8, 1, 40000, torch.int32, None, {}),
    ("d8_B24_generic", 64, 192, 8, 2, 256, None, None, {}),
]


def _module(layout, device, **kw):
    name, out_f, in_f, d, S, K, idt, gr, opts = layout
    enc = make_encoding(out_f, in_f, d=d, S=S, K=K, id_dtype=idt, group_rows=gr, seed=zlib.crc32(name.encode()) % 1000, **opts)
    return PackedGroupedBlockRVQLinear(enc, **kw).to(device)


@pytest.mark.parametrize("layout", LAYOUTS, ids=[l[0] for l in LAYOUTS])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "f16", "f32"])
def test_reconstruct_bitexact(layout, out_dtype, gpu_device):
    mod = _module(layout, gpu_device)
    w = mod.reconstruct_weight(out_dtype=out_dtype)
    ref = oracle_weight(module_buffers_as_encoding(mod), out_dtype)
    wc = w.cpu()
    nan_w, nan_r = torch.isnan(wc.float()), torch.isnan(ref.float())
    assert torch.equal(nan_w, nan_r)
    assert torch.equal(bits(wc)[~nan_w], bits(ref)[~nan_r]), f"{layout[0]}: dequantised weights differ"


@pytest.mark.parametrize("layout", [l for l in LAYOUTS if l[4] >= 2], ids=[l[0] for l in LAYOUTS if l[4] >= 2])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "f16", "f32"])
def test_reconstruct_fast_bitexact(layout, out_dtype, gpu_device):
    mod = _module(layout, gpu_device)
    S = layout[4]
    for k in range(1, S + 1):
        for g in mod.groups:
            g.set_effective_stages_per_split(k)
        w = mod.reconstruct_weight_fast(out_dtype=out_dtype).cpu()
        if mod.groups[0].supports_fast_reconstruct():
            ref = oracle_weight(module_buffers_as_encoding(mod), out_dtype, active=list(range(k)))
        else:
            ref = oracle_weight(module_buffers_as_encoding(mod), out_dtype)
        assert torch.equal(bits(w), bits(ref)), f"{layout[0]} k={k}"


@pytest.mark.parametrize("layout", LAYOUTS, ids=[l[0] for l in LAYOUTS])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float16], ids=["xbf16", "xf16"])
@pytest.mark.parametrize("m", [1, 4, 16, 37, 200])
def test_linear_fp32_parity(layout, x_dtype, m, gpu_device):
    mod = _module(layout, gpu_device)
    g = torch.Generator().manual_seed(m)
    x = torch.randn(m, mod.in_features, generator=g).to(x_dtype)
    y = mod._hip_linear(x.to(gpu_device), fast=False, out_dtype=torch.float32)
    w_ref = oracle_weight(module_buffers_as_encoding(mod), x_dtype)
    ref = c_oracle.linear_f64(x, w_ref)
    err = rel_err(y, ref)
    assert err <= TOL, f"{layout[0]} m={m}: max|dy|/max|y| = {err:.3e} > {TOL}"
    assert err <= 1e-5, f"{layout[0]} m={m}: {err:.3e} is above fp32 accumulation error"


# The prefill launcher picks its tile shape from the grid size;
# WAL2026_PREFILL_TILE forces one: short = 128 x-rows x 256 weight rows,
# tall = 256 x 256 (S <= 2, 16-bit tables), wide = 256 x 128.
TILES = ["short", "tall", "wide"]


@pytest.mark.parametrize("layout", LAYOUTS, ids=[l[0] for l in LAYOUTS])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float16], ids=["xbf16", "xf16"])
@pytest.mark.parametrize("m", [17, 300])
@pytest.mark.parametrize("tile", TILES)
def test_prefill_tile_shapes_parity(layout, x_dtype, m, tile, gpu_device, monkeypatch):
    monkeypatch.setenv("WAL2026_PREFILL_TILE", tile)
    mod = _module(layout, gpu_device)
    g = torch.Generator().manual_seed(m + 7)
    x = torch.randn(m, mod.in_features, generator=g).to(x_dtype)
    y = mod._hip_linear(x.to(gpu_device), fast=False, out_dtype=torch.float32)
    w_ref = oracle_weight(module_buffers_as_encoding(mod), x_dtype)
    err = rel_err(y, c_oracle.linear_f64(x, w_ref))
    assert err <= 1e-5, f"{layout[0]} m={m} {tile}: max|dy|/max|y| = {err:.3e}"


@pytest.mark.parametrize("layout", LAYOUTS[:11], ids=[l[0] for l in LAYOUTS[:11]])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float16], ids=["xbf16", "xf16"])
@pytest.mark.parametrize("tile", TILES)
def test_onehot_prefill_tiles_bitexact(layout, x_dtype, tile, gpu_device, monkeypatch):
    """x = I (M = in_features > 16: prefill kernel) gives y = W^T exactly."""
    monkeypatch.setenv("WAL2026_PREFILL_TILE", tile)
    mod = _module(layout, gpu_device)
    eye = torch.eye(mod.in_features, dtype=x_dtype, device=gpu_device)
    y = mod._hip_linear(eye, fast=False, out_dtype=torch.float32).cpu()
    ref = oracle_weight(module_buffers_as_encoding(mod), x_dtype).float()
    assert torch.equal(bits(y.t().contiguous()), bits(ref)) or torch.equal(y.t(), ref), layout[0]


@pytest.mark.parametrize("layout", LAYOUTS[:9], ids=[l[0] for l in LAYOUTS[:9]])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float16], ids=["xbf16", "xf16"])
def test_onehot_decode_tiles_bitexact(layout, x_dtype, gpu_device):
    """16 one-hot rows per call (decode kernel) read out 16 weight columns."""
    mod = _module(layout, gpu_device)
    ref = oracle_weight(module_buffers_as_encoding(mod), x_dtype).float()
    k_in = mod.in_features
    for c0 in range(0, k_in, 16):
        cols = list(range(c0, min(c0 + 16, k_in)))
        x = torch.zeros(len(cols), k_in, dtype=x_dtype)
        for i, c in enumerate(cols):
            x[i, c] = 1.0
        y = mod._hip_linear(x.to(gpu_device), fast=False, out_dtype=torch.float32).cpu()
        got = y.t()
        want = ref[:, cols]
        assert torch.equal(got, want), f"{layout[0]} columns {c0}..{cols[-1]}"


@pytest.mark.parametrize("layout", [l for l in LAYOUTS if l[4] >= 2][:6], ids=[l[0] for l in LAYOUTS if l[4] >= 2][:6])
@pytest.mark.parametrize("m", [1, 16, 64])
def test_fast_strategy_parity(layout, m, gpu_device):
    mod = _module(layout, gpu_device, matmul_strategy="per_group_fast")
    for g in mod.groups:
        g.set_effective_stages_per_split(1)
    x = torch.randn(m, mod.in_features, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    y = mod._hip_linear(x.to(gpu_device), fast=True, out_dtype=torch.float32)
    if mod.groups[0].supports_fast_reconstruct():
        w_ref = oracle_weight(module_buffers_as_encoding(mod), torch.bfloat16, active=[0])
    else:
        w_ref = oracle_weight(module_buffers_as_encoding(mod), torch.bfloat16)
    assert rel_err(y, c_oracle.linear_f64(x, w_ref)) <= TOL


STAGEWISE_LAYOUTS = [l for l in LAYOUTS if l[0] in {
    "c1like_s2_u8", "s1_k4096_i16", "s1_k256_scale16_ragged_groups", "s3_groups256_ragged", "s4_u8",
    "s2_stage_scales", "s2_bf16_codebooks", "d32_generic", "d4_padded_generic", "s5_generic"}]


def _ulp_dist(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    def key(t):
        v = bits(t).to(torch.int32) & 0xFFFF
        return torch.where(v >= 0x8000, 0x8000 - v, v)
    return (key(a) - key(b)).abs()


@pytest.mark.parametrize("layout", STAGEWISE_LAYOUTS, ids=[l[0] for l in STAGEWISE_LAYOUTS])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float16], ids=["xbf16", "xf16"])
@pytest.mark.parametrize("m", [1, 33])
def test_stagewise_strategy_parity(layout, x_dtype, m, gpu_device):
    """stagewise_einsum (src/runtime.py:878-894, :1466-1475) against the
    oracle.  The reference rounds every stage's contraction, every partial
    sum and the bias add to x dtype, so two correct fp32-accumulating
    implementations agree bit for bit except where accumulation order flips
    one of those roundings: one x-dtype ulp of an intermediate, which
    cancellation in the later adds can make a few ulps of a small output.
    Bar: at least 98 % of outputs bit-equal, and max|dy| / max|y| within two
    ulps of the largest output (2^-7 for bf16, 2^-9 for fp16)."""
    mod = _module(layout, gpu_device, matmul_strategy="stagewise_einsum")
    g = torch.Generator().manual_seed(7)
    mod.bias = (torch.randn(mod.out_features, generator=g) * 0.1).to(torch.bfloat16).to(gpu_device)
    x = torch.randn(m, mod.in_features, generator=g).to(x_dtype)
    y = mod(x.to(gpu_device)).cpu()
    assert y.dtype == x_dtype
    enc = module_buffers_as_encoding(mod)
    ref = torch.cat([c_oracle.stagewise_linear(oracle_group(ge), x) for ge in enc.groups], dim=1)
    ref = (ref.float() + mod.bias.cpu().to(x_dtype).float()).to(x_dtype)
    d = _ulp_dist(y, ref)
    assert float((d == 0).double().mean()) >= 0.98, layout[0]
    assert rel_err(y, ref) <= (2.0 ** -7 if x_dtype == torch.bfloat16 else 2.0 ** -9), layout[0]


SCALED_LAYOUTS = [l for l in LAYOUTS if l[8].get("scale_run")]


@pytest.mark.parametrize("layout", SCALED_LAYOUTS, ids=[l[0] for l in SCALED_LAYOUTS])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float16], ids=["xbf16", "xf16"])
def test_scale_runs_detected_and_fast_parity(layout, x_dtype, gpu_device):
    """Shared row scales are passed to the library as a compact buffer
    (scale_rows > 1); reconstruct_weight_fast semantics (S = 1) on that path."""
    mod = _module(layout, gpu_device, matmul_strategy="per_group_fast")
    assert mod._descriptor().layer.scale_rows >= 16
    x = torch.randn(3, mod.in_features, generator=torch.Generator().manual_seed(4)).to(x_dtype)
    y = mod._hip_linear(x.to(gpu_device), fast=True, out_dtype=torch.float32)
    w_ref = oracle_weight(module_buffers_as_encoding(mod), x_dtype, active=[0])
    assert rel_err(y, c_oracle.linear_f64(x, w_ref)) <= 1e-5
    # the decode kernel's weights, read out through one-hot rows, are exact
    eye = torch.eye(16, mod.in_features, dtype=x_dtype)
    got = mod._hip_linear(eye.to(gpu_device), fast=True, out_dtype=torch.float32).cpu().t()
    assert torch.equal(got, w_ref[:, :16].float())


@pytest.mark.parametrize("m", [1, 5, 40])
def test_forward_bias_and_output_dtype(m, gpu_device):
    """forward(x) in x dtype with the bf16 bias buffer cast to x dtype
    (src/runtime.py:1229-1230, :1503-1505)."""
    enc = make_encoding(192, 256, S=2, group_rows=64, seed=11)
    bias = torch.randn(192, generator=torch.Generator().manual_seed(1))
    mod = PackedGroupedBlockRVQLinear(enc, bias).to(gpu_device)
    for x_dtype in (torch.bfloat16, torch.float16):
        x = torch.randn(2, m, 256, generator=torch.Generator().manual_seed(m)).to(x_dtype)
        y = mod(x.to(gpu_device))
        assert y.shape == (2, m, 192) and y.dtype == x_dtype
        w_ref = oracle_weight(module_buffers_as_encoding(mod), x_dtype)
        b_ref = mod.bias.cpu().to(x_dtype)
        ref = c_oracle.linear_f64(x.reshape(-1, 256), w_ref, b_ref)
        ref_rounded = ref.to(x_dtype).double()
        got = y.reshape(-1, 192).cpu().double()
        # The 2e-3 bar is defined on fp32-accumulated outputs (tested above);
        # an output rounded to bf16 can itself be 2^-9 away, so here the bar is
        # one ulp of x dtype from the correctly rounded reference.
        ulp = 2.0 ** -7 if x_dtype == torch.bfloat16 else 2.0 ** -10
        assert bool(((got - ref_rounded).abs() <= ulp * ref.abs().clamp_min(1e-3)).all())


def test_fp32_activations(gpu_device):
    enc = make_encoding(64, 128, S=2, seed=5)
    mod = PackedGroupedBlockRVQLinear(enc).to(gpu_device)
    x = torch.randn(3, 128, generator=torch.Generator().manual_seed(2))
    y = mod(x.to(gpu_device))
    assert y.dtype == torch.float32
    w_ref = oracle_weight(module_buffers_as_encoding(mod), torch.float32)
    assert rel_err(y, c_oracle.linear_f64(x, w_ref)) <= 1e-6


def test_deterministic(gpu_device):
    enc = make_encoding(512, 1024, S=3, group_rows=256, seed=9)
    mod = PackedGroupedBlockRVQLinear(enc).to(gpu_device)
    for m in (1, 16, 100):
        x = torch.randn(m, 1024, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16).to(gpu_device)
        a = mod(x)
        b = mod(x)
        assert torch.equal(bits(a), bits(b))


def test_empty_batch(gpu_device):
    enc = make_encoding(64, 128, S=1, K=256, seed=1)
    mod = PackedGroupedBlockRVQLinear(enc).to(gpu_device)
    y = mod(torch.zeros(0, 128, dtype=torch.bfloat16, device=gpu_device))
    assert y.shape == (0, 64)


def test_bad_ids_refused(gpu_device):
    enc = make_encoding(32, 64, S=1, K=4096, seed=2)
    ids = enc.groups[0].stage_ids[0].clone()
    ids[3, 5] = 5000  # outside the 4096-entry codebook
    g0 = enc.groups[0]
    import dataclasses

    bad = dataclasses.replace(g0, stage_ids=(ids,))
    enc_bad = dataclasses.replace(enc, groups=(bad,))
    mod = PackedGroupedBlockRVQLinear(enc_bad).to(gpu_device)
    with pytest.raises(IndexError):
        mod(torch.zeros(1, 64, dtype=torch.bfloat16, device=gpu_device))


def test_cpu_input_fails_loudly(gpu_device):
    enc = make_encoding(32, 64, S=1, seed=2)
    mod = PackedGroupedBlockRVQLinear(enc).to(gpu_device)
    with pytest.raises(RuntimeError):
        mod(torch.zeros(1, 64, dtype=torch.bfloat16))


@pytest.mark.parametrize("M", [1, 16, 64])
def test_baseline_shapes_smoke(M, gpu_device):
    """One linear of each benchmark format at its real shape, checked at the
    2e-3 bar (M = 1 and 16 decode, 64 prefill)."""
    from wal2026_amd import synth

    for cname, (out_f, in_f) in [("c3", (4096, 4096)), ("c5", (3584, 3584)), ("c2", (2048, 2048))]:
        cfg = synth.CONFIGS[cname]
        gen = synth.generator(0)
        enc = synth.make_encoding(out_f, in_f, cfg, gen)
        mod = PackedGroupedBlockRVQLinear(enc).to(gpu_device)
        x = synth.make_activation(M, in_f, cfg.x_dtype, gen)
        y = mod._hip_linear(x.to(gpu_device), fast=False, out_dtype=torch.float32)
        rows = slice(0, 512)
        sub = module_buffers_as_encoding(mod)
        w_ref = oracle_weight(sub, cfg.x_dtype)[rows]
        ref = c_oracle.linear_f64(x, w_ref)
        assert rel_err(y[:, rows], ref) <= TOL, cname
