"""Pins the CPU oracle (oracle/rvq_oracle.c) before anything is compared with it.

Each check is chosen so that a plausible mistake in the restatement fails it:
* conversions against numpy's and torch's casts over random bit patterns
  (a wrong tie rule, subnormal shift or overflow bound fails);
* reconstruct_weight / reconstruct_weight_fast bit-for-bit against the
  reference's torch op sequence executed by torch (oracle/ref_ops.py): a
  dropped stage, a wrong rounding point, a missing scale or a transposed
  index fails;
* closed forms and invariants that do not depend on either implementation:
  S = 1 with a constant codebook, an all-zero stage, one-hot contraction,
  a float64 error bound, linearity of the contraction;
* the committed golden fixtures (tests/golden/*.json), whose expected values
  were derived by hand from the IEEE-754 definitions (see make_golden.py).
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from _cases import bits, make_encoding, oracle_group
from oracle import c_oracle, ref_ops

GOLDEN = Path(__file__).resolve().parent / "golden"


def _random_f32(n, seed):
    g = torch.Generator().manual_seed(seed)
    u = torch.randint(0, 2**32, (n,), generator=g, dtype=torch.int64).to(torch.int32)
    return u.view(torch.float32)


def test_f32_to_f16_matches_numpy_and_torch():
    L = c_oracle.lib()
    f = _random_f32(60000, 1)
    # add the values around every rounding boundary that matters
    specials = torch.tensor([0.0, -0.0, 65504.0, 65519.996, 65520.0, 65536.0, 2.0**-24, 2.0**-25, 3 * 2.0**-26,
                             2.0**-25 * 1.0000001, 2.0**-14, 2.0**-14 - 2.0**-25, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11,
                             float("inf"), -float("inf")])
    f = torch.cat([f, specials])
    with np.errstate(over="ignore"):
        want_np = f.numpy().astype(np.float16).view(np.uint16)
    want_t = f.to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([L.or_f32_to_f16(float(v)) for v in f.tolist()], dtype=np.uint16)
    finite = ~np.isnan(f.numpy())
    assert np.array_equal(got[finite], want_np[finite])
    assert np.array_equal(got[finite], want_t[finite])


def test_f32_to_bf16_matches_torch():
    L = c_oracle.lib()
    f = torch.cat([_random_f32(60000, 2), torch.tensor([1.0 + 2.0**-8, 1.0 + 3 * 2.0**-8, 3.3895314e38, 3.39e38])])
    want = f.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([L.or_f32_to_bf16(float(v)) for v in f.tolist()], dtype=np.uint16)
    finite = ~np.isnan(f.numpy())
    assert np.array_equal(got[finite], want[finite])
    assert L.or_f32_to_bf16(float("nan")) == 0x7FC0


def test_f16_to_f32_exact_for_all_patterns():
    L = c_oracle.lib()
    allh = np.arange(65536, dtype=np.uint16)
    want = allh.view(np.float16).astype(np.float32)
    got = np.array([L.or_f16_to_f32(int(h)) for h in allh], dtype=np.float32)
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))
    assert np.isnan(got[~ok]).all()


CASES = [
    dict(out_features=48, in_features=72, d=8, S=3, K=256),
    dict(out_features=40, in_features=64, d=8, S=1, K=4096),
    dict(out_features=33, in_features=50, d=4, S=2, K=64, stage_scales=True),
    dict(out_features=32, in_features=64, d=8, S=2, K=256, block_scale=True),
    dict(out_features=32, in_features=96, d=32, S=2, K=256, cb_dtype=torch.bfloat16),
    dict(out_features=64, in_features=64, d=8, S=2, K=256, special=True),
]


@pytest.mark.parametrize("case", CASES, ids=[f"case{i}" for i in range(len(CASES))])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "f16", "f32"])
def test_reconstruct_matches_torch_ops(case, out_dtype):
    enc = make_encoding(**case, seed=7)
    for g in enc.groups:
        got = c_oracle.reconstruct_weight(oracle_group(g), out_dtype)
        want = ref_ops.reconstruct_weight(list(g.stage_ids), list(g.codebooks), g.row_scale, g.original_shape[1],
                                          out_dtype, g.stage_scales, g.block_scale)
        assert torch.equal(bits(got), bits(want))


@pytest.mark.parametrize("case", [c for c in CASES if not c.get("block_scale")], ids=lambda c: f"S{c['S']}d{c['d']}")
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "f16", "f32"])
def test_reconstruct_fast_matches_torch_ops(case, out_dtype):
    enc = make_encoding(**case, seed=8)
    S = case["S"]
    for g in enc.groups:
        for active in ([0], list(range(S)), [s for s in range(S) if s % 2 == 0] or [0]):
            got = c_oracle.reconstruct_weight_fast(oracle_group(g), active, out_dtype)
            want = ref_ops.reconstruct_weight_fast(list(g.stage_ids), list(g.codebooks), g.row_scale,
                                                   g.original_shape[1], out_dtype, active, g.stage_scales)
            assert torch.equal(bits(got), bits(want)), active


def test_active_stage_indices_fixture():
    data = json.loads((GOLDEN / "active_stages.json").read_text())
    for item in data:
        got = ref_ops.active_stage_indices(item["stages_per_split"], item["effective"])
        assert got == item["expected"], item


def test_golden_vectors():
    """Hand-derived IEEE values (tests/golden/reconstruct_golden.json)."""
    data = json.loads((GOLDEN / "reconstruct_golden.json").read_text())
    for item in data:
        g = c_oracle.OracleGroup(
            [torch.tensor(ids, dtype=torch.uint8).reshape(1, -1) for ids in item["ids"]],
            [torch.tensor(cb, dtype=torch.int16).view(torch.float16).reshape(item["K"], item["d"])
             for cb in item["codebook_bits"]],
            torch.tensor(item["row_scale_bits"], dtype=torch.int16).view(torch.float16).reshape(1, 1),
            in_features=item["in_features"], block_size=item["d"])
        out_dtype = {"bf16": torch.bfloat16, "f16": torch.float16}[item["out_dtype"]]
        w = c_oracle.reconstruct_weight(g, out_dtype)
        got = [v & 0xFFFF for v in bits(w).reshape(-1).tolist()]
        assert got == item["expected_bits"], item["name"]


def test_s1_constant_codebook_closed_form():
    """S = 1, every codeword c: W = rne(rne(c) * rne(s)) independently of ids."""
    for c in (0.0137, -0.0021, 1.5e-6, 0.5):
        for s in (0.75, 1.3, 0.5039):
            cb = torch.full((16, 8), c).to(torch.float16)
            ids = torch.randint(0, 16, (5, 4), generator=torch.Generator().manual_seed(1)).to(torch.uint8)
            rs = torch.full((5, 1), s).to(torch.float16)
            g = c_oracle.OracleGroup([ids], [cb], rs, in_features=32, block_size=8)
            w = c_oracle.reconstruct_weight(g, torch.bfloat16)
            c16 = float(torch.tensor(c).to(torch.float16))
            s16 = float(torch.tensor(s).to(torch.float16))
            expect = float(torch.tensor(float(torch.tensor(c16).to(torch.bfloat16)) *
                                        float(torch.tensor(s16).to(torch.bfloat16))).to(torch.bfloat16))
            assert torch.all(w.float() == expect)


def test_zero_stage_adds_nothing():
    enc = make_encoding(24, 64, d=8, S=2, K=32, seed=3)
    g = enc.groups[0]
    zero_cb = torch.zeros_like(g.codebooks[1])
    one = c_oracle.OracleGroup([g.stage_ids[0]], [g.codebooks[0]], g.row_scale, in_features=64, block_size=8)
    two = c_oracle.OracleGroup(list(g.stage_ids), [g.codebooks[0], zero_cb], g.row_scale, in_features=64, block_size=8)
    for dt in (torch.bfloat16, torch.float16, torch.float32):
        a = c_oracle.reconstruct_weight(one, dt)
        b = c_oracle.reconstruct_weight(two, dt)
        assert torch.equal(a, b)  # value-equal (+0 vs -0 allowed)


def test_float64_error_bound():
    """W_bf16 = rne(rne(t) * rne(s)) with t the fp32 stage sum: three bf16
    roundings of relative size <= u = 2^-8 each, plus the fp32 sum error
    (<= 2 * 2^-24 * s * sum|c| for three stages).  Checked in float64 against
    s * sum(c) computed from the raw inputs."""
    enc = make_encoding(64, 128, d=8, S=3, K=256, seed=4)
    g = enc.groups[0]
    w = c_oracle.reconstruct_weight(oracle_group(g), torch.bfloat16).double()
    vals = [c.double()[i.long().reshape(-1)] for i, c in zip(g.stage_ids, g.codebooks)]
    s = g.row_scale.double()
    exact = sum(vals).view(64, 128) * s
    abs_sum = sum(v.abs() for v in vals).view(64, 128) * s
    u = 2.0 ** -8
    bound = ((1 + u) ** 3 - 1) * exact.abs() + (1 + u) ** 3 * 2 * 2.0 ** -24 * abs_sum + 2.0 ** -133
    assert bool(((w - exact).abs() <= bound).all())
    # and the bound is not vacuous: a dropped stage breaks it
    w_bad = c_oracle.reconstruct_weight(c_oracle.OracleGroup(list(g.stage_ids[:2]), list(g.codebooks[:2]),
                                                             g.row_scale, in_features=128, block_size=8),
                                        torch.bfloat16).double()
    assert not bool(((w_bad - exact).abs() <= bound).all())


def test_linear_f64_matches_numpy():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(7, 33, generator=g).to(torch.bfloat16)
    w = torch.randn(11, 33, generator=g).to(torch.float16)
    b = torch.randn(11, generator=g).to(torch.bfloat16)
    y = c_oracle.linear_f64(x, w, b).numpy()
    want = x.double().numpy() @ w.double().numpy().T + b.double().numpy()
    assert np.allclose(y, want, rtol=1e-15, atol=1e-15)


def test_onehot_contraction_reads_weights():
    """The one-hot probe the reference's gate uses (x = e_k -> y[:, n] = W[n, k])."""
    enc = make_encoding(16, 32, d=8, S=2, K=64, seed=6)
    w = c_oracle.reconstruct_weight(oracle_group(enc.groups[0]), torch.bfloat16)
    x = torch.eye(32, dtype=torch.bfloat16)
    y = c_oracle.linear_f64(x, w)
    assert torch.equal(y.t().float(), w.float())


def test_triton_semantics_closed_form():
    """S = 1, unit row scale: out = round_x(x @ round_x(cb[ids])^T)."""
    g = torch.Generator().manual_seed(9)
    ids = torch.randint(0, 32, (1, 12, 4), generator=g).to(torch.uint8)
    cb = (torch.randn(1, 32, 8, generator=g) * 0.05).to(torch.float16)
    x = torch.randn(3, 32, generator=g).to(torch.bfloat16)
    rs = torch.ones(12, dtype=torch.float16)
    out = c_oracle.triton_rvq_matmul(x, ids, cb, rs, out_dtype=torch.float32)
    w = ref_ops.triton_rvq_matmul_weight(ids, cb, torch.bfloat16)
    want = x.double() @ w.double().t()
    assert torch.allclose(out.double(), want, rtol=1e-6, atol=1e-7)


def test_triton_semantics_row_scale_on_accumulator():
    """The Triton kernel applies the row scale to the fp32 accumulator, not
    to each weight (src/triton_id_matmul.py:212-216).  Pinned three ways:
    * power-of-two scales: out = rho * x @ round_x(sum_s cb)^T, the product
      exact in fp32, against the float64 closed form;
    * scales in [0.5, 1.5): the same closed form in float64, within fp32
      rounding (rtol 2e-6);
    * a planted mistake, the scale folded into each rounded weight
      (round_x(round_x(w) * rho)), misses that bound by orders of magnitude,
      so the check tells the two apart."""
    g = torch.Generator().manual_seed(19)
    S, N, B, d, K = 2, 24, 6, 8, 64
    ids = torch.randint(0, K, (S, N, B), generator=g).to(torch.uint8)
    cb = (torch.randn(S, K, d, generator=g) * 0.05).to(torch.float16)
    x = torch.randn(4, B * d, generator=g).to(torch.bfloat16)
    w = ref_ops.triton_rvq_matmul_weight(ids, cb, torch.bfloat16).double()  # [N, B*d] in x dtype
    base = x.double() @ w.t()
    pow2 = torch.tensor([2.0 ** ((i % 7) - 3) for i in range(N)], dtype=torch.float16)
    out = c_oracle.triton_rvq_matmul(x, ids, cb, pow2, out_dtype=torch.float32).double()
    assert torch.allclose(out, base * pow2.double(), rtol=1e-6, atol=0)
    rho = (torch.rand(N, generator=g) + 0.5).to(torch.float16)
    out = c_oracle.triton_rvq_matmul(x, ids, cb, rho, out_dtype=torch.float32).double()
    want = base * rho.double()
    assert float(((out - want).abs() / want.abs().max()).max()) <= 2e-6
    planted = x.double() @ (w * rho.double().unsqueeze(1)).to(torch.bfloat16).double().t()
    assert float(((planted - want).abs() / want.abs().max()).max()) > 1e-4
    # a dropped scale is caught too
    assert not torch.allclose(c_oracle.triton_rvq_matmul(x, ids, cb, torch.ones(N, dtype=torch.float16),
                                                         out_dtype=torch.float32).double(), want, rtol=1e-3)


def test_id_route_weight_golden():
    """Hand-derived fp16/bf16 rounding of both route modes (mode 0: product in
    the buffers' dtype then cast, src/runtime.py:89-97; mode 1: operands cast
    to x dtype then multiplied, src/triton_id_matmul.py:59-60), including
    double-rounding ties, an fp16 overflow only mode 0 takes and a subnormal
    tie (tests/golden/route_golden.json, derivations in make_golden.py)."""
    cases = json.loads((GOLDEN / "route_golden.json").read_text())
    dt = {"f16": torch.float16, "bf16": torch.bfloat16}
    for c in cases:
        bdt, xdt = dt[c["buffer_dtype"]], dt[c["x_dtype"]]
        sgn = lambda v: v - 0x10000 if v >= 0x8000 else v
        cs = torch.tensor([sgn(c["codebook_sum_bits"])], dtype=torch.int16).view(bdt)
        rs = torch.tensor([[sgn(c["row_scale_bits"])]], dtype=torch.int16).view(bdt)
        ids = torch.zeros(1, 1, dtype=torch.int16)
        for mode in (0, 1):
            got = c_oracle.id_route_weight(ids, cs, rs, mode=mode, x_dtype=xdt)
            assert int(bits(got).reshape(-1)[0]) & 0xFFFF == c[f"mode{mode}_bits"], (c["name"], mode)


def test_id_route_weight_matches_torch_ops():
    g = torch.Generator().manual_seed(10)
    ids = torch.randint(0, 300, (9, 40), generator=g).to(torch.int16)
    cs = (torch.randn(300, generator=g) * 0.1).to(torch.float16)
    rs = (torch.rand(9, 1, generator=g) + 0.5).to(torch.float16)
    for mode in (0, 1):
        for xdt in (torch.bfloat16, torch.float16):
            got = c_oracle.id_route_weight(ids, cs, rs, mode=mode, x_dtype=xdt)
            want = ref_ops.id_route_weight(ids, cs, rs, mode=mode, x_dtype=xdt)
            assert torch.equal(bits(got), bits(want)), (mode, xdt)


def test_linearity_of_contraction():
    """x1 + x2 contracts to y1 + y2 (in float64) on the oracle weight."""
    enc = make_encoding(20, 48, d=8, S=2, K=64, seed=12)
    w = c_oracle.reconstruct_weight(oracle_group(enc.groups[0]), torch.float32)
    g = torch.Generator().manual_seed(1)
    x1 = torch.randn(2, 48, generator=g)
    x2 = torch.randn(2, 48, generator=g)
    y12 = c_oracle.linear_f64(x1 + x2, w)
    assert torch.allclose(y12, c_oracle.linear_f64(x1, w) + c_oracle.linear_f64(x2, w), rtol=1e-5, atol=1e-6)
    assert not math.isnan(float(y12.sum()))


def _ulp_dist(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in units in the last place between two 16-bit float tensors
    (monotone integer view of the bit patterns)."""
    def key(t):
        v = bits(t).to(torch.int32) & 0xFFFF
        return torch.where(v >= 0x8000, 0x8000 - v, v)
    return (key(a) - key(b)).abs()


@pytest.mark.parametrize("x_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("S,stage_scales,in_f", [(1, False, 64), (2, True, 44), (3, False, 40)])
def test_stagewise_matches_torch_ops(x_dtype, S, stage_scales, in_f):
    """or_stagewise_linear against the reference's op sequence run by torch
    (src/runtime.py:878-894).  Both round each stage's contraction to x dtype;
    they may differ only where fp32 accumulation order flips that rounding, so
    at most 1 ulp, and rarely."""
    enc = make_encoding(24, in_f, d=8, S=S, K=64, stage_scales=stage_scales, seed=20 + S)
    g0 = enc.groups[0]
    x = torch.randn(5, in_f, generator=torch.Generator().manual_seed(3)).to(x_dtype)
    got = c_oracle.stagewise_linear(oracle_group(g0), x)
    want = ref_ops.stagewise_block_matmul(x, list(g0.stage_ids), list(g0.codebooks), g0.row_scale, in_f,
                                          g0.stage_scales)
    d = _ulp_dist(got, want)
    assert int(d.max()) <= 1
    assert float((d == 0).double().mean()) >= 0.95


def test_stagewise_closed_form_single_stage():
    """S = 1, unit row scale: y = round_x(x . round_x(cb[ids])^T), i.e. the
    float64 contraction of the reconstructed weight rounded once."""
    enc = make_encoding(16, 48, d=8, S=1, K=32, seed=31)
    g0 = enc.groups[0]
    g0 = type(g0)(**{**g0.__dict__, "row_scale": torch.ones_like(g0.row_scale)})
    x = torch.randn(4, 48, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    got = c_oracle.stagewise_linear(oracle_group(g0), x)
    w = c_oracle.reconstruct_weight(oracle_group(g0), torch.bfloat16)
    want = c_oracle.linear_f64(x, w).float().to(torch.bfloat16)
    assert torch.equal(bits(got), bits(want))


def test_stagewise_rejects_block_scale():
    enc = make_encoding(8, 16, d=8, S=1, K=16, block_scale=True, seed=2)
    with pytest.raises(ValueError):
        c_oracle.stagewise_linear(oracle_group(enc.groups[0]), torch.zeros(1, 16, dtype=torch.float16))
