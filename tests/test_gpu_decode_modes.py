"""GPU parity of every decode-kernel layout (x-mode), forced and planned.

The decode kernel (M <= 16) has five ways of feeding the MFMA's activation
fragments (rvq_plan.h): x staged in LDS and read per item (lds), staged and
held in registers (reg), straight from global memory into registers (greg),
row runs transposed through LDS per item (gtr), and direct global loads per
item (global).  WAL2026_DECODE_XMODE forces one; every test asserts, through
wal_rvq_linear_info, the mode that the call it checks ran.

Bar (written in each test):
* fp32 outputs against the float64 contraction of the oracle's bit-exact
  weight: max|dy| / max|y| <= 2e-3 (the parity bar), and <= 1e-5 (what fp32
  accumulation of exact products gives);
* weights inside the kernel read out through one-hot activation rows
  (x[i] = e_c gives y[i, n] = W[n, c] exactly), bit for bit.
"""
from __future__ import annotations

import zlib

import pytest
import torch

from _cases import make_encoding, module_buffers_as_encoding, oracle_weight, rel_err
from oracle import c_oracle
from wal2026_amd import PackedGroupedBlockRVQLinear, _lib, synth

pytestmark = pytest.mark.gpu
TOL = 2e-3

# (name, out, in, S, K, id dtype, group_rows, scale_run); B = in / 8 blocks,
# nchunk = B / 64 chunks per row (more than the 8 waves: each wave takes
# several chunks per tile, CPT > 1)
LAYOUTS = [
    ("s2_u8_b64", 256, 512, 2, 256, None, None, None),
    ("s1_k4096_scale128_b128", 384, 1024, 1, 4096, torch.uint16, None, 128),
    ("s3_groups256_b48", 600, 384, 3, 256, None, 256, None),
    ("s1_k4096_scale32_b576", 96, 4608, 1, 4096, torch.uint16, None, 32),
    ("s2_u8_b640_groups", 80, 5120, 2, 256, None, 48, None),
]
MODES = ["reg", "lds", "greg", "gtr", "global"]


def _applies(layout, mode):
    return mode not in ("reg", "greg") or layout[2] // 8 <= 512


CASES = [(l, mode, m) for l in LAYOUTS for mode in MODES if _applies(l, mode) for m in (1, 4, 9, 16)]


def _module(layout, device):
    name, out_f, in_f, S, K, idt, gr, run = layout
    enc = make_encoding(out_f, in_f, S=S, K=K, id_dtype=idt, group_rows=gr, scale_run=run,
                        seed=zlib.crc32(name.encode()) % 1000)
    return PackedGroupedBlockRVQLinear(enc, matmul_strategy="hip_block_rvq").to(device)


def _onehot_cols(in_f: int, m: int) -> list[int]:
    """m distinct columns: both ends of the row, chunk and block edges, and
    columns of a wave's second chunk slot when the row has more than 8."""
    picks = [0, in_f - 1, 7, 8, 511, 512, in_f // 2, 513, 1, in_f - 8, 255, 256, in_f - 513, 4095, 4096, 3]
    out = []
    for c in picks:
        c = min(max(c, 0), in_f - 1)
        if c not in out:
            out.append(c)
    c = 2
    while len(out) < m:
        if c not in out:
            out.append(c)
        c += 5
    return out[:m]


def _check(mod, x_dtype, m, device, seed, *, want_mode=None, exact=True):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(m, mod.in_features, generator=gen).to(x_dtype)
    xd = x.to(device)
    try:
        info = mod.launch_info(xd)
    except _lib.WalError as e:
        # a forced layout whose LDS (x rows, tables, partial sums) does not
        # fit at this M; the planner never picks one
        if e.status == _lib.EUNSUPPORTED:
            pytest.skip(f"forced x-mode does not fit this layout at m={m}")
        raise
    assert info["kernel"] == "decode", info
    if want_mode is not None:
        assert info["x_mode"] == want_mode, info
    y = mod._hip_linear(xd, fast=False, out_dtype=torch.float32)
    w_ref = oracle_weight(module_buffers_as_encoding(mod), x_dtype)
    err = rel_err(y, c_oracle.linear_f64(x, w_ref))
    assert err <= TOL, f"{info}: max|dy|/max|y| = {err:.3e} > {TOL}"
    assert err <= 1e-5, f"{info}: {err:.3e} is above fp32 accumulation error"
    if exact:
        cols = _onehot_cols(mod.in_features, m)
        eye = torch.zeros(m, mod.in_features, dtype=x_dtype)
        for i, c in enumerate(cols):
            eye[i, c] = 1.0
        eyed = eye.to(device)
        assert mod.launch_info(eyed) == info
        got = mod._hip_linear(eyed, fast=False, out_dtype=torch.float32).cpu()
        for i, c in enumerate(cols):
            assert torch.equal(got[i], w_ref[:, c].float()), (info, i, c)
    return info


@pytest.mark.parametrize("layout,mode,m", CASES, ids=[f"{l[0]}-{mode}-m{m}" for l, mode, m in CASES])
@pytest.mark.parametrize("x_dtype", [torch.bfloat16, torch.float16], ids=["xbf16", "xf16"])
def test_forced_xmode_parity(layout, mode, m, x_dtype, gpu_device, monkeypatch):
    monkeypatch.setenv("WAL2026_DECODE_XMODE", mode)
    print(f"[decode-modes] {layout[0]} mode={mode} m={m} x={x_dtype}", flush=True)
    mod = _module(layout, gpu_device)
    _check(mod, x_dtype, m, gpu_device, seed=m * 31 + len(mode), want_mode=mode)


def _bench_linear(cname, out_f, in_f, dev, seed=0):
    cfg = synth.CONFIGS[cname]
    enc = synth.make_encoding(out_f, in_f, cfg, synth.generator(seed))
    return cfg, PackedGroupedBlockRVQLinear(enc, matmul_strategy="hip_block_rvq").to(dev)


# (id, config, out, in, m, x-mode the planner picks there)
FULL = [
    ("c3_down_m1", "c3", 4096, 14336, 1, "lds"),
    ("c3_down_m2", "c3", 4096, 14336, 2, "lds"),
    ("c3_down_m3", "c3", 4096, 14336, 3, "lds"),
    ("c3_down_m4", "c3", 4096, 14336, 4, "global"),
    ("c5_down_m1", "c5", 3584, 18944, 1, "lds"),
    ("c2_down_m1", "c2", 2048, 8192, 1, "lds"),
    ("c1_m1", "c1", 2048, 2048, 1, "reg"),
]


@pytest.mark.parametrize("case", FULL, ids=[c[0] for c in FULL])
def test_full_size_planned_modes(case, gpu_device, monkeypatch):
    """The benchmark linears whose planned decode layout no other test
    reaches: every down_proj at M <= 4 (x beyond the 4096 columns that sit in
    registers) and c1's 2048 x 2048 fp16 linear; parity of the whole output
    and one-hot readout of m weight columns."""
    monkeypatch.delenv("WAL2026_DECODE_XMODE", raising=False)
    name, cname, out_f, in_f, m, mode = case
    print(f"[decode-modes] full {name}", flush=True)
    cfg, mod = _bench_linear(cname, out_f, in_f, gpu_device)
    assert cfg.x_dtype == (torch.float16 if cname == "c1" else torch.bfloat16)
    _check(mod, cfg.x_dtype, m, gpu_device, seed=5, want_mode=mode)


def test_full_c3_down_linearity(gpu_device, monkeypatch):
    """y(x1 + x2) = y(x1) + y(x2) for the c3 down_proj (XM_LDS) over disjoint
    supports (x1 + x2 is exact), up to fp32 sums."""
    monkeypatch.delenv("WAL2026_DECODE_XMODE", raising=False)
    cfg, mod = _bench_linear("c3", 4096, 14336, gpu_device)
    x = torch.randn(1, 14336, generator=torch.Generator().manual_seed(8)).to(cfg.x_dtype)
    x1 = x.clone()
    x1[:, 7168:] = 0
    x2 = x - x1
    f = lambda t: mod._hip_linear(t.to(gpu_device), fast=False, out_dtype=torch.float32)
    assert mod.launch_info(x.to(gpu_device))["x_mode"] == "lds"
    assert rel_err(f(x1) + f(x2), f(x)) <= 1e-5
