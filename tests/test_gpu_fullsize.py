"""GPU parity at the benchmark configurations' full sizes.

Whole weight matrices of the real shapes (Llama-3-8B gate_proj for c3 and c4,
Qwen2.5-7B gate_proj for c5) are checked against the CPU oracle:
* the dequantised weight bit for bit (the whole matrix);
* decode outputs (M = 1) in fp32 against the float64 contraction of the
  oracle's weight, max|dy| / max|y| <= 2e-3;
* prefill outputs (M = 2048) on a sample of activation rows, same bar (the
  oracle's float64 contraction of every row would take minutes);
* linearity of the decode kernel over the full matrix:
  y(x1 + x2) = y(x1) + y(x2) up to fp32 accumulation.
"""
from __future__ import annotations

import pytest
import torch

from _cases import bits, module_buffers_as_encoding, oracle_weight, rel_err
from oracle import c_oracle
from wal2026_amd import PackedGroupedBlockRVQLinear, _lib, synth

pytestmark = pytest.mark.gpu
TOL = 2e-3

SHAPES = [
    ("c3_gate", "c3", 14336, 4096),
    ("c4_gate", "c4", 14336, 4096),
    ("c5_gate", "c5", 18944, 3584),
]


def _layer(cname, out_f, in_f, dev, seed=0):
    cfg = synth.CONFIGS[cname]
    gen = synth.generator(seed)
    enc = synth.make_encoding(out_f, in_f, cfg, gen)
    return cfg, PackedGroupedBlockRVQLinear(enc, matmul_strategy="hip_block_rvq").to(dev), gen


@pytest.mark.parametrize("name,cname,out_f,in_f", SHAPES, ids=[s[0] for s in SHAPES])
def test_full_weight_bitexact(name, cname, out_f, in_f, gpu_device):
    print(f"[fullsize] reconstruct {name} {out_f}x{in_f}", flush=True)
    cfg, mod, _ = _layer(cname, out_f, in_f, gpu_device)
    got = mod.reconstruct_weight(cfg.x_dtype).cpu()
    want = oracle_weight(module_buffers_as_encoding(mod), cfg.x_dtype)
    assert torch.equal(bits(got), bits(want)), name


# (shape, m, the planner's (x-mode, table slots) there)
DECODE_CASES = [(SHAPES[0], 1, ("reg", 2)), (SHAPES[0], 4, ("greg", 2)), (SHAPES[0], 16, ("greg", 1)),
                (SHAPES[2], 1, ("reg", 2))]


@pytest.mark.parametrize("shape,m,plan", DECODE_CASES, ids=[f"{s[0]}_m{m}" for s, m, _ in DECODE_CASES])
def test_full_decode_parity_and_linearity(shape, m, plan, gpu_device, monkeypatch):
    """The gate_proj shapes (4096 or 3584 columns: every wave owns one
    64-block chunk, so its x fragments are held in registers).  M = 1, 4, 16
    at c3 cover the layouts the launch planner picks there: x rows staged in
    LDS with two table slots (reg); x fragments straight from global memory
    into registers with two slots (greg), then with one slot."""
    monkeypatch.delenv("WAL2026_DECODE_XMODE", raising=False)
    name, cname, out_f, in_f = shape
    print(f"[fullsize] decode {name} m={m}", flush=True)
    cfg, mod, gen = _layer(cname, out_f, in_f, gpu_device)
    x = synth.make_activation(m, in_f, cfg.x_dtype, gen)
    info = mod.launch_info(x.to(gpu_device))
    assert (info["x_mode"], info["table_slots"]) == plan, info
    y = mod._hip_linear(x.to(gpu_device), fast=False, out_dtype=torch.float32)
    w_ref = oracle_weight(module_buffers_as_encoding(mod), cfg.x_dtype)
    assert rel_err(y, c_oracle.linear_f64(x, w_ref)) <= TOL, name
    # linearity: x1 and x2 chosen so that x1 + x2 is exact in bf16 (disjoint
    # supports), so y(x1 + x2) and y(x1) + y(x2) differ only by fp32 sums
    x1 = x.clone()
    x1[:, in_f // 2:] = 0
    x2 = x - x1
    dev = gpu_device
    y1 = mod._hip_linear(x1.to(dev), fast=False, out_dtype=torch.float32)
    y2 = mod._hip_linear(x2.to(dev), fast=False, out_dtype=torch.float32)
    assert rel_err(y1 + y2, y) <= 1e-5, name


@pytest.mark.parametrize("tile", ["auto", "short", "wide"])
def test_full_prefill_parity_sampled_rows(tile, gpu_device, monkeypatch):
    """c4: S = 2, K = 256, 8-bit ids, bf16 x, M = 2048 through the prefill
    kernel, with the launcher's tile choice and with the 128 x 256 and 256 x
    128 tiles forced; 28 sampled rows of y against the oracle."""
    if tile != "auto":
        monkeypatch.setenv("WAL2026_PREFILL_TILE", tile)
    print(f"[fullsize] prefill c4 gate 2048x14336x4096 tile={tile}", flush=True)
    cfg, mod, gen = _layer("c4", 14336, 4096, gpu_device)
    x = synth.make_activation(2048, 4096, cfg.x_dtype, gen)
    y = mod._hip_linear(x.to(gpu_device), fast=False, out_dtype=torch.float32).cpu()
    rows = torch.randperm(2048, generator=torch.Generator().manual_seed(5))[:24]
    rows = torch.cat([rows, torch.tensor([0, 127, 128, 2047])])
    w_ref = oracle_weight(module_buffers_as_encoding(mod), cfg.x_dtype)
    ref = c_oracle.linear_f64(x[rows], w_ref)
    assert rel_err(y[rows], ref) <= TOL


def test_full_prefill_fused_gate_up(gpu_device, monkeypatch):
    """c4's fused gate_up launch (28672 x 4096, M = 2048): 112 weight tiles by
    8 x tiles, so the 256 x 256 kernel runs 96 tiles whole and splits the last
    16 into 256 x 128 halves (the round that whole tiles would leave half
    empty); gate and up are different encodings.  28 sampled rows of y
    against the oracle, and the fused outputs equal to each linear's own."""
    from wal2026_amd import FusedBlockRVQLinears

    monkeypatch.delenv("WAL2026_PREFILL_TILE", raising=False)
    # the fused kernel, unsplit, for the module forwards too: its per-row
    # arithmetic is the same in the fused and the separate launches, so they
    # agree bit for bit (the two-pass form's library GEMM may sum a 28672-row
    # and a 14336-row product in different orders)
    monkeypatch.setenv("WAL2026_PREFILL_TWO_PASS", "0")
    monkeypatch.setenv("WAL2026_PREFILL_KSPLIT", "1")
    print("[fullsize] prefill c4 gate_up 2048x28672x4096", flush=True)
    cfg, gate, gen = _layer("c4", 14336, 4096, gpu_device, seed=0)
    _, up, _ = _layer("c4", 14336, 4096, gpu_device, seed=1)
    x = synth.make_activation(2048, 4096, cfg.x_dtype, gen)
    xd = x.to(gpu_device)
    fused = FusedBlockRVQLinears([gate, up])
    assert fused.launch_info(xd)["tile_shape"] == "tall"
    # the fused launch with fp32 outputs (the 2e-3 bar is for fp32 outputs),
    # then the module's own bf16 outputs
    c = fused._call_for(xd)
    y32 = _lib.ops().rvq_linear(xd, c[0], c[1], c[2], None, torch.float32).cpu()
    yg, yu = fused(xd)
    rows = torch.randperm(2048, generator=torch.Generator().manual_seed(6))[:24]
    rows = torch.cat([rows, torch.tensor([0, 255, 256, 2047])])
    for i, (mod, y) in enumerate(((gate, yg), (up, yu))):
        w_ref = oracle_weight(module_buffers_as_encoding(mod), cfg.x_dtype)
        ref = c_oracle.linear_f64(x[rows], w_ref)
        assert rel_err(y32[rows, 14336 * i:14336 * (i + 1)], ref) <= TOL
        assert torch.equal(bits(y.contiguous()), bits(mod(xd)))


@pytest.mark.parametrize("m", [5, 9, 16])
def test_full_decode_down_proj_transposed_x(m, gpu_device, monkeypatch):
    """c3 down_proj (4096 x 14336) at 4 < M <= 16: x (up to 458 KB) fits
    neither LDS nor registers, so each item's x fragments are loaded as row
    runs and transposed through a per-wave LDS scratch, one or two 8-row
    halves (M = 5: one half; 9: a partial second half; 16: both full)."""
    monkeypatch.delenv("WAL2026_DECODE_XMODE", raising=False)
    print(f"[fullsize] decode c3_down m={m}", flush=True)
    cfg, mod, gen = _layer("c3", 4096, 14336, gpu_device)
    x = synth.make_activation(m, 14336, cfg.x_dtype, gen)
    assert mod.launch_info(x.to(gpu_device))["x_mode"] == "gtr"
    y = mod._hip_linear(x.to(gpu_device), fast=False, out_dtype=torch.float32)
    w_ref = oracle_weight(module_buffers_as_encoding(mod), cfg.x_dtype)
    assert rel_err(y, c_oracle.linear_f64(x, w_ref)) <= TOL
    # one-hot rows read the kernel's weights out exactly: a distinct column
    # per row (rows 8-15 go through the second transpose half), spread over
    # the row, including the first and last block of a chunk
    cols = [0, 7, 8, 511, 512, 4095, 7000, 14335, 1, 63, 64, 1023, 1024, 8191, 8192, 14329][: m]
    eye = torch.zeros(m, 14336, dtype=cfg.x_dtype)
    for i, c in enumerate(cols):
        eye[i, c] = 1.0
    got = mod._hip_linear(eye.to(gpu_device), fast=False, out_dtype=torch.float32).cpu()
    for i, c in enumerate(cols):
        assert torch.equal(got[i], w_ref[:, c].float()), (m, c)
