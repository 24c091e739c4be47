"""The drop-in boundary end to end, on the GPU.

A tiny model with the module paths of TARGET_LINEAR_SUFFIXES
(``layers.N.self_attn.{q,k,v,o}_proj``, ``layers.N.mlp.{gate,up,down}_proj``):
* encodings saved as the reference's v1 map file (src/encoding_io.py:10-94),
  built here as a plain dict in that layout (not with this build's writer),
  loaded with load_grouped_encoding_map, installed with
  replace_with_preencoded_packed_block_rvq, and run;
* replace_with_packed_block_rvq (encode on the device, then install) once.
Each installed layer's forward is checked against the oracle (weights
bit-exact through reconstruct_weight; fp32 outputs <= 2e-3, observed ~1e-6),
and the returned stat dicts carry exactly the reference's keys
(src/runtime.py:2116-2141, :2183-2197).
"""
from __future__ import annotations

import pytest
import torch
from torch import nn

from _cases import bits, make_encoding, module_buffers_as_encoding, oracle_weight, rel_err
from oracle import c_oracle
from wal2026_amd import (TARGET_LINEAR_SUFFIXES, FusedBlockRVQLinears, PackedGroupedBlockRVQLinear,
                         load_grouped_encoding_map, replace_with_packed_block_rvq,
                         replace_with_preencoded_packed_block_rvq, set_effective_stages_by_name)

pytestmark = pytest.mark.gpu
TOL = 2e-3

# keys of the reference's per-layer stat dicts
PREENCODED_KEYS = {"name", "tensor_name", "runtime_decision", "matmul_strategy", "matmul_chunk_rows",
                   "local_palette_group_cols", "hot_topk", "hot_score_mode", "hot_min_stage_share",
                   "hot_score_threshold_ratio", "rel_mse", "storage_bytes", "bits_per_weight"}
ENCODE_KEYS = PREENCODED_KEYS | {"group_rows", "block_size", "codebook_size", "num_stages", "product_splits",
                                 "normalize_blocks", "transform_kind", "calibrate_stage_scales",
                                 "residual_correction"}

HIDDEN, KV, INTER = 256, 64, 512
SHAPES = {"self_attn.q_proj": (HIDDEN, HIDDEN), "self_attn.k_proj": (KV, HIDDEN), "self_attn.v_proj": (KV, HIDDEN),
          "self_attn.o_proj": (HIDDEN, HIDDEN), "mlp.gate_proj": (INTER, HIDDEN), "mlp.up_proj": (INTER, HIDDEN),
          "mlp.down_proj": (HIDDEN, INTER)}


class _Attn(nn.Module):
    def __init__(self):
        super().__init__()
        self.q_proj = nn.Linear(HIDDEN, HIDDEN, bias=True)
        self.k_proj = nn.Linear(HIDDEN, KV, bias=False)
        self.v_proj = nn.Linear(HIDDEN, KV, bias=False)
        self.o_proj = nn.Linear(HIDDEN, HIDDEN, bias=False)


class _Mlp(nn.Module):
    def __init__(self):
        super().__init__()
        self.gate_proj = nn.Linear(HIDDEN, INTER, bias=False)
        self.up_proj = nn.Linear(HIDDEN, INTER, bias=False)
        self.down_proj = nn.Linear(INTER, HIDDEN, bias=False)


class _Layer(nn.Module):
    def __init__(self):
        super().__init__()
        self.self_attn = _Attn()
        self.mlp = _Mlp()


class TinyModel(nn.Module):
    def __init__(self, n_layers=2):
        super().__init__()
        self.layers = nn.ModuleList([_Layer() for _ in range(n_layers)])


def _v1_group(enc) -> dict:
    """One BlockRVQEncoding as the reference's v1 field dict (src/encoding_io.py:10-31)."""
    cpu = lambda t: None if t is None else t.detach().cpu()
    return {
        "stage_ids": [t.cpu() for t in enc.stage_ids],
        "codebooks": [t.cpu() for t in enc.codebooks],
        "stage_value_dims": list(enc.stage_value_dims),
        "stages_per_split": list(enc.stages_per_split),
        "stage_scales": cpu(enc.stage_scales),
        "residual_correction": enc.residual_correction,
        "residual_signs": cpu(enc.residual_signs),
        "residual_scale": cpu(enc.residual_scale),
        "row_scale": enc.row_scale.cpu(),
        "block_scale": cpu(enc.block_scale),
        "transform_kind": enc.transform_kind,
        "transform_matrix": cpu(enc.transform_matrix),
        "transform_bias": cpu(enc.transform_bias),
        "product_splits": int(enc.product_splits),
        "original_shape": list(enc.original_shape),
        "padded_cols": int(enc.padded_cols),
        "block_size": int(enc.block_size),
        "sample_rel_mse": float(enc.sample_rel_mse),
    }


def _check_layer(mod: PackedGroupedBlockRVQLinear, x_dtype, device, m=3, seed=0):
    w = mod.reconstruct_weight(out_dtype=x_dtype).cpu()
    w_ref = oracle_weight(module_buffers_as_encoding(mod), x_dtype)
    assert torch.equal(bits(w), bits(w_ref))
    x = torch.randn(m, mod.in_features, generator=torch.Generator().manual_seed(seed)).to(x_dtype)
    y = mod._hip_linear(x.to(device), fast=False, out_dtype=torch.float32)
    b = None if mod.bias is None else mod.bias.cpu().to(x_dtype)
    err = rel_err(y, c_oracle.linear_f64(x, w_ref, b))
    assert err <= TOL and err <= 1e-5, err
    yx = mod(x.to(device))
    assert yx.dtype == x_dtype and yx.shape == (m, mod.out_features)


def test_preencoded_v1_file_install_and_forward(tmp_path, gpu_device):
    torch.manual_seed(0)
    model = TinyModel().to(gpu_device)
    encodings = {}
    for li in range(2):
        for j, (suffix, (out_f, in_f)) in enumerate(SHAPES.items()):
            # two formats: attention 2-stage uint8 in 64-row groups, MLP 1-stage
            # 4096-entry int16 with scales shared by 16-row runs
            if suffix.startswith("self_attn"):
                enc = make_encoding(out_f, in_f, S=2, K=256, group_rows=64, seed=100 * li + j)
            else:
                enc = make_encoding(out_f, in_f, S=1, K=4096, seed=100 * li + j, scale_run=16)
            encodings[f"layers.{li}.{suffix}"] = enc
    assert {n.split(".", 2)[2] for n in encodings} == set(TARGET_LINEAR_SUFFIXES)
    payload = {"version": 1, "encodings": {
        name: {"groups": [_v1_group(g) for g in enc.groups], "row_slices": [list(s) for s in enc.row_slices],
               "original_shape": list(enc.original_shape)} for name, enc in encodings.items()}}
    path = tmp_path / "encodings_v1.pt"
    torch.save(payload, path)
    loaded = load_grouped_encoding_map(path)
    assert set(loaded) == set(encodings)
    stats = replace_with_preencoded_packed_block_rvq(model, loaded, matmul_strategy="hip_block_rvq")
    assert len(stats) == 14
    for st in stats:
        assert set(st) == PREENCODED_KEYS, st["name"]
        assert st["runtime_decision"] == "preencoded_packed_block_rvq" and st["matmul_strategy"] == "hip_block_rvq"
        assert st["storage_bytes"] > 0 and st["bits_per_weight"] > 0
    q = model.layers[0].self_attn.q_proj
    assert isinstance(q, PackedGroupedBlockRVQLinear) and q.bias is not None and q.bias.dtype == torch.bfloat16
    sd = model.state_dict()
    assert "layers.0.self_attn.q_proj.groups.0.stage_ids_0" in sd and "layers.1.mlp.down_proj.groups.0.row_scale" in sd
    for name, mod in model.named_modules():
        if isinstance(mod, PackedGroupedBlockRVQLinear):
            print(f"[boundary] {name}", flush=True)
            _check_layer(mod, torch.bfloat16, gpu_device, seed=len(name))
    # fusing the linears that share an input reproduces each one's output
    attn, mlp = model.layers[1].self_attn, model.layers[1].mlp
    x = torch.randn(2, HIDDEN, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(gpu_device)
    for lins in ((attn.q_proj, attn.k_proj, attn.v_proj), (mlp.gate_proj, mlp.up_proj)):
        fused = FusedBlockRVQLinears(lins)(x)
        for got, lin in zip(fused, lins):
            assert torch.equal(bits(got.contiguous()), bits(lin(x)))
    # per-role stage caps reach the installed groups (src/runtime.py:2289-2308)
    counts = set_effective_stages_by_name(model, 1, None)
    assert counts == {"attn": 8, "mlp": 0, "other": 0}
    assert model.layers[0].self_attn.q_proj.groups[0].effective_stages_per_split == 1


def test_v1_file_version_checked(tmp_path):
    path = tmp_path / "bad.pt"
    torch.save({"version": 2, "encodings": {}}, path)
    with pytest.raises(ValueError, match="unsupported encoding map version"):
        load_grouped_encoding_map(path)


def test_encode_and_install(gpu_device):
    """replace_with_packed_block_rvq: the encoder runs on the device (HIP
    assignment and centroid sums), then the installed layers run."""
    torch.manual_seed(1)
    model = TinyModel(n_layers=1).to(gpu_device)
    targets = ("layers.0.self_attn.q_proj", "layers.0.mlp.down_proj")
    stats = replace_with_packed_block_rvq(model, targets, group_rows=128, block_size=8, codebook_size=64,
                                          num_stages=2, sample_limit=4096, kmeans_iters=2,
                                          matmul_strategy="hip_block_rvq")
    assert [s["name"] for s in stats] == list(targets)
    for st in stats:
        assert set(st) == ENCODE_KEYS
        assert st["runtime_decision"] == "packed_block_rvq"
        assert 0.0 < st["rel_mse"] < 1.0  # a 2 x 64-entry residual code captures part of the weight
        assert st["codebook_size"] == 64 and st["num_stages"] == 2 and st["block_size"] == 8
    q = model.layers[0].self_attn.q_proj
    assert isinstance(q, PackedGroupedBlockRVQLinear) and q.bias is not None
    assert isinstance(model.layers[0].self_attn.k_proj, nn.Linear)  # not a target: untouched
    _check_layer(q, torch.bfloat16, gpu_device)
    _check_layer(model.layers[0].mlp.down_proj, torch.float16, gpu_device)
