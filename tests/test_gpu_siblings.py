"""fuse_sibling_linears on the GPU: q/k/v and gate/up of a decoder layer,
called one by one by unchanged model code, run as one launch per group.

* every output equals the linear's own forward bit for bit (M = 1, 4, 40;
  bf16 and fp16; with biases; prefill rows on the fused kernel unsplit), and
  the siblings after the first are served from that launch;
* an input changed in place, or another input, launches afresh (the stash is
  keyed on the tensor object and its version counter); inference-mode tensors
  (no version counter) work;
* groups that cannot share a launch (RECON beside FAST strategies) are left
  alone; unfuse_sibling_linears restores separate launches.
Reference call pattern: each linear's forward, src/runtime.py:1362-1507.
"""
from __future__ import annotations

import pytest
import torch
from torch import nn

from _cases import bits, make_encoding
from wal2026_amd import PackedGroupedBlockRVQLinear, fuse_sibling_linears, unfuse_sibling_linears

pytestmark = pytest.mark.gpu
HIDDEN, KV, INTER = 512, 128, 1024


def _lin(out_f, in_f, seed, bias=False, strategy="hip_block_rvq"):
    enc = make_encoding(out_f, in_f, S=2, K=256, seed=seed)
    b = (torch.randn(out_f, generator=torch.Generator().manual_seed(seed)) * 0.5).to(torch.bfloat16) if bias else None
    return PackedGroupedBlockRVQLinear(enc, bias=b, matmul_strategy=strategy)


class _Attn(nn.Module):
    def __init__(self, s, k_strategy="hip_block_rvq"):
        super().__init__()
        self.q_proj = _lin(HIDDEN, HIDDEN, s + 1, bias=True)
        self.k_proj = _lin(KV, HIDDEN, s + 2, strategy=k_strategy)
        self.v_proj = _lin(KV, HIDDEN, s + 3)
        self.o_proj = _lin(HIDDEN, HIDDEN, s + 4)


class _Mlp(nn.Module):
    def __init__(self, s):
        super().__init__()
        self.gate_proj = _lin(INTER, HIDDEN, s + 5)
        self.up_proj = _lin(INTER, HIDDEN, s + 6, bias=True)
        self.down_proj = _lin(HIDDEN, INTER, s + 7)


class _Layer(nn.Module):
    def __init__(self, s, k_strategy="hip_block_rvq"):
        super().__init__()
        self.self_attn = _Attn(s, k_strategy)
        self.mlp = _Mlp(s)

    def forward(self, x):
        a = self.self_attn
        q, k, v = a.q_proj(x), a.k_proj(x), a.v_proj(x)
        o = a.o_proj(q)
        g, u = self.mlp.gate_proj(x), self.mlp.up_proj(x)
        d = self.mlp.down_proj(g * u)
        return q, k, v, o, g, u, d


def _model(device, k_strategy="hip_block_rvq"):
    return nn.ModuleList([_Layer(10 * i, k_strategy) for i in range(2)]).to(device)


def _run(model, x):
    outs = []
    for layer in model:
        outs += list(layer(x))
    return outs


@pytest.mark.parametrize("m", [1, 4, 40])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_sibling_fusion_equals_separate_launches(m, dt, gpu_device, monkeypatch):
    # prefill rows (m = 40) on the fused kernel unsplit: the same per-row
    # arithmetic in the group's launch and in each linear's own (the two-pass
    # form's library GEMM, or a split chosen from the tile count, may sum in
    # another order)
    monkeypatch.setenv("WAL2026_PREFILL_TWO_PASS", "0")
    monkeypatch.setenv("WAL2026_PREFILL_KSPLIT", "1")
    model = _model(gpu_device)
    x = torch.randn(m, HIDDEN, generator=torch.Generator().manual_seed(m)).to(dt).to(gpu_device)
    ref = _run(model, x)
    names = fuse_sibling_linears(model)
    assert names == ["0.self_attn.{q_proj,k_proj,v_proj}", "0.mlp.{gate_proj,up_proj}",
                     "1.self_attn.{q_proj,k_proj,v_proj}", "1.mlp.{gate_proj,up_proj}"]
    # the first sibling's call launches for the group; the others are served from it
    att = model[0].self_attn
    att.q_proj(x)
    assert att.k_proj._sibling._pending == {1, 2}
    att.k_proj(x), att.v_proj(x)
    assert att.k_proj._sibling._pending == set() and att.k_proj._sibling._outs is None
    got = _run(model, x)
    for r, g in zip(ref, got):
        assert g.shape == r.shape and g.dtype == r.dtype
        assert torch.equal(bits(g), bits(r))
    assert unfuse_sibling_linears(model) == 10
    assert all(lin._sibling is None for lin in model.modules() if isinstance(lin, PackedGroupedBlockRVQLinear))


def test_sibling_fusion_relaunches_for_new_or_changed_input(gpu_device):
    model = _model(gpu_device)
    att = model[0].self_attn
    x = torch.randn(4, HIDDEN, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(gpu_device)
    x0 = x.clone()
    x2 = x.clone()
    x2.add_(0.5)
    k_ref, v_ref = att.k_proj(x2), att.v_proj(x0)
    fuse_sibling_linears(model)
    att.q_proj(x)
    x.add_(0.5)  # changed in place after the group's launch: k must see the new values
    assert torch.equal(bits(att.k_proj(x)), bits(k_ref))
    att.q_proj(x2)
    y = x0.clone()  # another tensor object than the group's launch read
    assert torch.equal(bits(att.v_proj(y)), bits(v_ref))
    with torch.inference_mode():
        xi = torch.randn(2, HIDDEN, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(gpu_device)
        outs = [att.q_proj(xi), att.k_proj(xi), att.v_proj(xi)]
    unfuse_sibling_linears(model)
    for lin, o in zip((att.q_proj, att.k_proj, att.v_proj), outs):
        assert torch.equal(bits(lin(xi)), bits(o))


def test_groups_that_cannot_share_a_launch_stay_separate(gpu_device):
    model = _model(gpu_device, k_strategy="per_group_fast")
    names = fuse_sibling_linears(model)
    assert names == ["0.mlp.{gate_proj,up_proj}", "1.mlp.{gate_proj,up_proj}"]
    assert model[0].self_attn.q_proj._sibling is None
