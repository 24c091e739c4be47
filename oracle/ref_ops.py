"""The reference's torch op sequences for this path, run by torch on the CPU.

TEST INFRASTRUCTURE ONLY.  The reference's arithmetic for the Block-RVQ linear
is a sequence of torch ops (gather, dtype casts, add, mul, F.linear).  These
functions issue the same ops in the same order on plain tensors, so that:

* the C oracle's own IEEE rounding can be checked bit-for-bit against torch's
  casts and bf16/fp16 arithmetic (tests/test_oracle.py), and
* ``bench.py`` can time the reference's CPU path (the ``cpu_baseline`` leg).

Inputs are the buffers of one group as CPU tensors:
``stage_ids`` (list of [R, B] integer tensors), ``codebooks`` (list of [K, d]),
``row_scale`` ([R, 1]), optional ``stage_scales`` ([S]) and ``block_scale``.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def reconstruct_weight(stage_ids, codebooks, row_scale, in_features, out_dtype,
                       stage_scales=None, block_scale=None):
    """src/runtime.py:379-414 for groups without residual correction/transform."""
    rows, bpr = stage_ids[0].shape
    d = codebooks[0].shape[1]
    acc = torch.zeros(rows * bpr, d, dtype=torch.float32)                 # :382
    scales = None if stage_scales is None else stage_scales.to(torch.float32)
    for s, (ids, cb) in enumerate(zip(stage_ids, codebooks)):
        part = cb[ids.reshape(-1).long()].to(torch.float32)               # :385
        if scales is not None:
            part = part * scales[s]                                       # :387
        acc += part                                                       # :388
    if block_scale is not None:
        acc = acc * block_scale.reshape(-1, 1).to(torch.float32)          # :399
    w = acc.view(rows, bpr * d)[:, :in_features]                          # :413
    return w.to(out_dtype) * row_scale.to(out_dtype)                      # :414


def active_stage_indices(stages_per_split, effective_stages_per_split):
    """src/runtime.py:352-372: first k stages of every split, split-major."""
    keep = max(1, int(effective_stages_per_split))
    out = []
    offset = 0
    for count in stages_per_split:
        out.extend(offset + j for j in range(min(keep, int(count))))
        offset += int(count)
    return out or [0]


def reconstruct_weight_fast(stage_ids, codebooks, row_scale, in_features, out_dtype,
                            active, stage_scales=None):
    """src/runtime.py:568-598 with the cache of :431-448 (plain groups)."""
    cache = []
    for s, cb in enumerate(codebooks):
        c = cb.to(out_dtype)                                              # :441
        if stage_scales is not None:
            c = c * stage_scales[s].to(out_dtype)                         # :443
        cache.append(c.contiguous())
    rows, bpr = stage_ids[0].shape
    d = codebooks[0].shape[1]
    first = active[0]
    recon = cache[first].index_select(0, stage_ids[first].reshape(-1).to(torch.int64))   # :590-591
    for s in active[1:]:
        recon.add_(cache[s].index_select(0, stage_ids[s].reshape(-1).to(torch.int64)))  # :592-594
    w = recon.view(rows, bpr * d)[:, :in_features]                                         # :596
    w.mul_(row_scale.to(out_dtype).contiguous())                                           # :597
    return w


def per_group_forward(x, groups, row_slices, out_features, bias=None):
    """src/runtime.py:1501-1507 (the default ``per_group`` strategy).

    ``groups`` is a list of dicts with keys stage_ids, codebooks, row_scale,
    in_features and optional stage_scales/block_scale; ``bias`` is the bf16
    buffer of src/runtime.py:1229-1230.
    """
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    parts = []
    for (r0, r1), g in zip(row_slices, groups):
        b = None if bias is None else bias[r0:r1].to(x2.dtype)
        w = reconstruct_weight(g["stage_ids"], g["codebooks"], g["row_scale"], g["in_features"],
                               x2.dtype, g.get("stage_scales"), g.get("block_scale"))
        parts.append(F.linear(x2, w, b))
    return torch.cat(parts, dim=-1).reshape(*lead, out_features)


def stagewise_block_matmul(x, stage_ids, codebooks, row_scale, in_features, stage_scales=None):
    """src/runtime.py:878-894: per stage an einsum in x dtype, summed in x dtype."""
    rows, bpr = stage_ids[0].shape
    d = codebooks[0].shape[1]
    pad = bpr * d - in_features
    xb = (F.pad(x, (0, pad), value=0.0) if pad else x).reshape(-1, bpr, d)   # :881-885
    out = torch.zeros((xb.shape[0], rows), dtype=xb.dtype)                  # :886
    ss = None if stage_scales is None else stage_scales.to(xb.dtype)        # :887
    for s, (ids, cb) in enumerate(zip(stage_ids, codebooks)):
        blocks = cb[ids.reshape(-1).long()].view(rows, bpr, d).to(xb.dtype)  # :889
        if ss is not None:
            blocks = blocks * ss[s]                                          # :891
        out = out + torch.einsum("mbd,rbd->mr", xb, blocks)                  # :892
    return out * row_scale.reshape(1, rows).to(out.dtype)                   # :894


def triton_rvq_matmul_weight(stage_ids, codebooks, x_dtype):
    """The per-block weight of src/triton_id_matmul.py:195-208: the fp32 sum of
    all stages, cast to x.dtype.  stage_ids [S, N, B], codebooks [S, K, d]."""
    S, N, B = stage_ids.shape
    d = codebooks.shape[2]
    acc = torch.zeros(N * B, d, dtype=torch.float32)
    for s in range(S):
        acc = acc + codebooks[s][stage_ids[s].reshape(-1).long()].to(torch.float32)
    return acc.view(N, B * d).to(x_dtype)


def id_route_weight(ids, codebook_sum, row_scale, *, mode, x_dtype):
    """mode 0: src/runtime.py:89-97 (product in the buffers' dtype, then cast);
    mode 1: src/triton_id_matmul.py:55-61 (cast each operand, product in x dtype)."""
    if mode == 0:
        w = codebook_sum[ids.long()] * row_scale
        return w.to(x_dtype)
    return codebook_sum[ids.long()].to(x_dtype) * row_scale.reshape(-1, 1).to(x_dtype)
