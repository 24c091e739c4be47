"""Runtime linear layers over compressed weights, executed by HIP kernels.

Drop-in for the reference's DRL runtime (src/runtime.py): the same classes,
constructor signatures, buffer names (so ``state_dict`` keys match), strategy
names and installers.  Every forward and every weight reconstruction runs in
libwal2026_amd.so (include/wal2026_amd.h); tensors must be on a ROCm GPU and
the library must be built -- there is no CPU or torch fallback.

Strategy mapping for ``PackedGroupedBlockRVQLinear`` (src/runtime.py:1362-1507):

* ``per_group``, ``full_weight``, ``chunked_weight``, ``stacked_matmul`` and
  the new ``hip_block_rvq``: the reference's reconstruct_weight arithmetic
  (src/runtime.py:379-414) followed by the contraction, in ONE launch for all
  row groups (decode kernel for M <= 16, prefill kernel above).  For a
  prefill call with an output in x's dtype, the torch operator runs the
  reference's own order of work instead -- the dense weight (bit-exact, one
  launch), then torch's GEMM -- wherever its cost model finds that faster on
  MI355X (narrow layers at every prefill M, wide ones at large M).
* ``per_group_fast``, ``full_weight_fast``: reconstruct_weight_fast arithmetic
  over the active stages (src/runtime.py:568-598).
* ``triton_block_rvq``: per group, the fused Triton kernel's arithmetic where
  the reference would run it (src/runtime.py:1476-1489), else reconstruct_weight.
* ``stagewise_einsum``: stagewise_block_matmul's per-stage rounding
  (src/runtime.py:878-894), one launch for all row groups.
* The experimental hot/cold / palette strategies are accepted by the
  constructor (same validation as the reference) but raise
  NotImplementedError in forward.
"""
from __future__ import annotations

import ctypes
import math

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import _lib
from .block_vq import BlockRVQEncoding, GroupedBlockRVQEncoding, encode_grouped_block_residual_vq

TARGET_LINEAR_SUFFIXES = (
    "self_attn.q_proj",
    "self_attn.k_proj",
    "self_attn.v_proj",
    "self_attn.o_proj",
    "mlp.gate_proj",
    "mlp.up_proj",
    "mlp.down_proj",
)

# The reference's whitelist (src/runtime.py:1192) plus the HIP strategy.
MATMUL_STRATEGIES = frozenset({
    "per_group", "per_group_fast", "full_weight", "full_weight_fast", "full_weight_hot", "full_weight_hot_v2",
    "chunked_weight", "local_palette", "triton_hot_cold_persistent", "stage_local_hot_cold",
    "stage_local_hot_cold_b1", "stage_local_hot_cold_b2", "stage_local_hot_cold_b3", "stagewise_einsum",
    "triton_block_rvq", "stacked_matmul", "hip_block_rvq",
})
_RECON_STRATEGIES = frozenset({"per_group", "full_weight", "chunked_weight", "stacked_matmul", "hip_block_rvq"})
_FAST_STRATEGIES = frozenset({"per_group_fast", "full_weight_fast"})
_HOT_STRATEGIES = ("full_weight_hot", "full_weight_hot_v2", "triton_hot_cold_persistent", "stage_local_hot_cold",
                   "stage_local_hot_cold_b1", "stage_local_hot_cold_b2", "stage_local_hot_cold_b3")


def rel_mse(w: Tensor, w_hat: Tensor, eps: float = 1e-12) -> Tensor:
    """mean((w - w_hat)^2) / mean(w^2) (src/route_encoder.py:82-85)."""
    return (w - w_hat).pow(2).mean() / w.pow(2).mean().clamp_min(eps)


# ---------------------------------------------------------------------------
# C-ABI descriptors
# ---------------------------------------------------------------------------

def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


class _LayerDesc:
    """ctypes wal_rvq_layer for a list of PackedBlockRVQGroup on one device,
    plus the device copy of its plan (kept alive here)."""

    def __init__(self, groups, row_slices, in_features: int, out_features: int, device: torch.device):
        g0 = groups[0]
        S = g0.num_stages
        ids0 = getattr(g0, "stage_ids_0")
        cb0 = getattr(g0, "codebook_0")
        for g in groups:
            if g.transform_kind != "none" or g.transform_matrix is not None or g.transform_bias is not None:
                raise NotImplementedError("wal2026_amd: transform encodings are not supported by the HIP runtime")
            if g.residual_correction != "none" or g.residual_signs is not None or g.residual_scale is not None:
                raise NotImplementedError("wal2026_amd: residual sign correction is not supported by the HIP runtime")
            if (g.num_stages != S or g.block_size != g0.block_size or g.in_features != in_features
                    or getattr(g, "stage_ids_0").shape[1] != ids0.shape[1]
                    or getattr(g, "codebook_0").shape[0] != cb0.shape[0]
                    or getattr(g, "stage_ids_0").dtype != ids0.dtype
                    or getattr(g, "codebook_0").dtype != cb0.dtype
                    or g.row_scale.dtype != g0.row_scale.dtype):
                raise NotImplementedError("wal2026_amd: row groups of one layer must share stage count, block size, "
                                          "codebook size and dtypes")
        arr = (_lib.WalGroup * len(groups))()
        all_ids = []
        for i, ((r0, r1), g) in enumerate(zip(row_slices, groups)):
            w = arr[i]
            for s in range(S):
                ids = getattr(g, f"stage_ids_{s}")
                cb = getattr(g, f"codebook_{s}")
                _lib.require_rocm(ids, cb)
                if not ids.is_contiguous() or not cb.is_contiguous():
                    raise ValueError("stage_ids/codebook buffers must be contiguous")
                if tuple(ids.shape) != (r1 - r0, ids0.shape[1]) or cb.shape[1] != g0.block_size:
                    raise ValueError(f"group {i} stage {s}: unexpected buffer shape")
                w.stage_ids[s] = ids.data_ptr()
                w.codebooks[s] = cb.data_ptr()
                all_ids.append(ids)
            rs = g.row_scale.reshape(-1)
            if rs.numel() != r1 - r0:
                raise ValueError(f"group {i}: row_scale has {rs.numel()} entries for {r1 - r0} rows")
            w.row_scale = rs.data_ptr()
            w.stage_scales = _ptr(g.stage_scales)
            w.block_scale = _ptr(g.block_scale)
            if g.block_scale is not None and g.block_scale.numel() != (r1 - r0) * ids0.shape[1]:
                raise ValueError(f"group {i}: block_scale shape mismatch")
            if g.stage_scales is not None and g.stage_scales.numel() != S:
                raise ValueError(f"group {i}: stage_scales has {g.stage_scales.numel()} entries for {S} stages")
            w.row0 = r0
            w.rows = r1 - r0
        K = int(cb0.shape[0])
        # ids must index the codebook: the reference's gather raises on a bad
        # index; here a bad index is refused before any launch (one host sync
        # when the descriptor is built, never per forward).
        lo, hi = _lib.id_range(*all_ids)
        if lo < 0 or hi >= K:
            raise IndexError(f"stage_ids hold index range [{lo}, {hi}] outside [0, codebook_size={K})")
        scale_dt = g0.row_scale.dtype
        for g in groups:
            for extra in (g.stage_scales, g.block_scale):
                if extra is not None and extra.dtype != scale_dt:
                    raise NotImplementedError("wal2026_amd: scale buffers of one layer must share a dtype")
        scale_rows, compact = _scale_runs(groups, row_slices)
        if compact is not None:
            for w, rs in zip(arr, compact):
                w.row_scale = rs.data_ptr()
        self.compact_scales = compact  # keeps the compact buffers alive
        L = _lib.WalLayer()
        L.in_features = in_features
        L.out_features = out_features
        L.block_size = g0.block_size
        L.blocks_per_row = int(ids0.shape[1])
        L.codebook_size = K
        L.num_stages = S
        L.id_dtype = _lib.id_tag(ids0.dtype)
        L.codebook_dtype = _lib.float_tag(cb0.dtype)
        L.scale_dtype = _lib.float_tag(scale_dt)
        L.scale_rows = scale_rows
        L.n_groups = len(groups)
        L.groups = ctypes.cast(arr, ctypes.POINTER(_lib.WalGroup))
        L.plan = None
        self.arr = arr
        self.layer = L
        self.plan = None
        if len(groups) > 1:
            lib = _lib.lib()
            size = ctypes.c_size_t(0)
            _lib.check(lib.wal_rvq_plan_size(ctypes.byref(L), ctypes.byref(size)))
            host = torch.empty(size.value, dtype=torch.uint8)
            _lib.check(lib.wal_rvq_plan_build(ctypes.byref(L), host.data_ptr(), size.value))
            self.plan = host.to(device)
            L.plan = self.plan.data_ptr()
        self.device = device
        self.key = _desc_key(groups)
        self.fused_ok = g0.block_size == 8 and S <= 4
        self._calls: dict[tuple[int, int], _lib.WalLayer] = {}
        self._images: dict[tuple[int, int], Tensor] = {}

    def layer_for(self, semantics: int, x_dtype: torch.dtype) -> "_lib.WalLayer":
        """The wal_rvq_layer for a linear call: the base descriptor plus the
        codebook image for this semantics and activation dtype, built on the
        device the first time (wal_rvq_image_build) and cached here, like the
        reference's derived codebook caches (src/runtime.py:431-448)."""
        xtag = _lib.FLOAT_DTYPES.get(x_dtype)
        key = (semantics, -1 if xtag is None else xtag)
        call = self._calls.get(key)
        if call is None:
            call = _lib.WalLayer.from_buffer_copy(self.layer)
            if self.fused_ok and x_dtype in (torch.float16, torch.bfloat16):
                lib = _lib.lib()
                size = ctypes.c_size_t(0)
                if lib.wal_rvq_image_size(ctypes.byref(self.layer), semantics, xtag, ctypes.byref(size)) == _lib.OK:
                    img = torch.empty(size.value, dtype=torch.uint8, device=self.device)
                    _lib.check(lib.wal_rvq_image_build(ctypes.byref(self.layer), semantics, xtag, img.data_ptr(),
                                                       size.value, _lib.stream_ptr(self.device)))
                    call.image = img.data_ptr()
                    call.image_tag = _lib.image_tag(semantics, xtag)
                    self._images[key] = img
            self._calls[key] = call
        return call


# Bumped whenever a group's active stages change, so that layers holding a
# cached call (with its stage mask) rebuild it.
_STAGE_EPOCH = [0]

_SCALE_RUNS = (128, 64, 32, 16)


def _scale_runs(groups, row_slices) -> tuple[int, list[Tensor] | None]:
    """Longest R in _SCALE_RUNS such that every row group's row_scale is
    constant (bit for bit) over aligned runs of R rows, with the compact
    per-run copies of the groups' scales; (1, None) when there is none.

    The reference keeps one scale per row (src/runtime.py:278); a layer whose
    rows share scales in aligned runs (per-128-row-group scales expanded to
    rows) gives the library the same values through a shorter buffer, and
    with runs of 16 or more rows the decode kernel can fold the scale into its
    staged codebook.  One host sync per candidate R, when the descriptor is
    built."""
    if groups[0].row_scale.dtype not in (torch.float16, torch.bfloat16):
        return 1, None
    bits = torch.cat([g.row_scale.reshape(-1).view(torch.int16) for g in groups])
    for R in _SCALE_RUNS:
        if any((r0 - row_slices[0][0]) % R for r0, _ in row_slices):
            continue
        comp = bits[::R]
        if not torch.equal(comp.repeat_interleave(R)[: bits.numel()], bits):
            continue
        base = row_slices[0][0]
        compact = []
        for (r0, r1), g in zip(row_slices, groups):
            lo, hi = (r0 - base) // R, -(-(r1 - base) // R)
            compact.append(comp[lo:hi].view(g.row_scale.dtype).contiguous())
        return R, compact
    return 1, None


_KERNEL_NAMES = {_lib.KERNEL_NONE: "none", _lib.KERNEL_DECODE: "decode", _lib.KERNEL_PREFILL: "prefill",
                 _lib.KERNEL_GENERIC: "generic"}
_TILE_NAMES = {_lib.TILE_SHORT: "short", _lib.TILE_TALL: "tall", _lib.TILE_WIDE: "wide"}


def _launch_info(layer: "_lib.WalLayer", semantics: int, x: Tensor) -> dict:
    """wal_rvq_linear_info for a call of ``layer`` on activations x (2-D view
    of ``x``; only its shape, dtype and alignment are read)."""
    x_flat = x.reshape(-1, x.shape[-1])
    info = _lib.WalLaunchInfo()
    _lib.check(_lib.lib().wal_rvq_linear_info(ctypes.byref(layer), semantics, x_flat.data_ptr(), x_flat.shape[0],
                                              _lib.float_tag(x_flat.dtype), ctypes.byref(info)))
    out = {"kernel": _KERNEL_NAMES[info.kernel]}
    if info.kernel == _lib.KERNEL_DECODE:
        out.update(x_mode=_lib.XMODE_NAMES[info.x_mode], table_slots=info.table_slots, grid=info.grid,
                   share=info.share, lds_bytes=info.lds_bytes)
    elif info.kernel == _lib.KERNEL_PREFILL:
        out.update(tile_shape=_TILE_NAMES[info.tile_shape], grid=info.grid, k_steps=info.share,
                   k_splits=info.k_splits)
        # the torch operator's choice for an output in x's dtype: the dense
        # weight (wal_rvq_reconstruct) then torch's GEMM, or the fused kernel
        out["two_pass"] = bool(_lib.ops().rvq_prefill_two_pass(ctypes.addressof(layer), semantics,
                                                               x_flat.shape[0], x_flat.dtype))
    return out


def _desc_key(groups) -> tuple:
    g0 = groups[0]
    return (g0.row_scale.data_ptr(), getattr(g0, "stage_ids_0").data_ptr(), len(groups),
            groups[-1].row_scale.data_ptr())


# ---------------------------------------------------------------------------
# Block-RVQ modules
# ---------------------------------------------------------------------------

class PackedBlockRVQGroup(nn.Module):
    """Buffers of one row group (src/runtime.py:248-290): ``stage_ids_{i}``
    (index dtype kept), ``codebook_{i}`` (fp16), ``row_scale`` ([R, 1] fp16),
    optional ``stage_scales``, ``block_scale``, ``residual_*`` and
    ``transform_*``."""

    def __init__(self, enc: BlockRVQEncoding) -> None:
        super().__init__()
        self.block_size = int(enc.block_size)
        self.in_features = int(enc.original_shape[1])
        self.out_features = int(enc.original_shape[0])
        self.padded_cols = int(enc.padded_cols)
        self.num_stages = len(enc.stage_ids)
        self.product_splits = int(enc.product_splits)
        self.stages_per_split = tuple(int(x) for x in enc.stages_per_split)
        self.transform_kind = enc.transform_kind
        for i, ids in enumerate(enc.stage_ids):
            self.register_buffer(f"stage_ids_{i}", ids.contiguous())
        for i, cb in enumerate(enc.codebooks):
            self.register_buffer(f"codebook_{i}", cb.contiguous().to(torch.float16))
        self._optional("stage_scales", enc.stage_scales, torch.float16)
        self.residual_correction = enc.residual_correction
        self._optional("residual_signs", enc.residual_signs, None)
        self._optional("residual_scale", enc.residual_scale, torch.float16)
        self.register_buffer("row_scale", enc.row_scale.to(torch.float16).contiguous())
        self._optional("block_scale", enc.block_scale, torch.float16)
        self._optional("transform_matrix", enc.transform_matrix, torch.float16)
        self._optional("transform_bias", enc.transform_bias, torch.float16)
        # Variable-stage decoding (src/runtime.py:339-344, :352-377).
        self.effective_stages_per_split: int = max(self.stages_per_split) if self.stages_per_split else self.num_stages
        self._active_stage_indices: tuple[int, ...] | None = None
        self._triton_stage_ids: Tensor | None = None
        self._triton_codebooks: Tensor | None = None
        self._triton_cache_device: torch.device | None = None
        self._desc: _LayerDesc | None = None

    def _optional(self, name: str, t: Tensor | None, dtype) -> None:
        if t is None:
            setattr(self, name, None)
        else:
            t = t.contiguous() if dtype is None else t.to(dtype).contiguous()
            self.register_buffer(name, t)

    def _apply(self, fn, recurse: bool = True):
        self._desc = None
        self._triton_stage_ids = self._triton_codebooks = None
        return super()._apply(fn, recurse)

    def invalidate_caches(self) -> None:
        """Drop the device descriptor, id-range check and codebook images
        (rebuilt on the next call).  Needed after changing buffers in place."""
        self._desc = None
        self._triton_stage_ids = self._triton_codebooks = None

    def _load_from_state_dict(self, *args, **kwargs):
        self.invalidate_caches()  # load_state_dict copies into the buffers in place
        return super()._load_from_state_dict(*args, **kwargs)

    def _stage_tensors(self) -> list[tuple[Tensor, Tensor]]:
        return [(getattr(self, f"stage_ids_{i}"), getattr(self, f"codebook_{i}")) for i in range(self.num_stages)]

    def _compute_active_stage_indices(self) -> tuple[int, ...]:
        """First ``effective_stages_per_split`` stages of every split, in the
        split-major stage order (src/runtime.py:352-372)."""
        if self._active_stage_indices is not None:
            return self._active_stage_indices
        keep = max(1, int(self.effective_stages_per_split))
        idx: list[int] = []
        offset = 0
        for count in self.stages_per_split:
            idx.extend(offset + j for j in range(min(keep, int(count))))
            offset += int(count)
        self._active_stage_indices = tuple(idx) if idx else (0,)
        return self._active_stage_indices

    def set_effective_stages_per_split(self, k: int) -> None:
        self.effective_stages_per_split = int(k)
        self._active_stage_indices = None
        _STAGE_EPOCH[0] += 1

    def active_stage_mask(self) -> int:
        mask = 0
        for s in self._compute_active_stage_indices():
            mask |= 1 << int(s)
        return mask

    def supports_fast_reconstruct(self) -> bool:
        """Plain RVQ group (src/runtime.py:416-429)."""
        return (self.block_scale is None and self.transform_kind == "none" and self.transform_matrix is None
                and self.transform_bias is None and self.residual_correction == "none"
                and self.residual_signs is None and self.residual_scale is None)

    supports_stagewise_block_matmul = supports_fast_reconstruct  # same predicate, src/runtime.py:837-846

    def supports_triton_block_matmul(self) -> bool:
        """Where the reference would run its fused kernel (src/runtime.py:848-853)."""
        if not self.supports_stagewise_block_matmul():
            return False
        if self.block_size != 32 or self.padded_cols != self.in_features:
            return False
        return all(getattr(self, f"stage_ids_{i}").dtype == torch.uint8 for i in range(self.num_stages))

    def _descriptor(self) -> _LayerDesc:
        dev = self.row_scale.device
        if self._desc is None or self._desc.device != dev or self._desc.key != _desc_key([self]):
            self._desc = _LayerDesc([self], [(0, self.out_features)], self.in_features, self.out_features, dev)
        return self._desc

    def _reconstruct(self, out_dtype: torch.dtype, semantics: int, mask: int) -> Tensor:
        dev = _lib.require_rocm(self.row_scale)
        desc = self._descriptor()
        out = torch.empty(self.out_features, self.in_features, dtype=out_dtype, device=dev)
        _lib.check(_lib.lib().wal_rvq_reconstruct(ctypes.byref(desc.layer), semantics, mask, out.data_ptr(),
                                                  _lib.float_tag(out_dtype), _lib.stream_ptr(dev)))
        return out

    def reconstruct_weight(self, out_dtype: torch.dtype) -> Tensor:
        """src/runtime.py:379-414, bit-exact, on the GPU."""
        return self._reconstruct(out_dtype, _lib.RECONSTRUCT, 0)

    def reconstruct_weight_fast(self, out_dtype: torch.dtype) -> Tensor:
        """src/runtime.py:568-598, bit-exact, on the GPU (non-plain groups use
        reconstruct_weight with all stages, as the reference does)."""
        if not self.supports_fast_reconstruct():
            return self.reconstruct_weight(out_dtype)
        return self._reconstruct(out_dtype, _lib.RECONSTRUCT_FAST, self.active_stage_mask())

    def _triton_state(self) -> tuple[Tensor, Tensor]:
        """Stacked ids [S, N, B] and codebooks [S, K, d] with stage scales
        folded in fp32 and rounded back to the codebook dtype
        (src/runtime.py:855-876)."""
        if not self.supports_triton_block_matmul():
            raise ValueError("triton block matmul only supports plain uint8, block_size=32 encodings")
        dev = self.row_scale.device
        if self._triton_stage_ids is None or self._triton_codebooks is None or self._triton_cache_device != dev:
            self._triton_stage_ids = torch.stack(
                [getattr(self, f"stage_ids_{i}").contiguous() for i in range(self.num_stages)]).contiguous()
            cbs = []
            for i in range(self.num_stages):
                cb = getattr(self, f"codebook_{i}").contiguous()
                if self.stage_scales is not None:
                    cb = (cb.to(torch.float32) * self.stage_scales[i].to(torch.float32)).to(cb.dtype)
                cbs.append(cb)
            self._triton_codebooks = torch.stack(cbs).contiguous()
            self._triton_cache_device = dev
        return self._triton_stage_ids, self._triton_codebooks

    def triton_block_matmul(self, x_flat: Tensor) -> Tensor:
        from .kernels import rvq_group_linear_matmul

        if not x_flat.is_cuda:
            raise ValueError("triton block matmul expects CUDA input")
        stage_ids, codebooks = self._triton_state()
        return rvq_group_linear_matmul(x_flat, stage_ids, codebooks, self.row_scale)

    def stagewise_block_matmul(self, x_flat: Tensor) -> Tensor:
        """src/runtime.py:878-894 on the GPU: per stage, the codewords in x
        dtype contracted and rounded to x dtype, summed in x dtype over all
        stages, times row_scale in x dtype."""
        if not self.supports_stagewise_block_matmul():
            raise ValueError("stagewise_block_matmul only supports unnormalized, transform-free encodings")
        return _stagewise_linear(self._descriptor(), x_flat, self.out_features, None)


def _stagewise_linear(desc: _LayerDesc, x_flat: Tensor, out_features: int, bias: Tensor | None,
                      out_dtype: torch.dtype | None = None) -> Tensor:
    """One STAGEWISE launch over every group of ``desc``; the bias (the
    module's bf16 buffer) is cast to x dtype and added to the rounded result
    (src/runtime.py:1466-1475)."""
    dev = _lib.require_rocm(x_flat)
    x_c = x_flat.contiguous()
    y = torch.empty(x_c.shape[0], out_features, dtype=out_dtype or x_flat.dtype, device=dev)
    if x_c.shape[0] == 0:
        return y
    btag = _lib.float_tag(bias.dtype) if bias is not None else _lib.F32
    _lib.check(_lib.lib().wal_rvq_linear(ctypes.byref(desc.layer), _lib.STAGEWISE, 0, x_c.data_ptr(), x_c.shape[0],
                                         _lib.float_tag(x_c.dtype), _ptr(bias), btag, y.data_ptr(),
                                         _lib.float_tag(y.dtype), _lib.stream_ptr(dev)))
    return y


class PackedGroupedBlockRVQLinear(nn.Module):
    """Linear layer over a GroupedBlockRVQEncoding (src/runtime.py:1175-1507)."""

    def __init__(
        self,
        enc: GroupedBlockRVQEncoding,
        bias: Tensor | None = None,
        *,
        matmul_strategy: str = "per_group",
        matmul_chunk_rows: int | None = None,
        local_palette_group_cols: int | None = None,
        hot_topk: int | None = None,
        hot_score_mode: str = "row_scale_norm",
        hot_min_stage_share: float = 0.0,
        hot_score_threshold_ratio: float = 0.0,
    ) -> None:
        super().__init__()
        # Constructor validation of src/runtime.py:1190-1211.
        if matmul_strategy == "triton_hot_cold_persistent" and local_palette_group_cols is None:
            local_palette_group_cols = 256
        if matmul_strategy not in MATMUL_STRATEGIES:
            raise ValueError(f"unsupported matmul_strategy: {matmul_strategy}")
        if matmul_strategy == "chunked_weight" and (matmul_chunk_rows is None or int(matmul_chunk_rows) <= 0):
            raise ValueError("chunked_weight requires a positive matmul_chunk_rows")
        if matmul_strategy in {"local_palette", "triton_hot_cold_persistent"} and (
                local_palette_group_cols is None or int(local_palette_group_cols) <= 0):
            raise ValueError(f"{matmul_strategy} requires a positive local_palette_group_cols")
        if matmul_strategy in _HOT_STRATEGIES and (hot_topk is None or int(hot_topk) <= 0):
            raise ValueError(f"{matmul_strategy} requires a positive hot_topk")
        self.in_features = int(enc.original_shape[1])
        self.out_features = int(enc.original_shape[0])
        self.groups = nn.ModuleList([PackedBlockRVQGroup(g) for g in enc.groups])
        self.row_slices = tuple(tuple(int(v) for v in s) for s in enc.row_slices)
        self.matmul_strategy = matmul_strategy
        self.matmul_chunk_rows = None if matmul_chunk_rows is None else int(matmul_chunk_rows)
        self.local_palette_group_cols = None if local_palette_group_cols is None else int(local_palette_group_cols)
        self.hot_topk = None if hot_topk is None else int(hot_topk)
        self.hot_score_mode = hot_score_mode
        self.hot_min_stage_share = float(hot_min_stage_share)
        self.hot_score_threshold_ratio = float(hot_score_threshold_ratio)
        if bias is not None:
            self.register_buffer("bias", bias.to(torch.bfloat16).contiguous())  # src/runtime.py:1229-1230
        else:
            self.bias = None
        self._desc: _LayerDesc | None = None
        # (device, x dtype, fast) -> (layer address, semantics, stage mask, stage epoch, layer struct)
        self._calls: dict = {}
        self._sibling: _SiblingFusion | None = None  # fuse_sibling_linears
        prev = 0
        for r0, r1 in self.row_slices:
            if r0 != prev or r1 <= r0:
                raise ValueError("row_slices must be contiguous and ascending")
            prev = r1
        if prev != self.out_features:
            raise ValueError("row_slices do not cover out_features")

    def _apply(self, fn, recurse: bool = True):
        self._desc = None
        self._calls = {}
        return super()._apply(fn, recurse)

    def invalidate_caches(self) -> None:
        """Drop the cached descriptors, calls and codebook images of the layer
        and its groups (rebuilt on the next call); needed after changing or
        replacing buffers other than through .to() / load_state_dict."""
        self._desc = None
        self._calls = {}
        for g in self.groups:
            g.invalidate_caches()

    def _load_from_state_dict(self, *args, **kwargs):
        self._desc = None  # the groups reset their own caches
        self._calls = {}
        return super()._load_from_state_dict(*args, **kwargs)

    def _call_for(self, x: Tensor, fast: bool):
        """The cached (layer address, semantics, stage mask) of a call on x's
        device and dtype, built on first use; None when the groups decode
        different stage subsets (one launch per group then)."""
        key = (x.device, x.dtype, fast)
        c = self._calls.get(key)
        if c is not None and c[3] == _STAGE_EPOCH[0]:
            return c
        _lib.require_rocm(x, self.groups[0].row_scale)
        sem = _lib.RECONSTRUCT_FAST if fast else _lib.RECONSTRUCT
        mask = self._uniform_mask() if fast else 0
        if mask is None:
            return None
        layer = self._descriptor().layer_for(sem, x.dtype)
        c = (ctypes.addressof(layer), sem, mask, _STAGE_EPOCH[0], layer)
        self._calls[key] = c
        return c

    def _descriptor(self) -> _LayerDesc:
        dev = self.groups[0].row_scale.device
        groups = list(self.groups)
        if self._desc is None or self._desc.device != dev or self._desc.key != _desc_key(groups):
            self._desc = _LayerDesc(groups, self.row_slices, self.in_features, self.out_features, dev)
        return self._desc

    def _uniform_mask(self) -> int | None:
        masks = {g.active_stage_mask() for g in self.groups}
        return masks.pop() if len(masks) == 1 else None

    # -- reconstruction ----------------------------------------------------
    def reconstruct_weight(self, out_dtype: torch.dtype = torch.bfloat16) -> Tensor:
        """Concatenated group weights (src/runtime.py:1234-1236), one launch."""
        dev = _lib.require_rocm(self.groups[0].row_scale)
        desc = self._descriptor()
        out = torch.empty(self.out_features, self.in_features, dtype=out_dtype, device=dev)
        _lib.check(_lib.lib().wal_rvq_reconstruct(ctypes.byref(desc.layer), _lib.RECONSTRUCT, 0, out.data_ptr(),
                                                  _lib.float_tag(out_dtype), _lib.stream_ptr(dev)))
        return out

    def reconstruct_weight_fast(self, out_dtype: torch.dtype = torch.bfloat16) -> Tensor:
        """src/runtime.py:1238-1240."""
        mask = self._uniform_mask()
        if mask is None or not all(g.supports_fast_reconstruct() for g in self.groups):
            return torch.cat([g.reconstruct_weight_fast(out_dtype) for g in self.groups], dim=0)
        dev = _lib.require_rocm(self.groups[0].row_scale)
        desc = self._descriptor()
        out = torch.empty(self.out_features, self.in_features, dtype=out_dtype, device=dev)
        _lib.check(_lib.lib().wal_rvq_reconstruct(ctypes.byref(desc.layer), _lib.RECONSTRUCT_FAST, mask,
                                                  out.data_ptr(), _lib.float_tag(out_dtype), _lib.stream_ptr(dev)))
        return out

    def launch_info(self, x: Tensor, fast: bool | None = None) -> dict:
        """Which kernel variant forward(x) launches (wal_rvq_linear_info):
        ``kernel`` ("decode", "prefill", "generic" or "none") and, for decode,
        ``x_mode`` / ``table_slots`` / ``grid`` / ``share`` / ``lds_bytes``,
        for prefill ``tile_shape``.  Nothing is launched."""
        if fast is None:
            fast = self.matmul_strategy in _FAST_STRATEGIES
        return _launch_info(self._descriptor().layer, _lib.RECONSTRUCT_FAST if fast else _lib.RECONSTRUCT, x)

    # -- forward -------------------------------------------------------------
    def _hip_linear(self, x: Tensor, fast: bool, out_dtype: torch.dtype | None = None) -> Tensor:
        """reconstruct_weight(_fast) arithmetic and the contraction, one
        launch for every row group, through the torch operator
        (torch.ops.wal2026_amd.rvq_linear); y has x's leading dims."""
        c = self._call_for(x, fast)
        if c is not None:
            return _lib.ops().rvq_linear(x, c[0], c[1], c[2], self.bias, out_dtype)
        # groups decode different stage subsets: one launch per group
        dev = x.device
        lead = x.shape[:-1]
        x_flat = x.reshape(-1, x.shape[-1])
        M = x_flat.shape[0]
        y = torch.empty(M, self.out_features, dtype=out_dtype or x.dtype, device=dev)
        sem = _lib.RECONSTRUCT_FAST
        for (r0, r1), g in zip(self.row_slices, self.groups):
            layer = g._descriptor().layer_for(sem, x.dtype)
            b = None if self.bias is None else self.bias[r0:r1]
            y[:, r0:r1] = _lib.ops().rvq_linear(x_flat, ctypes.addressof(layer), sem, g.active_stage_mask(), b,
                                                out_dtype)
        return y.reshape(*lead, self.out_features)

    def _stagewise(self, x_flat: Tensor, out_dtype: torch.dtype | None = None) -> Tensor:
        """Strategy stagewise_einsum (src/runtime.py:1466-1475): every group's
        stagewise_block_matmul plus its bias slice, in one launch."""
        for g in self.groups:
            if not g.supports_stagewise_block_matmul():
                raise ValueError("stagewise_block_matmul only supports unnormalized, transform-free encodings")
        return _stagewise_linear(self._descriptor(), x_flat, self.out_features, self.bias, out_dtype)

    def _triton_strategy(self, x_flat: Tensor) -> Tensor:
        """src/runtime.py:1476-1489: fused-kernel arithmetic on the groups the
        reference would run it on, reconstruct_weight + linear elsewhere; the
        bias is added to each rounded group output."""
        parts = []
        for (r0, r1), g in zip(self.row_slices, self.groups):
            if x_flat.is_cuda and g.supports_triton_block_matmul():
                part = g.triton_block_matmul(x_flat)
            else:
                part = _GroupView(g, self.in_features)._hip_linear(x_flat, fast=False)
            if self.bias is not None:
                part = part + self.bias[r0:r1].to(x_flat.dtype)
            parts.append(part)
        return torch.cat(parts, dim=-1)

    def forward(self, x: Tensor) -> Tensor:
        if self._sibling is not None:
            return self._sibling.output(self, x)
        s = self.matmul_strategy
        if s in _RECON_STRATEGIES:
            return self._hip_linear(x, fast=False)
        if s in _FAST_STRATEGIES:
            return self._hip_linear(x, fast=True)
        orig = x.shape
        x_flat = x.reshape(-1, orig[-1])
        if s == "triton_block_rvq":
            out = self._triton_strategy(x_flat)
        elif s == "stagewise_einsum":
            out = self._stagewise(x_flat)
        else:
            raise NotImplementedError(f"wal2026_amd: matmul_strategy={s!r} is one of the reference's experimental "
                                      "hot/cold or palette strategies, which this runtime does not implement; use "
                                      "'hip_block_rvq' (the reconstruct_weight arithmetic)")
        return out.reshape(*orig[:-1], self.out_features)


class FusedBlockRVQLinears(nn.Module):
    """Several PackedGroupedBlockRVQLinear layers that read the same input
    (q/k/v, gate/up of TARGET_LINEAR_SUFFIXES) run as ONE launch.

    Their row groups become one multi-group layer whose output rows are the
    linears' outputs side by side; ``forward(x)`` returns one output per
    linear (views of one [..., sum(out_features)] tensor), each equal to what
    that linear's own forward returns (the same arithmetic per row).  The
    reference has no counterpart: it calls each linear separately
    (src/runtime.py:1362); fusing saves the per-launch latency and codebook
    staging of the small linears.  The linears stay owned by the model; this
    module only holds references.
    """

    def __init__(self, linears) -> None:
        super().__init__()
        linears = list(linears)
        if not linears:
            raise ValueError("nothing to fuse")
        in_f = linears[0].in_features
        kinds = set()
        for lin in linears:
            if not isinstance(lin, PackedGroupedBlockRVQLinear):
                raise TypeError(f"cannot fuse {type(lin).__name__}")
            if lin.in_features != in_f:
                raise ValueError("fused linears must share in_features")
            kinds.add("fast" if lin.matmul_strategy in _FAST_STRATEGIES else
                      "recon" if lin.matmul_strategy in _RECON_STRATEGIES else lin.matmul_strategy)
        if len(kinds) != 1 or not kinds <= {"fast", "recon"}:
            raise ValueError(f"fused linears must all use reconstruct_weight or all reconstruct_weight_fast "
                             f"strategies (got {sorted(kinds)})")
        self._fast = kinds == {"fast"}
        self._linears = linears  # plain list: not submodules
        self.in_features = in_f
        self.out_features = [lin.out_features for lin in linears]
        self._desc: _LayerDesc | None = None
        self._bias: Tensor | None = None
        self._calls: dict = {}  # (device, x dtype) -> (layer address, semantics, mask, stage epoch, layer)

    def _groups_and_slices(self):
        groups, slices, base = [], [], 0
        for lin in self._linears:
            for (r0, r1), g in zip(lin.row_slices, lin.groups):
                groups.append(g)
                slices.append((base + r0, base + r1))
            base += lin.out_features
        return groups, slices, base

    def _descriptor(self) -> _LayerDesc:
        groups, slices, total = self._groups_and_slices()
        dev = groups[0].row_scale.device
        if self._desc is None or self._desc.device != dev or self._desc.key != _desc_key(groups):
            self._desc = _LayerDesc(groups, slices, self.in_features, total, dev)
            biases = [lin.bias for lin in self._linears]
            if any(b is not None for b in biases):
                self._bias = torch.cat([b if b is not None else torch.zeros(n, dtype=torch.bfloat16, device=dev)
                                        for b, n in zip(biases, self.out_features)]).contiguous()
            else:
                self._bias = None
        return self._desc

    def invalidate_caches(self) -> None:
        self._desc = None
        self._bias = None
        self._calls = {}

    def _call_for(self, x: Tensor):
        key = (x.device, x.dtype)
        c = self._calls.get(key)
        if c is not None and c[3] == _STAGE_EPOCH[0]:
            return c
        _lib.require_rocm(x, self._linears[0].groups[0].row_scale)
        desc = self._descriptor()
        sem = _lib.RECONSTRUCT_FAST if self._fast else _lib.RECONSTRUCT
        mask = 0
        if self._fast:
            masks = {g.active_stage_mask() for lin in self._linears for g in lin.groups}
            if len(masks) != 1:
                raise ValueError("fused reconstruct_weight_fast linears must decode the same stages")
            mask = masks.pop()
        layer = desc.layer_for(sem, x.dtype)
        c = (ctypes.addressof(layer), sem, mask, _STAGE_EPOCH[0], layer)
        self._calls[key] = c
        return c

    def launch_info(self, x: Tensor) -> dict:
        """Which kernel variant forward(x) launches (see
        PackedGroupedBlockRVQLinear.launch_info)."""
        return _launch_info(self._descriptor().layer, _lib.RECONSTRUCT_FAST if self._fast else _lib.RECONSTRUCT, x)

    def forward(self, x: Tensor) -> tuple[Tensor, ...]:
        c = self._call_for(x)
        y = _lib.ops().rvq_linear(x, c[0], c[1], c[2], self._bias, None)
        outs, o0 = [], 0
        for n in self.out_features:
            outs.append(y[..., o0:o0 + n])
            o0 += n
        return tuple(outs)


class _SiblingFusion:
    """The fused launch behind linears linked by fuse_sibling_linears.

    The first of them called on an input x runs ONE FusedBlockRVQLinears
    launch for all and returns its own output; the others, called next on the
    same tensor (same object, unchanged since: its version counter, and the
    same stage caps), return theirs from that launch instead of launching
    again.  A call on any other input launches afresh.  Each output is what
    the linear's own forward returns: bit for bit on the decode and unsplit
    fused prefill kernels (the same per-row arithmetic), to the last bits
    where the operator takes the two-pass form (the library GEMM of the
    concatenated weight may sum in another order).  For several rows of x
    they are column slices of one buffer, as torch.split returns them.
    """

    def __init__(self, linears) -> None:
        self.fused = FusedBlockRVQLinears(linears)
        self.ids = [id(lin) for lin in linears]
        self._x: Tensor | None = None
        self._key: tuple | None = None
        self._outs: tuple | None = None
        self._pending: set[int] = set()

    def output(self, lin: "PackedGroupedBlockRVQLinear", x: Tensor) -> Tensor:
        i = self.ids.index(id(lin))
        try:
            ver = x._version
        except RuntimeError:  # inference-mode tensors keep no version counter
            ver = None
        key = (ver, _STAGE_EPOCH[0])
        if self._outs is not None and x is self._x and key == self._key and i in self._pending:
            self._pending.discard(i)
            out = self._outs[i]
            if not self._pending:
                self._x = self._outs = None
            return out
        outs = self.fused(x)
        self._x, self._key, self._outs = x, key, outs
        self._pending = set(range(len(self.ids))) - {i}
        return outs[i]


# Linears that read the same input in the reference's decoder layers
# (TARGET_LINEAR_SUFFIXES, src/runtime.py:41-49).
SIBLING_GROUPS = (("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj"))


def fuse_sibling_linears(model: nn.Module, groups=SIBLING_GROUPS) -> list[str]:
    """Link the PackedGroupedBlockRVQLinear children of each module that
    holds a whole sibling group (q/k/v, gate/up) so that the model's unchanged
    forward runs each group as one launch (_SiblingFusion): the import swap
    then gets the fused launches without changes to the model code.  Groups
    whose linears cannot share a launch (different in_features, or RECON
    beside FAST strategies) are left alone.  Returns the linked groups'
    names.  No reference counterpart (the reference launches each linear,
    src/runtime.py:1362); unlink with unfuse_sibling_linears."""
    linked = []
    for name, parent in model.named_modules():
        for members in groups:
            lins = [getattr(parent, m, None) for m in members]
            if not all(isinstance(lin, PackedGroupedBlockRVQLinear) for lin in lins):
                continue
            try:
                fusion = _SiblingFusion(lins)
            except (TypeError, ValueError):
                continue
            for lin in lins:
                lin._sibling = fusion
            linked.append(f"{name}.{{{','.join(members)}}}" if name else "{" + ",".join(members) + "}")
    return linked


def unfuse_sibling_linears(model: nn.Module) -> int:
    """Undo fuse_sibling_linears; returns the number of linears unlinked."""
    n = 0
    for mod in model.modules():
        if isinstance(mod, PackedGroupedBlockRVQLinear) and mod._sibling is not None:
            mod._sibling = None
            n += 1
    return n


class _GroupView:
    """One group as a single-group layer without bias (for per-group calls)."""

    def __init__(self, group: PackedBlockRVQGroup, in_features: int):
        self.g = group
        self.in_features = in_features

    def _hip_linear(self, x_flat: Tensor, fast: bool) -> Tensor:
        g = self.g
        dev = _lib.require_rocm(x_flat, g.row_scale)
        x_c = x_flat.contiguous()
        if x_c.data_ptr() % 16:
            x_c = x_c.clone()
        y = torch.empty(x_c.shape[0], g.out_features, dtype=x_flat.dtype, device=dev)
        if x_c.shape[0] == 0:
            return y
        d = g._descriptor()
        _lib.check(_lib.lib().wal_rvq_linear(ctypes.byref(d.layer_for(_lib.RECONSTRUCT, x_c.dtype)), _lib.RECONSTRUCT,
                                             0, x_c.data_ptr(),
                                             x_c.shape[0], _lib.float_tag(x_c.dtype), None, _lib.F32, y.data_ptr(),
                                             _lib.float_tag(y.dtype), _lib.stream_ptr(dev)))
        return y


# ---------------------------------------------------------------------------
# Scalar route-codebook modules (d = 1)
# ---------------------------------------------------------------------------

class PackedIDRouteLinear(nn.Module):
    """Per-weight route id -> scalar codebook value x row scale
    (src/runtime.py:52-97).  Buffers: ``ids`` (int16 when the codebook has at
    most 32767 routes), ``codebook_sum`` (fp16), ``row_scale`` ([N, 1] fp16),
    ``bias`` (fp16)."""

    def __init__(self, ids: Tensor, codebook_w: Tensor, row_scale: Tensor, bias: Tensor | None = None) -> None:
        super().__init__()
        if codebook_w.shape[0] <= 32767 and ids.dtype != torch.int16:
            ids = ids.to(torch.int16)
        self.register_buffer("ids", ids.contiguous())
        self.register_buffer("codebook_sum", codebook_w.sum(dim=-1).contiguous().to(torch.float16))
        self.register_buffer("row_scale", row_scale.to(torch.float16).contiguous())
        if bias is not None:
            self.register_buffer("bias", bias.to(torch.float16).contiguous())
        else:
            self.bias = None
        self.out_features = ids.shape[0]
        self.in_features = ids.shape[1]

    @classmethod
    def from_encoded(cls, ids: Tensor, codebook_digits: Tensor, ladder: Tensor, row_scale: Tensor,
                     bias: Tensor | None = None, **_: object) -> "PackedIDRouteLinear":
        """src/runtime.py:77-87: signed per-route scales folded into fp16."""
        codebook_w = (codebook_digits.to(torch.float32) * ladder.to(torch.float32)).to(torch.float16)
        return cls(ids, codebook_w, row_scale.to(torch.float16), bias)

    def _check_route_buffers(self) -> torch.device:
        dev = _lib.require_rocm(self.ids, self.codebook_sum, self.row_scale)
        if self.codebook_sum.dtype != self.row_scale.dtype:
            raise NotImplementedError("wal2026_amd: codebook_sum and row_scale must share a dtype")
        return dev

    def _reconstruct(self, mode: int, out_dtype: torch.dtype) -> Tensor:
        dev = self._check_route_buffers()
        out = torch.empty(self.out_features, self.in_features, dtype=out_dtype, device=dev)
        _lib.check(_lib.lib().wal_id_route_reconstruct(
            self.ids.data_ptr(), _lib.id_tag(self.ids.dtype), self.out_features, self.in_features,
            self.codebook_sum.data_ptr(), self.codebook_sum.numel(), _lib.float_tag(self.codebook_sum.dtype),
            self.row_scale.data_ptr(), mode, _lib.float_tag(out_dtype), out.data_ptr(), _lib.stream_ptr(dev)))
        return out

    def reconstruct_weight(self) -> Tensor:
        """codebook_sum[ids] * row_scale in the buffers' dtype (src/runtime.py:89-93)."""
        return self._reconstruct(0, self.codebook_sum.dtype)

    def _route_linear(self, x: Tensor, mode: int) -> Tensor:
        dev = self._check_route_buffers()
        _lib.require_rocm(x)
        orig = x.shape
        x2 = x.reshape(-1, orig[-1]).contiguous()
        if x2.shape[1] != self.in_features:
            raise ValueError(f"Feature mismatch: {x2.shape[1]} != {self.in_features}")
        y = torch.empty(x2.shape[0], self.out_features, dtype=x.dtype, device=dev)
        if x2.shape[0]:
            b = self.bias
            _lib.check(_lib.lib().wal_id_route_linear(
                x2.data_ptr(), x2.shape[0], self.in_features, _lib.float_tag(x2.dtype), self.ids.data_ptr(),
                _lib.id_tag(self.ids.dtype), self.out_features, self.codebook_sum.data_ptr(),
                self.codebook_sum.numel(), _lib.float_tag(self.codebook_sum.dtype), self.row_scale.data_ptr(),
                _ptr(b), _lib.float_tag(b.dtype) if b is not None else _lib.F32, mode, y.data_ptr(),
                _lib.float_tag(y.dtype), _lib.stream_ptr(dev)))
        return y.reshape(*orig[:-1], self.out_features)

    def forward(self, x: Tensor) -> Tensor:
        """F.linear(x, W.to(x.dtype), bias.to(x.dtype)) (src/runtime.py:95-97)."""
        return self._route_linear(x, 0)


class FusedIDRouteLinear(PackedIDRouteLinear):
    """id_route_linear_matmul arithmetic, bias added after (src/runtime.py:100-105)."""

    def forward(self, x: Tensor) -> Tensor:
        return self._route_linear(x, 1)


class CachedPackedIDRouteLinear(PackedIDRouteLinear):
    """Materialises the dense weight once per (device, dtype) while it fits
    ``max_cache_bytes`` and then runs a library GEMM (src/runtime.py:108-167)."""

    def __init__(self, ids: Tensor, codebook_w: Tensor, row_scale: Tensor, bias: Tensor | None = None, *,
                 max_cache_bytes: int = 128 * 2**20) -> None:
        super().__init__(ids, codebook_w, row_scale, bias)
        self.max_cache_bytes = max(int(max_cache_bytes), 0)
        self._cached_weight: Tensor | None = None
        self._cached_weight_device: torch.device | None = None
        self._cached_weight_dtype: torch.dtype | None = None
        self.cache_hit_count = 0
        self.cache_miss_count = 0
        self.cache_skip_count = 0

    @classmethod
    def from_encoded(cls, ids: Tensor, codebook_digits: Tensor, ladder: Tensor, row_scale: Tensor,
                     bias: Tensor | None = None, *, max_cache_bytes: int = 128 * 2**20,
                     **_: object) -> "CachedPackedIDRouteLinear":
        codebook_w = (codebook_digits.to(torch.float32) * ladder.to(torch.float32)).to(torch.float16)
        return cls(ids, codebook_w, row_scale.to(torch.float16), bias, max_cache_bytes=max_cache_bytes)

    def clear_cache(self) -> None:
        self._cached_weight = None
        self._cached_weight_device = None
        self._cached_weight_dtype = None

    def _weight_for(self, x: Tensor) -> Tensor:
        weight_bytes = self.out_features * self.in_features * x.element_size()
        if self.max_cache_bytes > 0 and weight_bytes > self.max_cache_bytes:
            self.cache_skip_count += 1
            return self._reconstruct(0, x.dtype)
        if (self._cached_weight is None or self._cached_weight_device != x.device
                or self._cached_weight_dtype != x.dtype):
            self._cached_weight = self._reconstruct(0, x.dtype)
            self._cached_weight_device = x.device
            self._cached_weight_dtype = x.dtype
            self.cache_miss_count += 1
        else:
            self.cache_hit_count += 1
        return self._cached_weight

    def forward(self, x: Tensor) -> Tensor:
        _lib.require_rocm(x)
        weight = self._weight_for(x)
        return F.linear(x, weight, self.bias.to(x.dtype) if self.bias is not None else None)


class AdaptiveFusedIDRouteLinear(PackedIDRouteLinear):
    """Fused primary path guarded by the reference's validation contract
    (src/runtime.py:1595-1679): a RuntimeError from the primary, or a
    non-finite output during the first ``validate_calls`` calls, or (with
    ``shadow_validate``) a rel-MSE above ``shadow_rel_mse_tol`` against the
    packed path, switches to the packed path (both run on the GPU)."""

    def __init__(self, ids: Tensor, codebook_w: Tensor, row_scale: Tensor, bias: Tensor | None = None, *,
                 validate_calls: int = 1, disable_primary_after_nonfinite: bool = True,
                 shadow_validate: bool = False, shadow_rel_mse_tol: float = 1e-4) -> None:
        super().__init__(ids, codebook_w, row_scale, bias)
        self.validate_calls = max(int(validate_calls), 0)
        self.disable_primary_after_nonfinite = disable_primary_after_nonfinite
        self.shadow_validate = shadow_validate
        self.shadow_rel_mse_tol = float(shadow_rel_mse_tol)
        self._validation_calls_left = self.validate_calls
        self._primary_enabled = True
        self.fallback_count = 0
        self.shadow_mismatch_count = 0
        self.last_validation_rel_mse: float | None = None

    @classmethod
    def from_encoded(cls, ids: Tensor, codebook_digits: Tensor, ladder: Tensor, row_scale: Tensor,
                     bias: Tensor | None = None, *, validate_calls: int = 1,
                     disable_primary_after_nonfinite: bool = True, shadow_validate: bool = False,
                     shadow_rel_mse_tol: float = 1e-4, **_: object) -> "AdaptiveFusedIDRouteLinear":
        codebook_w = (codebook_digits.to(torch.float32) * ladder.to(torch.float32)).to(torch.float16)
        return cls(ids, codebook_w, row_scale.to(torch.float16), bias, validate_calls=validate_calls,
                   disable_primary_after_nonfinite=disable_primary_after_nonfinite,
                   shadow_validate=shadow_validate, shadow_rel_mse_tol=shadow_rel_mse_tol)

    def _primary_forward(self, x: Tensor) -> Tensor:
        return self._route_linear(x, 1)

    def forward(self, x: Tensor) -> Tensor:
        if not self._primary_enabled:
            return super().forward(x)
        try:
            out = self._primary_forward(x)
        except RuntimeError:
            self.fallback_count += 1
            if self.disable_primary_after_nonfinite:
                self._primary_enabled = False
            return super().forward(x)
        if self._validation_calls_left > 0:
            self._validation_calls_left -= 1
            if not bool(torch.isfinite(out).all().item()):
                self.fallback_count += 1
                if self.disable_primary_after_nonfinite:
                    self._primary_enabled = False
                return super().forward(x)
            if self.shadow_validate:
                reference = super().forward(x)
                denom = reference.float().square().mean().clamp_min(1e-12)
                value = float(((out.float() - reference.float()).square().mean() / denom).item())
                self.last_validation_rel_mse = value
                if value > self.shadow_rel_mse_tol:
                    self.shadow_mismatch_count += 1
                    if self.disable_primary_after_nonfinite:
                        self._primary_enabled = False
                    return reference
        return out


# ---------------------------------------------------------------------------
# Installers and stage controls
# ---------------------------------------------------------------------------

def _set_submodule(root: nn.Module, path: str, module: nn.Module) -> None:
    """Replace the submodule at dotted ``path`` (src/runtime.py:1716-1721)."""
    parent = root
    parts = path.split(".")
    for part in parts[:-1]:
        parent = getattr(parent, part)
    setattr(parent, parts[-1], module)


def _drop_dense(module: nn.Module) -> None:
    try:
        if hasattr(module, "_parameters"):
            module._parameters["weight"] = None
            module._parameters["bias"] = None
    except (AttributeError, TypeError, KeyError):
        pass


def _strategy_stats(matmul_strategy, matmul_chunk_rows, local_palette_group_cols, hot_topk, hot_score_mode,
                    hot_min_stage_share, hot_score_threshold_ratio) -> dict:
    return {
        "matmul_strategy": matmul_strategy,
        "matmul_chunk_rows": int(matmul_chunk_rows) if matmul_chunk_rows is not None else None,
        "local_palette_group_cols": int(local_palette_group_cols) if local_palette_group_cols is not None else None,
        "hot_topk": int(hot_topk) if hot_topk is not None else None,
        "hot_score_mode": hot_score_mode,
        "hot_min_stage_share": float(hot_min_stage_share),
        "hot_score_threshold_ratio": float(hot_score_threshold_ratio),
    }


@torch.no_grad()
def replace_with_packed_block_rvq(
    model: nn.Module,
    target_module_names: tuple[str, ...],
    *,
    group_rows: int = 2048,
    block_size: int = 32,
    codebook_size: int = 256,
    num_stages: int = 4,
    product_splits: int = 1,
    normalize_blocks: str = "none",
    transform_kind: str = "none",
    calibrate_stage_scales: bool = False,
    residual_correction: str = "none",
    sample_limit: int = 65_536,
    kmeans_iters: int = 8,
    batch_size: int = 16_384,
    matmul_strategy: str = "per_group",
    matmul_chunk_rows: int | None = None,
    local_palette_group_cols: int | None = None,
    hot_topk: int | None = None,
    hot_score_mode: str = "row_scale_norm",
    hot_min_stage_share: float = 0.0,
    hot_score_threshold_ratio: float = 0.0,
) -> list[dict[str, float]]:
    """Encode and swap the named nn.Linear modules (src/runtime.py:2052-2143);
    returns the same per-layer stat dicts."""
    targets = set(target_module_names)
    stats = []
    for name, module in list(model.named_modules()):
        if name not in targets or not isinstance(module, nn.Linear):
            continue
        w = module.weight.detach()
        enc = encode_grouped_block_residual_vq(
            w, group_rows=group_rows, block_size=block_size, codebook_size=codebook_size, num_stages=num_stages,
            product_splits=product_splits, normalize_blocks=normalize_blocks, transform_kind=transform_kind,
            calibrate_stage_scales=calibrate_stage_scales, residual_correction=residual_correction,
            sample_limit=sample_limit, kmeans_iters=kmeans_iters, batch_size=batch_size)
        packed = PackedGroupedBlockRVQLinear(
            enc, module.bias, matmul_strategy=matmul_strategy, matmul_chunk_rows=matmul_chunk_rows,
            local_palette_group_cols=local_palette_group_cols, hot_topk=hot_topk, hot_score_mode=hot_score_mode,
            hot_min_stage_share=hot_min_stage_share, hot_score_threshold_ratio=hot_score_threshold_ratio,
        ).to(w.device)
        approx = packed.reconstruct_weight(out_dtype=torch.bfloat16) if w.is_cuda else enc.reconstruct(torch.bfloat16)
        _set_submodule(model, name, packed)
        _drop_dense(module)
        stats.append({
            "name": name,
            "tensor_name": f"{name}.weight",
            "runtime_decision": "packed_block_rvq",
            **_strategy_stats(matmul_strategy, matmul_chunk_rows, local_palette_group_cols, hot_topk,
                              hot_score_mode, hot_min_stage_share, hot_score_threshold_ratio),
            "rel_mse": float(rel_mse(w.float(), approx.to(w.device).float()).item()),
            "storage_bytes": int(enc.storage_bytes()),
            "bits_per_weight": float(enc.bits_per_weight()),
            "group_rows": int(group_rows),
            "block_size": int(block_size),
            "codebook_size": int(codebook_size),
            "num_stages": int(num_stages),
            "product_splits": int(product_splits),
            "normalize_blocks": normalize_blocks,
            "transform_kind": transform_kind,
            "calibrate_stage_scales": bool(calibrate_stage_scales),
            "residual_correction": residual_correction,
        })
    return stats


@torch.no_grad()
def replace_with_preencoded_packed_block_rvq(
    model: nn.Module,
    encodings_by_name: dict[str, GroupedBlockRVQEncoding],
    *,
    matmul_strategy: str = "per_group",
    matmul_chunk_rows: int | None = None,
    local_palette_group_cols: int | None = None,
    hot_topk: int | None = None,
    hot_score_mode: str = "row_scale_norm",
    hot_min_stage_share: float = 0.0,
    hot_score_threshold_ratio: float = 0.0,
) -> list[dict[str, float]]:
    """Swap named nn.Linear modules for packed layers built from existing
    encodings (src/runtime.py:2146-2200)."""
    stats = []
    for name, module in list(model.named_modules()):
        if name not in encodings_by_name or not isinstance(module, nn.Linear):
            continue
        w = module.weight.detach()
        enc = encodings_by_name[name]
        packed = PackedGroupedBlockRVQLinear(
            enc, module.bias, matmul_strategy=matmul_strategy, matmul_chunk_rows=matmul_chunk_rows,
            local_palette_group_cols=local_palette_group_cols, hot_topk=hot_topk, hot_score_mode=hot_score_mode,
            hot_min_stage_share=hot_min_stage_share, hot_score_threshold_ratio=hot_score_threshold_ratio,
        ).to(w.device)
        approx = packed.reconstruct_weight(out_dtype=torch.bfloat16) if w.is_cuda else enc.reconstruct(torch.bfloat16)
        _set_submodule(model, name, packed)
        _drop_dense(module)
        stats.append({
            "name": name,
            "tensor_name": f"{name}.weight",
            "runtime_decision": "preencoded_packed_block_rvq",
            **_strategy_stats(matmul_strategy, matmul_chunk_rows, local_palette_group_cols, hot_topk,
                              hot_score_mode, hot_min_stage_share, hot_score_threshold_ratio),
            "rel_mse": float(rel_mse(w.float(), approx.to(w.device).float()).item()),
            "storage_bytes": int(enc.storage_bytes()),
            "bits_per_weight": float(enc.bits_per_weight()),
        })
    return stats


def set_global_effective_stages(model: nn.Module, stages: int) -> int:
    """Keep the first ``stages`` stages of every split in every group
    (src/runtime.py:2274-2286); returns the number of groups updated."""
    n = 0
    for m in model.modules():
        if isinstance(m, PackedBlockRVQGroup):
            m.set_effective_stages_per_split(int(stages))
            n += 1
    return n


def set_effective_stages_by_name(model: nn.Module, attn_stages: int | None, mlp_stages: int | None) -> dict[str, int]:
    """Per-role stage cap: ``.self_attn.`` layers get ``attn_stages``, ``.mlp.``
    layers ``mlp_stages`` (src/runtime.py:2289-2308)."""
    counts = {"attn": 0, "mlp": 0, "other": 0}
    for name, m in model.named_modules():
        if not isinstance(m, PackedGroupedBlockRVQLinear):
            continue
        bucket = "attn" if ".self_attn." in name else ("mlp" if ".mlp." in name else "other")
        target = attn_stages if bucket == "attn" else (mlp_stages if bucket == "mlp" else None)
        if target is None:
            continue
        for sub in m.modules():
            if isinstance(sub, PackedBlockRVQGroup):
                sub.set_effective_stages_per_split(int(target))
        counts[bucket] += 1
    return counts


def set_effective_stages_from_map(model: nn.Module, name_to_k: dict[str, int]) -> int:
    """Per-layer stage cap from {layer_name: k} (src/runtime.py:2311-2327)."""
    updated = 0
    for name, m in model.named_modules():
        if not isinstance(m, PackedGroupedBlockRVQLinear) or name not in name_to_k:
            continue
        for sub in m.modules():
            if isinstance(sub, PackedBlockRVQGroup):
                sub.set_effective_stages_per_split(int(name_to_k[name]))
        updated += 1
    return updated
