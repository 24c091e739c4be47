"""Block-RVQ data contract and offline encoder.

The dataclasses keep the reference's field names and order
(src/block_vq.py:230-338) so encodings built by either side are
interchangeable; ``encoding_io`` persists them in the reference's v1 map
format.  ``reconstruct`` runs the HIP dequantisation kernel
(``wal_rvq_reconstruct``); tensors on the CPU are staged through the GPU and
the result is returned on the caller's device.

The encoder (``encode_block_residual_vq`` / ``encode_grouped_block_residual_vq``)
is offline tooling that produces the index planes; it is not part of the
HIP hot path and runs with torch ops on the weight's device.  Its k-means is
seeded like the reference's (torch.Generator(0), src/block_vq.py:210-213,
:406-410) but its outputs are not pinned to the reference's bit for bit
(they depend on torch RNG streams and reduction order).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch import Tensor

__all__ = [
    "BlockRVQEncoding",
    "GroupedBlockRVQEncoding",
    "encode_block_residual_vq",
    "encode_grouped_block_residual_vq",
    "ideal_id_bits_per_weight",
    "storage_megabytes",
    "dense_bf16_storage_bytes",
]


def _id_storage_bytes(codebook_size: int) -> int:
    """Bytes per stored index for a codebook of this size (src/block_vq.py:150-157)."""
    if codebook_size <= 0:
        raise ValueError("codebook_size must be positive")
    if codebook_size <= 256:
        return 1
    if codebook_size <= 65_536:
        return 2
    return 4


def _id_storage_dtype(codebook_size: int) -> torch.dtype:
    """Index-plane dtype (src/block_vq.py:160-165): uint8 up to 256 entries,
    int16 up to 32767, int32 beyond."""
    if codebook_size <= 256:
        return torch.uint8
    if codebook_size <= 32_767:
        return torch.int16
    return torch.int32


def _reshape_blocks(w_norm: Tensor, block_size: int) -> tuple[Tensor, int, int]:
    """Zero-pad columns to a multiple of block_size and view as [rows * B, d]
    (src/block_vq.py:168-177)."""
    if w_norm.ndim != 2:
        raise ValueError("expected 2D weight matrix")
    if block_size < 1:
        raise ValueError("block_size must be >= 1")
    rows, cols = w_norm.shape
    padded = -(-cols // block_size) * block_size
    if padded != cols:
        w_norm = torch.nn.functional.pad(w_norm, (0, padded - cols))
    return w_norm.reshape(rows * (padded // block_size), block_size), rows, padded


@dataclass
class BlockRVQEncoding:
    """One row group's Block-RVQ encoding (src/block_vq.py:230-313)."""

    stage_ids: tuple[Tensor, ...]
    codebooks: tuple[Tensor, ...]
    stage_value_dims: tuple[int, ...]
    stages_per_split: tuple[int, ...]
    stage_scales: Tensor | None
    residual_correction: str
    residual_signs: Tensor | None
    residual_scale: Tensor | None
    row_scale: Tensor
    block_scale: Tensor | None
    transform_kind: str
    transform_matrix: Tensor | None
    transform_bias: Tensor | None
    product_splits: int
    original_shape: tuple[int, int]
    padded_cols: int
    block_size: int
    sample_rel_mse: float

    @property
    def num_stages(self) -> int:
        return len(self.codebooks)

    @property
    def stage_shape(self) -> tuple[int, int]:
        return tuple(int(x) for x in self.stage_ids[0].shape)

    def reconstruct(self, out_dtype: torch.dtype | None = None) -> Tensor:
        """Dense weight, bit-identical to src/block_vq.py:259-289, computed by
        the HIP dequantisation kernel."""
        return GroupedBlockRVQEncoding(
            groups=(self,), row_slices=((0, self.original_shape[0]),), original_shape=self.original_shape
        ).reconstruct(out_dtype)

    def storage_bytes(self) -> int:
        """Compressed bytes (src/block_vq.py:291-309): indices at their ideal
        width, 2 bytes per codebook value and per row scale, plus the optional
        buffers at their element size."""
        total = 0
        for ids, cb, value_dim in zip(self.stage_ids, self.codebooks, self.stage_value_dims):
            total += ids.numel() * _id_storage_bytes(int(cb.shape[0]))
            total += int(cb.shape[0]) * int(value_dim) * 2
        for extra in (self.stage_scales, self.residual_signs, self.residual_scale, self.block_scale,
                      self.transform_matrix, self.transform_bias):
            if extra is not None:
                total += extra.numel() * extra.element_size()
        return total + self.row_scale.numel() * 2

    def bits_per_weight(self) -> float:
        rows, cols = self.original_shape
        return 8.0 * self.storage_bytes() / max(rows * cols, 1)


@dataclass
class GroupedBlockRVQEncoding:
    """Row-sliced groups, each with its own codebooks (src/block_vq.py:316-338)."""

    groups: tuple[BlockRVQEncoding, ...]
    row_slices: tuple[tuple[int, int], ...]
    original_shape: tuple[int, int]

    @property
    def sample_rel_mse(self) -> float:
        rows = float(sum(g.original_shape[0] for g in self.groups))
        if rows <= 0.0:
            return 0.0
        return float(sum(g.sample_rel_mse * g.original_shape[0] for g in self.groups) / rows)

    def reconstruct(self, out_dtype: torch.dtype | None = None) -> Tensor:
        """Groups' dense weights concatenated on rows (src/block_vq.py:329-331),
        computed by the HIP dequantisation kernel."""
        from .runtime import PackedGroupedBlockRVQLinear

        out_dtype = out_dtype or torch.float32
        home = self.groups[0].row_scale.device
        dev = home if home.type == "cuda" else _default_rocm_device()
        layer = PackedGroupedBlockRVQLinear(self).to(dev)
        w = layer.reconstruct_weight(out_dtype=out_dtype)
        return w.to(home)

    def storage_bytes(self) -> int:
        return sum(g.storage_bytes() for g in self.groups)

    def bits_per_weight(self) -> float:
        rows, cols = self.original_shape
        return 8.0 * self.storage_bytes() / max(rows * cols, 1)


def _default_rocm_device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("wal2026_amd: reconstruct needs a ROCm GPU (the HIP kernel is the only implementation)")
    return torch.device("cuda", torch.cuda.current_device())


# ---------------------------------------------------------------------------
# Offline encoder (k-means residual VQ).  Off the hot path.
# ---------------------------------------------------------------------------

def _nearest(blocks: Tensor, codebook: Tensor, batch_size: int) -> tuple[Tensor, Tensor]:
    """Index and squared distance of the nearest codeword for every block."""
    cb = codebook.to(device=blocks.device, dtype=torch.float32)
    cb_sq = (cb * cb).sum(1)
    ids = torch.empty(blocks.shape[0], dtype=torch.int64, device=blocks.device)
    dist = torch.empty(blocks.shape[0], dtype=torch.float32, device=blocks.device)
    for lo in range(0, blocks.shape[0], batch_size):
        chunk = blocks[lo:lo + batch_size].to(torch.float32)
        d = (chunk * chunk).sum(1, keepdim=True) + cb_sq[None, :] - 2.0 * (chunk @ cb.t())
        dist[lo:lo + batch_size], ids[lo:lo + batch_size] = d.min(1)
    return ids, dist


def _assign_to_codebook(blocks: Tensor, codebook: Tensor, batch_size: int = 16_384) -> tuple[Tensor, Tensor]:
    """Nearest codeword of every block: ``(ids int64, min_dist float32)``.

    Drop-in for the reference's ``_assign_to_codebook`` (src/block_vq.py:180-196),
    computed by one HIP kernel (``wal_rvq_assign``) on the blocks' ROCm device:
    ``dist = (|b|^2 + |c|^2) - 2 b.c`` in fp32, the sums and the dot product
    accumulated with fused multiply-adds in element order, the first minimal
    codeword on ties.  ``batch_size`` only bounded the reference's temporaries
    and is accepted and ignored.  Block sizes 1, 2, 4, 8, 16 and 32; finite
    inputs.  CPU tensors raise (the kernel is the only implementation).
    """
    del batch_size
    if blocks.numel() == 0:
        raise ValueError("blocks must be non-empty")
    if blocks.ndim != 2 or codebook.ndim != 2 or blocks.shape[1] != codebook.shape[1]:
        raise ValueError(f"expected blocks [n, d] and codebook [k, d], got {tuple(blocks.shape)} and "
                         f"{tuple(codebook.shape)}")
    from . import _lib

    dev = _lib.require_rocm(blocks)
    b = blocks.to(torch.float32).contiguous()
    if b.data_ptr() % 16:
        b = b.clone()
    cb = codebook.to(device=dev, dtype=torch.float32).contiguous()
    n, d = b.shape
    ids = torch.empty(n, dtype=torch.int64, device=dev)
    dist = torch.empty(n, dtype=torch.float32, device=dev)
    _lib.check(_lib.lib().wal_rvq_assign(b.data_ptr(), n, d, cb.data_ptr(), cb.shape[0], ids.data_ptr(),
                                         dist.data_ptr(), _lib.stream_ptr(dev)))
    return ids, dist


def _centroid_sums(ids: Tensor, blocks: Tensor, k: int) -> tuple[Tensor, Tensor]:
    """``(sums [k, d] fp32, counts [k] int64)`` of the k-means update on the GPU
    (``wal_rvq_centroid_sums``): ``counts = bincount(ids, minlength=k)`` and
    ``sums = zeros(k, d).index_add_(0, ids, blocks)`` with every sum taken in
    ascending block order, as torch's CPU ``index_add_`` adds (reference
    src/block_vq.py:216-218); deterministic, unlike atomics."""
    from . import _lib

    dev = _lib.require_rocm(ids, blocks)
    ids = ids.to(torch.int64).contiguous()
    b = blocks.to(torch.float32).contiguous()
    n, d = b.shape
    if ids.shape != (n,):
        raise ValueError(f"ids must have shape ({n},), got {tuple(ids.shape)}")
    if n:
        lo, hi = torch.stack([ids.min(), ids.max()]).tolist()
        if lo < 0 or hi >= k:
            raise IndexError(f"ids hold index range [{lo}, {hi}] outside [0, {k})")
    sums = torch.empty(k, d, dtype=torch.float32, device=dev)
    counts = torch.empty(k, dtype=torch.int64, device=dev)
    _lib.check(_lib.lib().wal_rvq_centroid_sums(ids.data_ptr(), n, b.data_ptr(), d, k, sums.data_ptr(),
                                                counts.data_ptr(), _lib.stream_ptr(dev)))
    return sums, counts


_HIP_ASSIGN_DIMS = (1, 2, 4, 8, 16, 32)


def _assign(blocks: Tensor, codebook: Tensor, batch_size: int) -> tuple[Tensor, Tensor]:
    """The encoder's assignment: the HIP kernel on a ROCm device for the block
    widths it covers, torch's expression of the same formula otherwise (CPU
    samples, unusual product-split widths)."""
    if blocks.is_cuda and blocks.shape[1] in _HIP_ASSIGN_DIMS:
        return _assign_to_codebook(blocks, codebook)
    return _nearest(blocks, codebook, batch_size)


def _fit_kmeans(blocks: Tensor, codebook_size: int, iters: int, batch_size: int = 16_384) -> Tensor:
    """Lloyd's k-means on the GPU, the reference's ``_fit_kmeans``
    (src/block_vq.py:199-227): initial codewords are the blocks at the first
    ``codebook_size`` positions of a permutation drawn from a generator on the
    blocks' device seeded with 0; every iteration assigns each block to its
    nearest codeword (``_assign_to_codebook``), replaces each non-empty
    cluster's codeword by its mean (``_centroid_sums``, then the fp32 division)
    and reseeds empty clusters from blocks drawn with the same generator."""
    del batch_size
    if blocks.ndim != 2:
        raise ValueError("expected 2D blocks")
    if blocks.shape[0] < codebook_size:
        raise ValueError("sample set must be at least as large as codebook_size")
    blocks = blocks.to(torch.float32)
    gen = torch.Generator(device=blocks.device)
    gen.manual_seed(0)
    first = torch.randperm(blocks.shape[0], generator=gen, device=blocks.device)[:codebook_size]
    codebook = blocks[first].clone()
    for _ in range(iters):
        ids, _ = _assign_to_codebook(blocks, codebook)
        sums, counts = _centroid_sums(ids, blocks, codebook_size)
        filled = counts > 0
        new = codebook.clone()
        new[filled] = sums[filled] / counts[filled].to(torch.float32)[:, None]
        empty = torch.nonzero(~filled).flatten()
        if empty.numel():
            pick = torch.randint(0, blocks.shape[0], (empty.numel(),), generator=gen, device=blocks.device)
            new[empty] = blocks[pick]
        codebook = new
    return codebook


def _kmeans(sample: Tensor, k: int, iters: int, batch_size: int) -> Tensor:
    """Lloyd iterations from a seeded random subset; empty clusters are
    reseeded from random samples.  On a ROCm device this is ``_fit_kmeans``
    (HIP assignment and centroid sums); a CPU sample (the encoder also runs
    offline on the host) takes torch's expression of the same steps."""
    if sample.is_cuda and sample.shape[1] in _HIP_ASSIGN_DIMS:
        return _fit_kmeans(sample, k, iters, batch_size)
    if sample.shape[0] < k:
        raise ValueError("sample set must be at least as large as codebook_size")
    sample = sample.to(torch.float32)
    gen = torch.Generator(device=sample.device)
    gen.manual_seed(0)
    cb = sample[torch.randperm(sample.shape[0], generator=gen, device=sample.device)[:k]].clone()
    for _ in range(iters):
        ids, _ = _nearest(sample, cb, batch_size)
        counts = torch.bincount(ids, minlength=k)
        sums = torch.zeros_like(cb).index_add_(0, ids, sample)
        filled = counts > 0
        cb = cb.clone()
        cb[filled] = sums[filled] / counts[filled].to(torch.float32)[:, None]
        empty = torch.nonzero(~filled).flatten()
        if empty.numel():
            pick = torch.randint(0, sample.shape[0], (empty.numel(),), generator=gen, device=sample.device)
            cb[empty] = sample[pick]
    return cb


@torch.no_grad()
def encode_block_residual_vq(
    weight: Tensor,
    *,
    block_size: int = 32,
    codebook_size: int = 256,
    num_stages: int = 2,
    product_splits: int = 1,
    stages_per_split: tuple[int, ...] | None = None,
    normalize_blocks: str = "none",
    transform_kind: str = "none",
    calibrate_stage_scales: bool = False,
    residual_correction: str = "none",
    sample_limit: int = 131_072,
    kmeans_iters: int = 8,
    batch_size: int = 16_384,
) -> BlockRVQEncoding:
    """Encode one weight matrix (signature of src/block_vq.py:341-356).

    Supported: block_size, codebook_size, num_stages, product_splits,
    stages_per_split, normalize_blocks (none/amax/l2 -> block_scale) and
    calibrate_stage_scales.  ``transform_kind`` other than "none" and
    ``residual_correction`` other than "none" produce encodings the HIP
    runtime does not execute, so they are rejected here.
    """
    if weight.ndim != 2:
        raise ValueError("expected 2D weight")
    if num_stages < 1:
        raise ValueError("num_stages must be >= 1")
    if product_splits < 1 or block_size % product_splits != 0:
        raise ValueError("product_splits must divide block_size and be >= 1")
    if transform_kind != "none":
        raise NotImplementedError("wal2026_amd: transform_kind other than 'none' is not supported by the HIP runtime")
    if residual_correction not in {"none", "sign"}:
        raise ValueError("residual_correction must be one of: none, sign")
    if residual_correction != "none":
        raise NotImplementedError("wal2026_amd: residual_correction='sign' is not supported by the HIP runtime")
    if normalize_blocks not in {"none", "amax", "l2"}:
        raise ValueError("normalize_blocks must be one of: none, amax, l2")
    if stages_per_split is None:
        split_counts = (int(num_stages),) * product_splits
    else:
        split_counts = tuple(int(c) for c in stages_per_split)
        if len(split_counts) != product_splits:
            raise ValueError("stages_per_split must have exactly product_splits entries")
        if any(c < 1 for c in split_counts):
            raise ValueError("each stages_per_split entry must be >= 1")

    row_scale = weight.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8).to(torch.float16)
    blocks, rows, padded = _reshape_blocks(weight.to(torch.float32) / row_scale.to(torch.float32), block_size)
    bpr = padded // block_size
    block_scale = None
    if normalize_blocks == "amax":
        block_scale = blocks.abs().amax(1, keepdim=True).clamp_min(1e-8)
    elif normalize_blocks == "l2":
        block_scale = (blocks * blocks).mean(1, keepdim=True).sqrt().clamp_min(1e-8)
    if block_scale is not None:
        blocks = blocks / block_scale

    residual = blocks.clone()
    n_sample = min(max(int(sample_limit), codebook_size), residual.shape[0])
    gen = torch.Generator(device=residual.device)
    gen.manual_seed(0)
    pick = torch.randperm(residual.shape[0], generator=gen, device=residual.device)[:n_sample]
    sample = residual[pick].clone()

    id_dtype = _id_storage_dtype(codebook_size)
    stage_ids: list[Tensor] = []
    codebooks: list[Tensor] = []
    value_dims: list[int] = []
    sub = block_size // product_splits
    for split, count in enumerate(split_counts):
        lo, hi = split * sub, (split + 1) * sub
        for _ in range(count):
            cb = _kmeans(sample[:, lo:hi], codebook_size, kmeans_iters, batch_size)
            ids, _ = _assign(residual[:, lo:hi], cb, batch_size)
            residual[:, lo:hi] -= cb[ids]
            sids, _ = _assign(sample[:, lo:hi], cb, batch_size)
            sample[:, lo:hi] -= cb[sids]
            full = torch.zeros(codebook_size, block_size, dtype=torch.float32, device=residual.device)
            full[:, lo:hi] = cb
            stage_ids.append(ids.view(rows, bpr).to(id_dtype))
            codebooks.append(full.to(torch.float16))
            value_dims.append(sub if product_splits > 1 else block_size)

    parts = [cb.to(torch.float32)[ids.reshape(-1).long()] for ids, cb in zip(stage_ids, codebooks)]
    recon = torch.stack(parts).sum(0)

    def weight_rel_mse(block_recon: Tensor) -> Tensor:
        r = block_recon if block_scale is None else block_recon * block_scale
        w = r.view(rows, padded)[:, : weight.shape[1]] * row_scale.to(torch.float32)
        ref = weight.to(torch.float32)
        return ((ref - w) ** 2).mean() / (ref ** 2).mean().clamp_min(1e-12)

    stage_scales = None
    if calibrate_stage_scales:
        # least-squares stage weights (ridge 1e-4), kept only if they help
        P = torch.stack([p.reshape(-1) for p in parts])
        gram = P @ P.t() + 1e-4 * torch.eye(len(parts), device=P.device)
        sol = torch.linalg.solve(gram, P @ blocks.reshape(-1)).clamp_min(0.0)
        if float(sol.sum()) > 0.0:
            cand = (torch.stack(parts) * sol[:, None, None]).sum(0)
            if bool(weight_rel_mse(cand) < weight_rel_mse(recon)):
                stage_scales = sol
                recon = cand
    err = blocks[pick] - recon[pick]
    sample_rel_mse = float(((err ** 2).mean() / (blocks[pick] ** 2).mean().clamp_min(1e-12)).item())
    return BlockRVQEncoding(
        stage_ids=tuple(stage_ids),
        codebooks=tuple(codebooks),
        stage_value_dims=tuple(value_dims),
        stages_per_split=split_counts,
        stage_scales=None if stage_scales is None else stage_scales.to(torch.float16),
        residual_correction="none",
        residual_signs=None,
        residual_scale=None,
        row_scale=row_scale,
        block_scale=None if block_scale is None else block_scale.view(rows, bpr).to(torch.float16),
        transform_kind="none",
        transform_matrix=None,
        transform_bias=None,
        product_splits=product_splits,
        original_shape=(int(weight.shape[0]), int(weight.shape[1])),
        padded_cols=padded,
        block_size=block_size,
        sample_rel_mse=sample_rel_mse,
    )


@torch.no_grad()
def encode_grouped_block_residual_vq(weight: Tensor, *, group_rows: int, **kwargs) -> GroupedBlockRVQEncoding:
    """Encode consecutive row groups independently (src/block_vq.py:539-585)."""
    if group_rows < 1:
        raise ValueError("group_rows must be >= 1")
    groups = []
    slices = []
    for r0 in range(0, int(weight.shape[0]), group_rows):
        r1 = min(r0 + group_rows, int(weight.shape[0]))
        groups.append(encode_block_residual_vq(weight[r0:r1], **kwargs))
        slices.append((r0, r1))
    return GroupedBlockRVQEncoding(groups=tuple(groups), row_slices=tuple(slices),
                                   original_shape=(int(weight.shape[0]), int(weight.shape[1])))


def storage_megabytes(num_bytes: int) -> float:
    return float(num_bytes) / 1e6


def dense_bf16_storage_bytes(weight: Tensor) -> int:
    return int(weight.numel()) * 2


def ideal_id_bits_per_weight(block_size: int, codebook_size: int, num_stages: int) -> float:
    """Entropy-free index bits per weight, ceil(log2 K) per stage per block
    (src/block_vq.py:638-639)."""
    return num_stages * math.ceil(math.log2(max(codebook_size, 2))) / float(block_size)
