"""Persisted encodings: the reference's v1 map format (src/encoding_io.py:10-94).

A file is a ``torch.save`` dict ``{"version": 1, "encodings": {name: grouped}}``
where each grouped encoding is ``{"groups": [...], "row_slices": [[r0, r1],
...], "original_shape": [rows, cols]}`` and each group is the field-by-field
dict of a BlockRVQEncoding with tensors on the CPU.  Files written by the
reference load here and vice versa.

Loading uses ``torch.load(..., weights_only=True)``: the payload is plain
containers, strings, numbers and tensors, so nothing in the file is executed.
"""
from __future__ import annotations

from pathlib import Path

import torch

from .block_vq import BlockRVQEncoding, GroupedBlockRVQEncoding

_TENSOR_FIELDS = ("stage_scales", "residual_signs", "residual_scale", "row_scale", "block_scale",
                  "transform_matrix", "transform_bias")


def _cpu(t):
    return None if t is None else t.detach().cpu()


def _serialize_block_encoding(enc: BlockRVQEncoding) -> dict[str, object]:
    out: dict[str, object] = {
        "stage_ids": [_cpu(t) for t in enc.stage_ids],
        "codebooks": [_cpu(t) for t in enc.codebooks],
        "stage_value_dims": [int(v) for v in enc.stage_value_dims],
        "stages_per_split": [int(v) for v in enc.stages_per_split],
        "residual_correction": enc.residual_correction,
        "transform_kind": enc.transform_kind,
        "product_splits": int(enc.product_splits),
        "original_shape": [int(v) for v in enc.original_shape],
        "padded_cols": int(enc.padded_cols),
        "block_size": int(enc.block_size),
        "sample_rel_mse": float(enc.sample_rel_mse),
    }
    for name in _TENSOR_FIELDS:
        out[name] = _cpu(getattr(enc, name))
    return out


def _deserialize_block_encoding(payload: dict[str, object], device: torch.device | None = None) -> BlockRVQEncoding:
    def move(t):
        return t if t is None or device is None else t.to(device)

    return BlockRVQEncoding(
        stage_ids=tuple(move(t) for t in payload["stage_ids"]),
        codebooks=tuple(move(t) for t in payload["codebooks"]),
        stage_value_dims=tuple(int(v) for v in payload["stage_value_dims"]),
        stages_per_split=tuple(int(v) for v in payload["stages_per_split"]),
        stage_scales=move(payload["stage_scales"]),
        residual_correction=str(payload["residual_correction"]),
        residual_signs=move(payload["residual_signs"]),
        residual_scale=move(payload["residual_scale"]),
        row_scale=move(payload["row_scale"]),
        block_scale=move(payload["block_scale"]),
        transform_kind=str(payload["transform_kind"]),
        transform_matrix=move(payload["transform_matrix"]),
        transform_bias=move(payload["transform_bias"]),
        product_splits=int(payload["product_splits"]),
        original_shape=tuple(int(v) for v in payload["original_shape"]),
        padded_cols=int(payload["padded_cols"]),
        block_size=int(payload["block_size"]),
        sample_rel_mse=float(payload["sample_rel_mse"]),
    )


def serialize_grouped_encoding(enc: GroupedBlockRVQEncoding) -> dict[str, object]:
    return {
        "groups": [_serialize_block_encoding(g) for g in enc.groups],
        "row_slices": [[int(a), int(b)] for a, b in enc.row_slices],
        "original_shape": [int(v) for v in enc.original_shape],
    }


def deserialize_grouped_encoding(payload: dict[str, object], device: torch.device | None = None) -> GroupedBlockRVQEncoding:
    return GroupedBlockRVQEncoding(
        groups=tuple(_deserialize_block_encoding(g, device=device) for g in payload["groups"]),
        row_slices=tuple(tuple(int(v) for v in s) for s in payload["row_slices"]),
        original_shape=tuple(int(v) for v in payload["original_shape"]),
    )


def save_grouped_encoding_map(path: str | Path, encodings: dict[str, GroupedBlockRVQEncoding]) -> Path:
    """src/encoding_io.py:77-85."""
    target = Path(path)
    target.parent.mkdir(parents=True, exist_ok=True)
    torch.save({"version": 1, "encodings": {k: serialize_grouped_encoding(v) for k, v in encodings.items()}}, target)
    return target


def load_grouped_encoding_map(path: str | Path, device: torch.device | None = None) -> dict[str, GroupedBlockRVQEncoding]:
    """src/encoding_io.py:88-94, with the safe loader."""
    payload = torch.load(Path(path), map_location="cpu", weights_only=True)
    if int(payload.get("version", 0)) != 1:
        raise ValueError(f"unsupported encoding map version: {payload.get('version')}")
    return {k: deserialize_grouped_encoding(v, device=device) for k, v in payload["encodings"].items()}
