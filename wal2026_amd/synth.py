"""Seeded synthetic encodings for the benchmark configurations.

Random-init weights of the named architectures' linear shapes, encoded
directly (no k-means): codebooks ~ N(0, 0.02) in fp16, indices uniform in
[0, K), scales ~ U(0.5, 1.5).  One torch.Generator per call, drawn in the
order codebooks -> ids -> scales -> x.

Configs (c1..c5 follow the benchmark's list):
  c1  one 2048x2048 linear, S=2, K=256, d=8, uint8 ids, per-row fp16 scale, fp16 x
  c2  Llama-3.2-1B stack (16 layers), S=2, K=256, d=8, uint8, one codebook set per linear, bf16 x
  c3  Llama-3-8B (32 layers), S=1, K=4096, d=8, 16-bit ids, fp16 scale shared by 128-row groups, bf16 x
  c4  Llama-3-8B shapes, S=2, K=256, d=8, uint8, per-row scale, bf16 x with M=2048 (prefill)
  c5  Qwen2.5-7B (28 layers), S=3, K=256, d=8, uint8, codebooks per 256-row group, per-row bf16 scale
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .block_vq import BlockRVQEncoding, GroupedBlockRVQEncoding, _id_storage_dtype

LINEAR_NAMES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


@dataclass(frozen=True)
class Config:
    name: str
    layers: int
    hidden: int
    kv_out: int
    intermediate: int
    num_stages: int
    codebook_size: int
    block_size: int
    group_rows: int | None      # rows per codebook group; None = one group per linear
    scale_rows: int             # rows sharing one scale value
    scale_dtype: torch.dtype    # dtype the scales are drawn in (the module stores fp16)
    x_dtype: torch.dtype
    m: int                      # activation rows
    id_dtype: torch.dtype | None = None  # None = the reference's storage dtype for K

    def shapes(self) -> list[tuple[str, int, int]]:
        """(name, out_features, in_features) of one layer's linears."""
        h, kv, i = self.hidden, self.kv_out, self.intermediate
        if self.name == "c1":
            return [("linear", 2048, 2048)]
        return [("q_proj", h, h), ("k_proj", kv, h), ("v_proj", kv, h), ("o_proj", h, h),
                ("gate_proj", i, h), ("up_proj", i, h), ("down_proj", h, i)]

    def ids_dtype(self) -> torch.dtype:
        return self.id_dtype or _id_storage_dtype(self.codebook_size)

    def compressed_bytes_per_layer(self) -> int:
        """Algorithmic bytes of one layer: ids + codebooks + scales (2 B each)."""
        total = 0
        ib = torch.empty(0, dtype=self.ids_dtype()).element_size()
        for _, n, k in self.shapes():
            B = -(-k // self.block_size)
            G = 1 if self.group_rows is None else -(-n // self.group_rows)
            total += self.num_stages * n * B * ib
            total += G * self.num_stages * self.codebook_size * self.block_size * 2
            total += n * 2
        return total

    def flops_per_layer(self, m: int | None = None) -> int:
        m = self.m if m is None else m
        return sum(2 * m * n * k for _, n, k in self.shapes())


CONFIGS: dict[str, Config] = {
    "c1": Config("c1", 1, 2048, 2048, 2048, 2, 256, 8, None, 1, torch.float16, torch.float16, 1),
    "c2": Config("c2", 16, 2048, 512, 8192, 2, 256, 8, None, 1, torch.float16, torch.bfloat16, 1),
    "c3": Config("c3", 32, 4096, 1024, 14336, 1, 4096, 8, None, 128, torch.float16, torch.bfloat16, 1),
    "c4": Config("c4", 32, 4096, 1024, 14336, 2, 256, 8, None, 1, torch.float16, torch.bfloat16, 2048),
    "c5": Config("c5", 28, 3584, 512, 18944, 3, 256, 8, 256, 1, torch.bfloat16, torch.bfloat16, 1),
}


def make_encoding(out_features: int, in_features: int, cfg: Config, generator: torch.Generator,
                  device: torch.device | str = "cpu") -> GroupedBlockRVQEncoding:
    """A random GroupedBlockRVQEncoding of the config's format."""
    d, S, K = cfg.block_size, cfg.num_stages, cfg.codebook_size
    B = -(-in_features // d)
    group_rows = cfg.group_rows or out_features
    slices = [(r0, min(r0 + group_rows, out_features)) for r0 in range(0, out_features, group_rows)]
    G = len(slices)
    cbs = (torch.randn(G, S, K, d, generator=generator, device=device) * 0.02).to(torch.float16)
    ids = torch.randint(0, K, (S, out_features, B), generator=generator, device=device, dtype=cfg.ids_dtype())
    n_scale = -(-out_features // cfg.scale_rows)
    scale = (torch.rand(n_scale, 1, generator=generator, device=device) + 0.5).to(cfg.scale_dtype)
    if cfg.scale_rows > 1:
        scale = scale.repeat_interleave(cfg.scale_rows, dim=0)[:out_features]
    groups = []
    for g, (r0, r1) in enumerate(slices):
        groups.append(BlockRVQEncoding(
            stage_ids=tuple(ids[s, r0:r1].contiguous() for s in range(S)),
            codebooks=tuple(cbs[g, s].contiguous() for s in range(S)),
            stage_value_dims=(d,) * S,
            stages_per_split=(S,),
            stage_scales=None,
            residual_correction="none",
            residual_signs=None,
            residual_scale=None,
            row_scale=scale[r0:r1].contiguous(),
            block_scale=None,
            transform_kind="none",
            transform_matrix=None,
            transform_bias=None,
            product_splits=1,
            original_shape=(r1 - r0, in_features),
            padded_cols=B * d,
            block_size=d,
            sample_rel_mse=0.0,
        ))
    return GroupedBlockRVQEncoding(groups=tuple(groups), row_slices=tuple(slices),
                                   original_shape=(out_features, in_features))


def make_activation(m: int, in_features: int, dtype: torch.dtype, generator: torch.Generator,
                    device: torch.device | str = "cpu") -> torch.Tensor:
    return torch.randn(m, in_features, generator=generator, device=device).to(dtype)


def generator(seed: int = 0, device: torch.device | str = "cpu") -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g
