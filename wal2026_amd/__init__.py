"""wal2026_amd: MI355X-native Block-RVQ / route-codebook linear forward.

Drop-in for the DRL-runtime compressed linear of AubakirovArman/wal2026
(src/runtime.py, src/block_vq.py, src/triton_id_matmul.py,
src/encoding_io.py).  The compute runs in libwal2026_amd.so (hand-written HIP
for gfx950, C ABI in include/wal2026_amd.h); this package is the host-side
mirror of the reference's Python interface.
"""
from .block_vq import (
    BlockRVQEncoding,
    GroupedBlockRVQEncoding,
    dense_bf16_storage_bytes,
    encode_block_residual_vq,
    encode_grouped_block_residual_vq,
    ideal_id_bits_per_weight,
    storage_megabytes,
)
from .encoding_io import load_grouped_encoding_map, save_grouped_encoding_map
from .kernels import id_route_linear_matmul, rvq_group_linear_matmul
from .runtime import (
    TARGET_LINEAR_SUFFIXES,
    AdaptiveFusedIDRouteLinear,
    CachedPackedIDRouteLinear,
    FusedBlockRVQLinears,
    FusedIDRouteLinear,
    PackedBlockRVQGroup,
    PackedGroupedBlockRVQLinear,
    PackedIDRouteLinear,
    fuse_sibling_linears,
    replace_with_packed_block_rvq,
    replace_with_preencoded_packed_block_rvq,
    set_effective_stages_by_name,
    set_effective_stages_from_map,
    set_global_effective_stages,
    unfuse_sibling_linears,
)

__all__ = [
    "AdaptiveFusedIDRouteLinear",
    "BlockRVQEncoding",
    "CachedPackedIDRouteLinear",
    "FusedBlockRVQLinears",
    "FusedIDRouteLinear",
    "GroupedBlockRVQEncoding",
    "PackedBlockRVQGroup",
    "PackedGroupedBlockRVQLinear",
    "PackedIDRouteLinear",
    "TARGET_LINEAR_SUFFIXES",
    "dense_bf16_storage_bytes",
    "encode_block_residual_vq",
    "encode_grouped_block_residual_vq",
    "fuse_sibling_linears",
    "id_route_linear_matmul",
    "ideal_id_bits_per_weight",
    "load_grouped_encoding_map",
    "replace_with_packed_block_rvq",
    "replace_with_preencoded_packed_block_rvq",
    "rvq_group_linear_matmul",
    "save_grouped_encoding_map",
    "set_effective_stages_by_name",
    "set_effective_stages_from_map",
    "set_global_effective_stages",
    "storage_megabytes",
    "unfuse_sibling_linears",
]
