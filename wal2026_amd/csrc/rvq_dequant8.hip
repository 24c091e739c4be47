// rvq_dequant8.hip -- the dense weight of a block-size-8 layer
// (PackedBlockRVQGroup.reconstruct_weight / reconstruct_weight_fast,
// src/runtime.py:379-414 / :568-598) for the layouts the MFMA kernels accept,
// written at HBM speed.
//
// A workgroup takes one tile of rows of one group, stages the group's
// codebooks in LDS in the MFMA kernels' form (rvq_fragment.h) and writes the
// tile's weights, one 8-weight block per lane and 64 consecutive blocks of a
// row per wave instruction.  Each block is rebuilt by the same fragment code
// the decode and prefill kernels multiply with (gather the S codewords, the
// reference's rounding, the row scale), with the row-scale product keeping
// the sign of a zero, which a dense weight shows.
#include "rvq_fragment.h"

namespace wal {

constexpr int kDq8Threads = 256;
constexpr int kDq8Batch = 8;  // items per wave whose loads are in flight together

template <int S, typename IdT, int LMODE, int SEM, int XDT>
__global__ __launch_bounds__(kDq8Threads) void rvq_dequant8_kernel(LayerArgs L, DtypeArgs D,
                                                                     uint16_t* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const FragTile<S> ti = get_frag_tile<S>(L, blockIdx.x);
  const int K = L.codebook_size;
  stage_codebooks<S, LMODE, SEM, XDT>(smem, ti.p, K, D);
  __syncthreads();
  const int B = L.blocks_per_row;
  const int nb = (B + 63) >> 6;  // 64-block items per row
  const int64_t in = L.in_features;
  const uint32_t kmax = (uint32_t)(K - 1);
  const int items = ti.rows * nb;
  // (uniform: an item's row, scale and index offsets are scalar work)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  // The tile's items are shared by the gridDim.y workgroups of its column
  // of the grid: wave w of workgroup y takes items w + NW y, w + NW y + NWY,
  // ... (NWY = NW gridDim.y); lane l takes block 64 c + l of the item's row,
  // so each index load and each weight store of a wave is one contiguous run
  // (64 ids, 1 KB of weights).  Batches of kDq8Batch items: every index and
  // scale load of a batch is issued before the first is used, so a batch
  // waits for memory once, not once per item.
  constexpr int NW = kDq8Threads / 64;
  const int NWY = NW * (int)gridDim.y;
  for (int base = wave + NW * (int)blockIdx.y; base < items; base += NWY * kDq8Batch) {
    uint32_t idv[kDq8Batch][S];
    float rsv[kDq8Batch];
#pragma unroll
    for (int u = 0; u < kDq8Batch; ++u) {
      const int it = min(base + NWY * u, items - 1);  // past the end: reload the last item
      const int rr = it / nb;
      const int b = min(64 * (it - rr * nb) + lane, B - 1);
      const int64_t r = ti.row0 + rr;
      rsv[u] = load_f(ti.p.row_scale, D.sc_dtype, scale_index(L, r));
#pragma unroll
      for (int s = 0; s < S; ++s) idv[u][s] = static_cast<const IdT*>(ti.p.ids[s])[r * B + b];
    }
#pragma unroll
    for (int u = 0; u < kDq8Batch; ++u) {
      const int it = base + NWY * u;
      const int rr = it / nb;
      const int b = 64 * (it - rr * nb) + lane;
      if (it < items && b < B) {
        uint32_t id[S];
#pragma unroll
        for (int s = 0; s < S; ++s) id[s] = min(idv[u][s], kmax);  // past the codebook: its last entry, as every kernel does
        const u32x4_t w = combine_wfrag<S, LMODE, SEM, XDT, true>(gather_wfrag<S, LMODE>(smem, id, K), L.active_mask,
                                                                  make_row_scale<XDT>(rsv[u]));
        *reinterpret_cast<u32x4_t*>(out + (ti.out_row0 + rr) * in + 8 * (int64_t)b) = w;
      }
    }
  }
}

template <int S, typename IdT, int LMODE, int SEM, int XDT>
static hipError_t dq8_go(const LayerArgs& L, const DtypeArgs& D, void* out, hipStream_t st) {
  auto kern = rvq_dequant8_kernel<S, IdT, LMODE, SEM, XDT>;
  const size_t lds = (size_t)S * L.codebook_size * lds_entry_bytes<LMODE>();
  hipError_t e = allow_max_lds(reinterpret_cast<const void*>(kern));
  if (e != hipSuccess) return e;
  // About 8 workgroups per CU (2 with tables of 32 KB or more): the tiles'
  // items are split over gridDim.y workgroups when the tiles alone are fewer
  // (a 4096-row layer has 256 16-row tiles), so that enough waves hide the
  // memory, LDS and VALU latencies of the item loop.  Measured at c4's
  // shapes (HIP events): down_proj 76.9 / 47.3 / 34.7 / 30.0 us with 1 / 2 /
  // 4 / 8 workgroups per tile, the fused gate/up weight 52.9 / 50.3 us with
  // 1 / 2.
  const int per_cu = lds >= 32 * 1024 ? 2 : 8;
  const int64_t want = (int64_t)per_cu * device_cu_count();
  const int items_per_tile = L.tile_rows * ((L.blocks_per_row + 63) / 64);
  int ny = (int)((want + L.n_tiles - 1) / L.n_tiles);
  ny = ny < 1 ? 1 : (ny > items_per_tile / 4 ? (items_per_tile / 4 > 0 ? items_per_tile / 4 : 1) : ny);
  hipLaunchKernelGGL(kern, dim3((unsigned)L.n_tiles, (unsigned)ny), dim3(kDq8Threads), lds, st, L, D,
                     static_cast<uint16_t*>(out));
  return hipGetLastError();
}

template <int S, typename IdT, int XDT>
static hipError_t dq8_sem(const LayerArgs& L, const DtypeArgs& D, int sem, int lmode, void* out, hipStream_t st) {
  if (sem == SEM_FAST) return dq8_go<S, IdT, LM_A16, SEM_FAST, XDT>(L, D, out, st);
  if constexpr (S == 1) {
    return dq8_go<S, IdT, LM_A16, SEM_RECON, XDT>(L, D, out, st);
  } else {
    if (lmode == LM_H16) return dq8_go<S, IdT, LM_H16, SEM_RECON, XDT>(L, D, out, st);
    return dq8_go<S, IdT, LM_F32, SEM_RECON, XDT>(L, D, out, st);
  }
}

template <typename IdT, int XDT>
static hipError_t dq8_stages(const LayerArgs& L, const DtypeArgs& D, int sem, int lmode, void* out, hipStream_t st) {
  switch (L.num_stages) {
    case 1: return dq8_sem<1, IdT, XDT>(L, D, sem, lmode, out, st);
    case 2: return dq8_sem<2, IdT, XDT>(L, D, sem, lmode, out, st);
    case 3: return dq8_sem<3, IdT, XDT>(L, D, sem, lmode, out, st);
    default: return dq8_sem<4, IdT, XDT>(L, D, sem, lmode, out, st);
  }
}

hipError_t launch_dequant8(const LayerArgs& L, const DtypeArgs& D, int sem, int lmode, void* out, hipStream_t st) {
  if (L.n_tiles == 0) return hipSuccess;
  const bool wide = D.id_dtype != WAL_U8;
  if (D.x_dtype == WAL_BF16)
    return wide ? dq8_stages<uint16_t, WAL_BF16>(L, D, sem, lmode, out, st)
                : dq8_stages<uint8_t, WAL_BF16>(L, D, sem, lmode, out, st);
  return wide ? dq8_stages<uint16_t, WAL_F16>(L, D, sem, lmode, out, st)
              : dq8_stages<uint8_t, WAL_F16>(L, D, sem, lmode, out, st);
}

}  // namespace wal
