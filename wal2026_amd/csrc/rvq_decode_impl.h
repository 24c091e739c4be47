// rvq_decode.hip -- Block-RVQ linear for M <= 16 (decode), block_size 8.
//
// The weight is never written to memory.  Layout of the work:
//   * A workgroup (NW waves) is persistent over a contiguous range of 16-row
//     tiles.  It keeps the codebooks of the current group in LDS (restaged
//     only when the tile's group changes).
//   * Each wave handles the 64-block chunks c = wave, wave + NW, ... of the
//     tile.  Lane l covers weight row n = l % 16 and the 16 consecutive blocks
//     [64c + 16q, 64c + 16q + 16), q = l / 16: one 128-bit load per stage for
//     8-bit ids (two for 16-bit ids) streams those indices from HBM.
//   * For each of the 16 blocks the lane gathers the S codewords from LDS,
//     rebuilds the 8 weights exactly as the reference's dequantisation does
//     (rvq_fragment.h) and feeds them as the B operand of
//     v_mfma_f32_16x16x32_{bf16,f16}; the A operand is x[m = l % 16] at the
//     same 8 columns (zero for m >= M).  MFMA k-slot group q <-> block
//     64c + 16q + t, for t = 0..15, so each lane's indices stay contiguous.
//   * The NW partial 16x16 accumulators are summed through LDS and the M x 16
//     outputs of the tile are written once.
// The next chunk's indices are loaded before the current chunk is computed.
#pragma once

#include "rvq_fragment.h"

namespace wal {

template <typename IdT>
struct IdChunk {
  static constexpr int kVec = sizeof(IdT);  // 128-bit loads per stage per chunk
};

template <typename IdT>
__device__ inline uint32_t extract_id(const u32x4_t (&v)[sizeof(IdT)], int t) {
  if constexpr (sizeof(IdT) == 1) {
    return (v[0][t >> 2] >> (8 * (t & 3))) & 0xffu;
  } else {
    return (v[t >> 3][(t >> 1) & 3] >> (16 * (t & 1))) & 0xffffu;
  }
}

template <int S, typename IdT, int LMODE, int SEM, int XDT, int NW>
__global__ __launch_bounds__(NW * 64) void rvq_decode_kernel(LayerArgs L, DtypeArgs D, EpilogueArgs E,
                                                             const uint16_t* __restrict__ x, int M) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr int ESZ = lds_entry_bytes<LMODE>();
  constexpr int NV = sizeof(IdT);
  const int K = L.codebook_size;
  uint8_t* lds_cb = smem;
  float* red = reinterpret_cast<float*>(smem + (size_t)S * K * ESZ);  // [2][NW][256]

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nl = lane & 15;
  const int q = lane >> 4;
  const int B = L.blocks_per_row;
  const int in = L.in_features;
  const int nchunk = (B + 63) >> 6;
  const int T = L.n_tiles;
  const int t_begin = (int)((int64_t)blockIdx.x * T / gridDim.x);
  const int t_end = (int)((int64_t)(blockIdx.x + 1) * T / gridDim.x);
  const uint32_t kmax = (uint32_t)(K - 1);

  int staged = -1;
  int buf = 0;
  for (int t = t_begin; t < t_end; ++t) {
    const TileInfo ti = get_tile(L, t);
    if (ti.group != staged) {
      __syncthreads();
      stage_codebooks<S, LMODE, SEM, XDT>(lds_cb, ti.g, K, D);
      __syncthreads();
      staged = ti.group;
    }
    const bool row_ok = nl < ti.rows;
    const int64_t r = ti.row0 + nl;
    const float rs_raw = row_ok ? load_f(ti.g.row_scale, D.sc_dtype, r / L.scale_rows) : 0.0f;
    const RowScale rs = make_row_scale<XDT>(rs_raw);

    const IdT* idp[S];
#pragma unroll
    for (int s = 0; s < S; ++s) idp[s] = reinterpret_cast<const IdT*>(ti.g.stage_ids[s]) + r * B;
    const uint16_t* xrow = x + (int64_t)nl * in;
    const bool x_ok = nl < M;

    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    u32x4_t ids_next[S][NV];
    int c = wave;
    {
      const int base = c * 64 + 16 * q;
      const bool ok = row_ok && c < nchunk && base < B;
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int v = 0; v < NV; ++v)
          ids_next[s][v] = ok ? reinterpret_cast<const u32x4_t*>(idp[s] + base)[v] : u32x4_t{0, 0, 0, 0};
    }
    for (; c < nchunk; c += NW) {
      const int base = c * 64 + 16 * q;
      const bool seg_ok = base < B;
      const bool ok = row_ok && seg_ok;
      u32x4_t ids[S][NV];
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int v = 0; v < NV; ++v) ids[s][v] = ids_next[s][v];
      {
        const int cn = c + NW;
        const int basen = cn * 64 + 16 * q;
        const bool okn = row_ok && cn < nchunk && basen < B;
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
          for (int v = 0; v < NV; ++v)
            ids_next[s][v] = okn ? reinterpret_cast<const u32x4_t*>(idp[s] + basen)[v] : u32x4_t{0, 0, 0, 0};
      }
      u32x4_t xf[16];
      const bool xok = x_ok && seg_ok;
#pragma unroll
      for (int tt = 0; tt < 16; ++tt)
        xf[tt] = xok ? *reinterpret_cast<const u32x4_t*>(xrow + (int64_t)(base + tt) * 8) : u32x4_t{0, 0, 0, 0};
#pragma unroll
      for (int tt = 0; tt < 16; ++tt) {
        uint32_t id[S];
#pragma unroll
        for (int s = 0; s < S; ++s) id[s] = min(extract_id<IdT>(ids[s], tt), kmax);
        u32x4_t w = make_wfrag<S, LMODE, SEM, XDT>(lds_cb, id, K, L.active_mask, rs);
        if (!ok) w = u32x4_t{0, 0, 0, 0};
        acc = mfma16<XDT>(xf[tt], w, acc);
      }
    }
    // lane holds D[m = 4q + i][n = nl], i = 0..3
    float* rb = red + (size_t)buf * NW * 256 + wave * 256;
#pragma unroll
    for (int i = 0; i < 4; ++i) rb[(4 * q + i) * 16 + nl] = acc[i];
    __syncthreads();
    if ((int)threadIdx.x < M * 16) {
      const int m = threadIdx.x >> 4;
      const int n = threadIdx.x & 15;
      const float* rr = red + (size_t)buf * NW * 256 + threadIdx.x;
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) v += rr[w * 256];
      if (n < ti.rows) store_output(E, m, ti.out_row0 + n, v);
    }
    buf ^= 1;
  }
}

constexpr int kDecodeWaves = 4;

template <int S, typename IdT, int LMODE, int SEM, int XDT>
static hipError_t decode_go(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, const void* x, int M,
                            int n_cu, hipStream_t st) {
  constexpr int NW = kDecodeWaves;
  const size_t lds = (size_t)S * L.codebook_size * lds_entry_bytes<LMODE>() + 2 * NW * 256 * sizeof(float);
  auto kern = rvq_decode_kernel<S, IdT, LMODE, SEM, XDT, NW>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  int per_cu = (int)((160 * 1024) / lds);
  if (per_cu > 4) per_cu = 4;
  if (per_cu < 1) per_cu = 1;
  int grid = n_cu * per_cu;
  if (grid > L.n_tiles) grid = L.n_tiles;
  if (grid < 1) return hipSuccess;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(NW * 64), lds, st, L, D, E, reinterpret_cast<const uint16_t*>(x), M);
  return hipGetLastError();
}

template <int S, typename IdT, int XDT>
static hipError_t decode_sem(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, int sem, int lmode,
                             const void* x, int M, int n_cu, hipStream_t st) {
  if (sem == SEM_FAST) return decode_go<S, IdT, LM_A16, SEM_FAST, XDT>(L, D, E, x, M, n_cu, st);
  if constexpr (S == 1) {
    return decode_go<S, IdT, LM_A16, SEM_RECON, XDT>(L, D, E, x, M, n_cu, st);
  } else {
    if (lmode == LM_H16) return decode_go<S, IdT, LM_H16, SEM_RECON, XDT>(L, D, E, x, M, n_cu, st);
    return decode_go<S, IdT, LM_F32, SEM_RECON, XDT>(L, D, E, x, M, n_cu, st);
  }
}

// Entry for one (activation dtype, index width); explicitly instantiated in
// rvq_decode_<x>_<ids>.hip so the variants compile in parallel.
template <int XDT, typename IdT>
hipError_t decode_entry(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, int sem, int lmode,
                        const void* x, int M, int n_cu, hipStream_t st) {
  switch (L.num_stages) {
    case 1: return decode_sem<1, IdT, XDT>(L, D, E, sem, lmode, x, M, n_cu, st);
    case 2: return decode_sem<2, IdT, XDT>(L, D, E, sem, lmode, x, M, n_cu, st);
    case 3: return decode_sem<3, IdT, XDT>(L, D, E, sem, lmode, x, M, n_cu, st);
    default: return decode_sem<4, IdT, XDT>(L, D, E, sem, lmode, x, M, n_cu, st);
  }
}

}  // namespace wal
