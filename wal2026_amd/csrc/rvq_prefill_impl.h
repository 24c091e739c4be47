// rvq_prefill.hip -- Block-RVQ linear for large M (prefill), block_size 8.
//
// Workgroup tile: 128 x rows (M) x 128 weight rows (N), k-step 64 columns
// (8 blocks).  256 threads = 4 waves in a 2 x 2 arrangement, each wave owning
// a 64 x 64 output sub-tile = 4 x 4 v_mfma_f32_16x16x32 tiles.
// Per k-step every thread
//   * loads 64 bytes of x (4 x 128-bit) into the x tile in LDS, and
//   * dequantises 4 blocks (32 weights) of one weight row from the LDS
//     codebooks with the reference's exact rounding (rvq_fragment.h) into the
//     W tile in LDS (bf16/fp16 -- the MFMA input dtype).
// Both tiles are double-buffered; the global loads for step k+1 are issued
// before the MFMAs of step k.  Rows are padded by 16 bytes so the 16 rows a
// ds_read_b128 touches fall in distinct banks.
#pragma once

#include "rvq_fragment.h"

namespace wal {

constexpr int PM = 128, PK = 64;  // x rows and columns per tile; 128 weight rows (tile kind 2)
constexpr int PSTRIDE = PK + 8;  // elements per LDS row (144 bytes)
constexpr int kTileElems = PM * PSTRIDE;

template <int S, typename IdT, int LMODE, int SEM, int XDT>
__global__ __launch_bounds__(256) void rvq_prefill_kernel(LayerArgs L, DtypeArgs D, EpilogueArgs E,
                                                          const uint16_t* __restrict__ x, int64_t M) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int K = L.codebook_size;
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);   // [2][PM][PSTRIDE]
  uint16_t* ws = xs + 2 * kTileElems;                  // [2][PN][PSTRIDE]
  uint8_t* lds_cb = reinterpret_cast<uint8_t*>(ws + 2 * kTileElems);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l16 = lane & 15, q = lane >> 4;
  const FragTile<S> ti = get_frag_tile<S>(L, blockIdx.x);
  const int64_t m0 = (int64_t)blockIdx.y * PM;
  const int B = L.blocks_per_row;
  const int in = L.in_features;
  const int nk = (in + PK - 1) / PK;
  const uint32_t kmax = (uint32_t)(K - 1);

  stage_codebooks<S, LMODE, SEM, XDT>(lds_cb, ti.p, K, D);

  // loader roles: row lr = tid / 2, half lh = tid % 2
  const int lr = tid >> 1, lh = tid & 1;
  const int64_t xm = m0 + lr;
  const bool x_row_ok = xm < M;
  const uint16_t* xrow = x + xm * in;
  const bool w_row_ok = lr < ti.rows;
  const int64_t wr = ti.row0 + lr;
  const float rs_raw = w_row_ok ? load_f(ti.p.row_scale, D.sc_dtype, scale_index(L, wr)) : 0.0f;
  const RowScale rs = make_row_scale<XDT>(rs_raw);
  const IdT* idp[S];
#pragma unroll
  for (int s = 0; s < S; ++s) idp[s] = reinterpret_cast<const IdT*>(ti.p.ids[s]) + wr * B;

  u32x4_t xreg[4];
  uint32_t idreg[S][4];

  auto load_step = [&](int k) {
    const int col0 = k * PK + 32 * lh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int col = col0 + 8 * i;
      xreg[i] = (x_row_ok && col < in) ? ldg128(xrow + col) : u32x4_t{0, 0, 0, 0};
    }
    const int b0 = k * (PK / 8) + 4 * lh;
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        idreg[s][i] = (w_row_ok && b0 + i < B) ? (uint32_t)ldg<IdT>(idp[s], b0 + i) : 0u;
  };
  auto store_step = [&](int k, int bufi) {
    uint16_t* xd = xs + bufi * kTileElems + lr * PSTRIDE + 32 * lh;
    uint16_t* wd = ws + bufi * kTileElems + lr * PSTRIDE + 32 * lh;
    const int b0 = k * (PK / 8) + 4 * lh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<u32x4_t*>(xd + 8 * i) = xreg[i];
      uint32_t id[S];
#pragma unroll
      for (int s = 0; s < S; ++s) id[s] = min(idreg[s][i], kmax);
      u32x4_t w = make_wfrag<S, LMODE, SEM, XDT>(lds_cb, id, K, L.active_mask, rs);
      if (!(w_row_ok && b0 + i < B)) w = u32x4_t{0, 0, 0, 0};
      *reinterpret_cast<u32x4_t*>(wd + 8 * i) = w;
    }
  };

  f32x4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  load_step(0);
  __syncthreads();  // codebooks staged
  store_step(0, 0);
  __syncthreads();
  for (int k = 0; k < nk; ++k) {
    const int cur = k & 1;
    if (k + 1 < nk) load_step(k + 1);
    const uint16_t* xa = xs + cur * kTileElems + (wm * 64 + l16) * PSTRIDE + 8 * q;
    const uint16_t* wb = ws + cur * kTileElems + (wn * 64 + l16) * PSTRIDE + 8 * q;
#pragma unroll
    for (int kk = 0; kk < PK; kk += 32) {
      u32x4_t a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const u32x4_t*>(xa + i * 16 * PSTRIDE + kk);
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const u32x4_t*>(wb + j * 16 * PSTRIDE + kk);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<XDT>(a[i], b[j], acc[i][j]);
    }
    if (k + 1 < nk) store_step(k + 1, cur ^ 1);
    __syncthreads();
  }

  // lane holds D[m = 4q + e][n = l16] of each 16 x 16 sub-tile
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int nloc = wn * 64 + j * 16 + l16;
      if (nloc >= ti.rows) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t m = m0 + wm * 64 + i * 16 + 4 * q + e;
        if (m < M) store_output(E, m, ti.out_row0 + nloc, acc[i][j][e]);
      }
    }
  }
}

template <int S, typename IdT, int LMODE, int SEM, int XDT>
static hipError_t prefill_go(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, const void* x,
                             int64_t M, hipStream_t st) {
  const size_t lds = (size_t)4 * kTileElems * sizeof(uint16_t) + (size_t)S * L.codebook_size * lds_entry_bytes<LMODE>();
  auto kern = rvq_prefill_kernel<S, IdT, LMODE, SEM, XDT>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  dim3 grid(L.n_tiles, (unsigned)((M + PM - 1) / PM));
  hipLaunchKernelGGL(kern, grid, dim3(256), lds, st, L, D, E, reinterpret_cast<const uint16_t*>(x), M);
  return hipGetLastError();
}

template <int S, typename IdT, int XDT>
static hipError_t prefill_sem(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, int sem, int lmode,
                              const void* x, int64_t M, hipStream_t st) {
  if (sem == SEM_FAST) return prefill_go<S, IdT, LM_A16, SEM_FAST, XDT>(L, D, E, x, M, st);
  if constexpr (S == 1) {
    return prefill_go<S, IdT, LM_A16, SEM_RECON, XDT>(L, D, E, x, M, st);
  } else {
    if (lmode == LM_H16) return prefill_go<S, IdT, LM_H16, SEM_RECON, XDT>(L, D, E, x, M, st);
    return prefill_go<S, IdT, LM_F32, SEM_RECON, XDT>(L, D, E, x, M, st);
  }
}

// Entry for one (activation dtype, index width); explicitly instantiated in
// rvq_prefill_<x>_<ids>.hip.
template <int XDT, typename IdT>
hipError_t prefill_entry(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, int sem, int lmode,
                         const void* x, int64_t M, hipStream_t st) {
  switch (L.num_stages) {
    case 1: return prefill_sem<1, IdT, XDT>(L, D, E, sem, lmode, x, M, st);
    case 2: return prefill_sem<2, IdT, XDT>(L, D, E, sem, lmode, x, M, st);
    case 3: return prefill_sem<3, IdT, XDT>(L, D, E, sem, lmode, x, M, st);
    default: return prefill_sem<4, IdT, XDT>(L, D, E, sem, lmode, x, M, st);
  }
}

}  // namespace wal
