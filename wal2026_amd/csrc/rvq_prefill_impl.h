// rvq_prefill_impl.h -- Block-RVQ linear for large M (prefill), block_size 8.
//
// Workgroup tile: BM = 32 * TM activation rows x 256 weight rows (tile kind 2),
// k-step 32 columns (4 blocks).  512 threads = 8 waves in a 2 (M) x 4 (N)
// arrangement; a wave owns 16 TM x 64 outputs = TM x 4 tiles of
// v_mfma_f32_16x16x32_{bf16,f16}.  Per k-step every thread
//   * dequantises 2 blocks (16 weights) of one weight row from the LDS
//     codebooks with the reference's exact rounding (make_wfrag) into the W
//     tile in LDS, in the MFMA input dtype, and
//   * copies one or two 16-byte pieces of x (the tile is BM rows x 64 bytes)
//     into the x tile in LDS.
// Both tiles are double-buffered.  The x pieces are loaded two k-steps ahead
// and the index bytes (16 blocks = 4 k-steps per load) one load group ahead,
// so the loads have two MFMA phases to arrive.  Rows are padded by 16 bytes
// (80-byte stride) so the 16 rows a ds_read_b128 fragment read touches fall in
// distinct banks.
//
// Grid: the x-row tile index varies fastest, so consecutive workgroups (which
// the dispatcher deals round-robin to the XCDs) share one weight tile and each
// XCD keeps revisiting the same few x tiles in its L2.
#pragma once

#include "rvq_fragment.h"

namespace wal {

constexpr int kPrefillThreads = 512;
constexpr int PBN = 256;        // weight rows per workgroup tile
constexpr int PBK = 32;         // k per step
constexpr int PSTR = PBK + 8;   // elements per LDS row (80 bytes)

template <int TM>
constexpr int prefill_bm() { return 32 * TM; }

template <int S, int LMODE>
WAL_HOST_DEVICE size_t prefill_lds_bytes(int TM, int K) {
  return (size_t)2 * (32 * TM + PBN) * PSTR * sizeof(uint16_t) + (size_t)S * K * lds_entry_bytes<LMODE>();
}

template <int S, typename IdT, int LMODE, int SEM, int XDT, int TM>
__global__ __launch_bounds__(kPrefillThreads) void rvq_prefill_kernel(LayerArgs L, DtypeArgs D, EpilogueArgs E,
                                                                      const uint16_t* __restrict__ x, int64_t M,
                                                                      int n_mt) {
  constexpr int BM = prefill_bm<TM>();
  constexpr int XP = BM * 4 / kPrefillThreads;  // 16-byte x pieces per thread per k-step (1 or 2)
  constexpr int NV = sizeof(IdT);                // 16-byte index loads per stage per group of 4 k-steps
  static_assert(XP >= 1 && BM * 4 % kPrefillThreads == 0, "x tile split");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);  // [2][BM][PSTR]
  uint16_t* ws = xs + 2 * BM * PSTR;                 // [2][PBN][PSTR]
  uint8_t* lds_cb = reinterpret_cast<uint8_t*>(ws + 2 * PBN * PSTR);

  const int K = L.codebook_size;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int l16 = lane & 15, q = lane >> 4;
  const int mt = (int)(blockIdx.x % (unsigned)n_mt);
  const int nt = (int)(blockIdx.x / (unsigned)n_mt);
  const FragTile<S> ti = get_frag_tile<S>(L, nt);
  const int64_t m0 = (int64_t)mt * BM;
  const int B = L.blocks_per_row;
  const int in = L.in_features;
  const int nk = B / 4;  // B % 16 == 0 (host contract): whole k-steps, whole index groups
  const uint32_t kmax = (uint32_t)(K - 1);

  stage_codebooks<S, LMODE, SEM, XDT>(lds_cb, ti.p, K, D);

  // dequantiser role: weight row wr_l, blocks 2 * wh + {0, 1} of every k-step
  const int wr_l = tid >> 1, wh = tid & 1;
  const bool w_row_ok = wr_l < ti.rows;
  const int64_t wr = ti.row0 + (w_row_ok ? wr_l : 0);
  const float rs_raw = w_row_ok ? load_f(ti.p.row_scale, D.sc_dtype, scale_index(L, wr)) : 0.0f;
  const RowScale rs = make_row_scale<XDT>(rs_raw);
  const IdT* idp[S];
#pragma unroll
  for (int s = 0; s < S; ++s) idp[s] = reinterpret_cast<const IdT*>(ti.p.ids[s]) + wr * B;

  // x loader role: piece p = tid + i * 512 -> row p / 4, 16-byte column p % 4
  const uint16_t* xrow[XP];
  bool xok[XP];
#pragma unroll
  for (int i = 0; i < XP; ++i) {
    const int p = tid + i * kPrefillThreads;
    const int64_t m = m0 + (p >> 2);
    xok[i] = m < M;
    xrow[i] = x + (xok[i] ? m : 0) * in + 8 * (p & 3);
  }

  u32x4_t xq[2][XP];           // x pieces of the next two k-steps
  u32x4_t idq[2][S][NV];       // index bytes of the current and next group of 4 k-steps
  auto load_x = [&](int k, u32x4_t (&dst)[XP]) {
#pragma unroll
    for (int i = 0; i < XP; ++i) dst[i] = xok[i] ? ldg128(xrow[i] + k * PBK) : u32x4_t{0, 0, 0, 0};
  };
  auto load_ids = [&](int grp, u32x4_t (&dst)[S][NV]) {
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int v = 0; v < NV; ++v) dst[s][v] = ldg128(reinterpret_cast<const uint8_t*>(idp[s] + grp * 16) + 16 * v);
  };
  auto store_x = [&](int buf, const u32x4_t (&src)[XP]) {
#pragma unroll
    for (int i = 0; i < XP; ++i) {
      const int p = tid + i * kPrefillThreads;
      *reinterpret_cast<u32x4_t*>(xs + (buf * BM + (p >> 2)) * PSTR + 8 * (p & 3)) = src[i];
    }
  };
  auto dequant = [&](int k, int buf, const u32x4_t (&ids)[S][NV]) {
    const int tstep = k & 3;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int t = 4 * tstep + 2 * wh + b;  // block inside the 16-block index group
      uint32_t id[S];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        uint32_t v;
        if constexpr (NV == 1) v = (ids[s][0][t >> 2] >> (8 * (t & 3))) & 0xffu;
        else v = (ids[s][t >> 3][(t >> 1) & 3] >> (16 * (t & 1))) & 0xffffu;
        id[s] = min(v, kmax);
      }
      u32x4_t w = make_wfrag<S, LMODE, SEM, XDT>(lds_cb, id, K, L.active_mask, rs);
      if (!w_row_ok) w = u32x4_t{0, 0, 0, 0};
      *reinterpret_cast<u32x4_t*>(ws + (buf * PBN + wr_l) * PSTR + 8 * (2 * wh + b)) = w;
    }
  };

  f32x4_t acc[TM][4];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // prologue: index group 0 (and 1), x of steps 0 and 1
  load_ids(0, idq[0]);
  if (nk > 4) load_ids(1, idq[1]);
  load_x(0, xq[0]);
  if (nk > 1) load_x(1, xq[1]);
  __syncthreads();  // codebooks staged
  dequant(0, 0, idq[0]);
  store_x(0, xq[0]);
  if (nk > 2) load_x(2, xq[0]);
  __syncthreads();

  const uint16_t* xa = xs + (wm * 16 * TM + l16) * PSTR + 8 * q;
  const uint16_t* wb = ws + (wn * 64 + l16) * PSTR + 8 * q;
  // Unrolled by 8 k-steps (two index groups) so that every register-array
  // index below is a compile-time constant: k0 is a multiple of 8, so the
  // buffer of step k is u & 1 and the index slot of group k / 4 is (u >> 2) & 1.
  for (int k0 = 0; k0 < nk; k0 += 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + u;
      if (k >= nk) break;  // uniform
      const int cur = u & 1;
      // MFMAs of step k (operands from buffer cur)
      u32x4_t b[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const u32x4_t*>(wb + (cur * PBN + j * 16) * PSTR);
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t*>(xa + (cur * BM + i * 16) * PSTR);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<XDT>(a, b[j], acc[i][j]);
      }
      // produce step k + 1 into buffer cur ^ 1 while the MFMAs run
      if (k + 1 < nk) {
        const int gs = ((u + 1) >> 2) & 1;  // index slot of group (k + 1) / 4
        dequant(k + 1, cur ^ 1, idq[gs]);
        store_x(cur ^ 1, xq[(u + 1) & 1]);
        if (k + 3 < nk) load_x(k + 3, xq[(u + 1) & 1]);
        // after the last step of a group is dequantised, the group two ahead
        // goes into its slot
        const int g = (k + 1) >> 2;
        if (((u + 1) & 3) == 3 && (g + 2) * 4 < nk) load_ids(g + 2, idq[gs]);
      }
      __syncthreads();
    }
  }

  // lane holds D[m = 4q + e][n = l16] of each 16 x 16 tile
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int nloc = wn * 64 + j * 16 + l16;
      if (nloc >= ti.rows) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t m = m0 + wm * 16 * TM + i * 16 + 4 * q + e;
        if (m < M) store_output(E, m, ti.out_row0 + nloc, acc[i][j][e]);
      }
    }
  }
}

template <int S, typename IdT, int LMODE, int SEM, int XDT, int TM>
static hipError_t prefill_tm(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, const void* x,
                             int64_t M, hipStream_t st) {
  const size_t lds = prefill_lds_bytes<S, LMODE>(TM, L.codebook_size);
  auto kern = rvq_prefill_kernel<S, IdT, LMODE, SEM, XDT, TM>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  const int n_mt = (int)((M + prefill_bm<TM>() - 1) / prefill_bm<TM>());
  dim3 grid((unsigned)(L.n_tiles * (int64_t)n_mt));
  hipLaunchKernelGGL(kern, grid, dim3(kPrefillThreads), lds, st, L, D, E, reinterpret_cast<const uint16_t*>(x), M,
                     n_mt);
  return hipGetLastError();
}

// One tile shape: 128 x-rows x 256 weight rows (TM = 4, a 64 x 64 tile per
// wave).  A 256-row x tile (TM = 8) would halve the LDS operand reads per MFMA
// but needs 128 accumulator registers per lane on top of the pipeline's ~100,
// more than the 256 a lane has at two waves per SIMD.
template <int S, typename IdT, int LMODE, int SEM, int XDT>
static hipError_t prefill_go(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, const void* x,
                             int64_t M, int n_cu, hipStream_t st) {
  (void)n_cu;
  return prefill_tm<S, IdT, LMODE, SEM, XDT, 4>(L, D, E, x, M, st);
}

template <int S, typename IdT, int XDT>
static hipError_t prefill_sem(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, int sem, int lmode,
                              const void* x, int64_t M, int n_cu, hipStream_t st) {
  if (sem == SEM_FAST) return prefill_go<S, IdT, LM_A16, SEM_FAST, XDT>(L, D, E, x, M, n_cu, st);
  if constexpr (S == 1) {
    return prefill_go<S, IdT, LM_A16, SEM_RECON, XDT>(L, D, E, x, M, n_cu, st);
  } else {
    if (lmode == LM_H16) return prefill_go<S, IdT, LM_H16, SEM_RECON, XDT>(L, D, E, x, M, n_cu, st);
    return prefill_go<S, IdT, LM_F32, SEM_RECON, XDT>(L, D, E, x, M, n_cu, st);
  }
}

// Entry for one (activation dtype, index width); explicitly instantiated in
// rvq_prefill_<x>_<ids>.hip.
template <int XDT, typename IdT>
hipError_t prefill_entry(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, int sem, int lmode,
                         const void* x, int64_t M, int n_cu, hipStream_t st) {
  switch (L.num_stages) {
    case 1: return prefill_sem<1, IdT, XDT>(L, D, E, sem, lmode, x, M, n_cu, st);
    case 2: return prefill_sem<2, IdT, XDT>(L, D, E, sem, lmode, x, M, n_cu, st);
    case 3: return prefill_sem<3, IdT, XDT>(L, D, E, sem, lmode, x, M, n_cu, st);
    default: return prefill_sem<4, IdT, XDT>(L, D, E, sem, lmode, x, M, n_cu, st);
  }
}

}  // namespace wal
