// rvq_decode_impl.h -- Block-RVQ linear for M <= 16 (decode), block_size 8.
//
// The weight is never written to memory.  Layout of the work:
//   * A workgroup of NW waves is persistent over a contiguous range of
//     16-row tiles.  It keeps the codebooks of the current row group in LDS
//     (restaged only when the tile's group changes) and, when it fits, the
//     activation rows x[0..M) as well.
//   * Within a tile the row's 64-block chunks are dealt to the waves: wave w
//     takes chunks w, w + NW, ...; every wave takes the same number CPT of
//     chunk slots per tile (a slot past the last chunk contributes zero), so
//     the sequence of (tile, slot) items is the same length for every wave
//     and the per-tile barriers are uniform.
//   * Lane l covers weight row n = l % 16 and the 16 consecutive blocks
//     [64c + 16q, 64c + 16q + 16), q = l / 16: one 128-bit load per stage for
//     8-bit ids, two for 16-bit ids.  Those loads run PF items ahead of the
//     compute, across tile boundaries (a ring of PF register slots).
//   * For each of the 16 blocks the lane gathers the S codewords from LDS,
//     rebuilds the 8 weights exactly as the reference's dequantisation does
//     (rvq_fragment.h) and feeds them as the B operand of
//     v_mfma_f32_16x16x32_{bf16,f16}; the A operand is x[min(l % 16, M - 1)] at
//     the same 8 columns (rows m >= M of the product are never stored).
//   * The NW partial 16x16 accumulators of a tile are summed through LDS and
//     the M x 16 outputs written once.
#pragma once

#include "rvq_fragment.h"

namespace wal {

constexpr int kDecodeWaves = 4;
constexpr int kDecodeThreads = kDecodeWaves * 64;

// Items of index loads in flight per wave: about 128 bytes per lane.
template <int S, typename IdT>
constexpr int decode_prefetch() {
  constexpr int w = S * (int)sizeof(IdT);
  return w <= 2 ? 4 : (w <= 4 ? 2 : 1);
}

template <typename IdT>
WAL_DEVICE uint32_t extract_id(const u32x4_t (&v)[sizeof(IdT)], int t) {
  if constexpr (sizeof(IdT) == 1) {
    return (v[0][t >> 2] >> (8 * (t & 3))) & 0xffu;
  } else {
    return (v[t >> 3][(t >> 1) & 3] >> (16 * (t & 1))) & 0xffffu;
  }
}

// Bytes of LDS a decode launch needs (codebooks + reduction buffer + x).
template <int LMODE>
WAL_HOST_DEVICE size_t decode_lds_bytes(int S, int K, bool xlds, int M, int in) {
  return (size_t)S * K * lds_entry_bytes<LMODE>() + 2 * kDecodeWaves * 256 * sizeof(float) +
         (xlds ? (size_t)M * in * sizeof(uint16_t) : 0);
}

template <int S, typename IdT, int LMODE, int SEM, int XDT, bool XLDS>
__global__ __launch_bounds__(kDecodeThreads) void rvq_decode_kernel(LayerArgs L, DtypeArgs D, EpilogueArgs E,
                                                                    const uint16_t* __restrict__ x, int M) {
  constexpr int NW = kDecodeWaves, PF = decode_prefetch<S, IdT>(), NV = sizeof(IdT);
  constexpr int ESZ = lds_entry_bytes<LMODE>();
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int K = L.codebook_size;
  const int B = L.blocks_per_row;
  const int in = L.in_features;
  uint8_t* lds_cb = smem;
  float* red = reinterpret_cast<float*>(smem + (size_t)S * K * ESZ);  // [2][NW][256]
  uint16_t* xs = reinterpret_cast<uint16_t*>(red + 2 * NW * 256);    // [M][in] when XLDS

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nl = lane & 15;
  const int q = lane >> 4;
  const int nchunk = (B + 63) >> 6;
  const int CPT = (nchunk + NW - 1) / NW;
  const int T = L.n_tiles;
  const int t_begin = (int)((int64_t)blockIdx.x * T / gridDim.x);
  const int n_tiles_wg = (int)((int64_t)(blockIdx.x + 1) * T / gridDim.x) - t_begin;
  const int n_items = n_tiles_wg * CPT;
  const uint32_t kmax = (uint32_t)(K - 1);
  const int xm = min(nl, M - 1);  // x row this lane feeds to the MFMA

  if constexpr (XLDS) {
    const int n16 = M * in / 8;  // in % 128 == 0
    for (int i = tid; i < n16; i += kDecodeThreads)
      reinterpret_cast<u32x4_t*>(xs)[i] = ldg128(x + (size_t)i * 8);
    // the first codebook staging below ends with a barrier before any read
  }

  // ---- index prefetch ring (issue cursor runs PF items ahead) -------------
  u32x4_t ring[PF][S][NV];
  int is_t = 0, is_c = 0;  // issue cursor: tile offset within the range, chunk slot
  FragTile<S> iti = get_frag_tile<S>(L, t_begin < T ? t_begin : 0);
  auto issue = [&](u32x4_t (&dst)[S][NV]) {
    const int c = wave + NW * is_c;
    const int base = c * 64 + 16 * q;
    const bool ok = is_t < n_tiles_wg && c < nchunk && base < B && nl < iti.rows;
    const int64_t r = iti.row0 + nl;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const IdT* p = reinterpret_cast<const IdT*>(iti.p.ids[s]) + r * B + base;
#pragma unroll
      for (int v = 0; v < NV; ++v) dst[s][v] = ok ? ldg128_stream(p + v * (16 / NV)) : u32x4_t{0, 0, 0, 0};
    }
    if (++is_c == CPT) {
      is_c = 0;
      ++is_t;
      if (is_t < n_tiles_wg) iti = get_frag_tile<S>(L, t_begin + is_t);
    }
  };
#pragma unroll
  for (int j = 0; j < PF; ++j) issue(ring[j]);

  // ---- compute ------------------------------------------------------------
  int staged = -1;
  int buf = 0;
  int ct_t = 0, ct_c = 0;  // compute cursor
  FragTile<S> cti = iti;
  RowScale rs = make_row_scale<XDT>(0.0f);
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int i0 = 0; i0 < n_items; i0 += PF) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      if (i0 + j >= n_items) break;  // uniform across the workgroup
      if (ct_c == 0) {
        cti = get_frag_tile<S>(L, t_begin + ct_t);
        if (cti.group != staged) {
          __syncthreads();  // every wave is done with the previous codebooks
          stage_codebooks<S, LMODE, SEM, XDT>(lds_cb, cti.p, K, D);
          __syncthreads();
          staged = cti.group;
        }
        const bool row_ok = nl < cti.rows;
        const float rs_raw = row_ok ? load_f(cti.p.row_scale, D.sc_dtype, (cti.row0 + nl) / L.scale_rows) : 0.0f;
        rs = make_row_scale<XDT>(rs_raw);
        acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      }
      const int c = wave + NW * ct_c;
      const int base = c * 64 + 16 * q;
      if (c < nchunk) {  // uniform across the wave
        // activations: zero for blocks past the row (base >= B)
        const bool seg_ok = base < B;
        u32x4_t xf[16];
#pragma unroll
        for (int tt = 0; tt < 16; ++tt) {
          const int64_t off = (int64_t)xm * in + (int64_t)(base + tt) * 8;
          if constexpr (XLDS) xf[tt] = seg_ok ? *reinterpret_cast<const u32x4_t*>(xs + off) : u32x4_t{0, 0, 0, 0};
          else xf[tt] = seg_ok ? ldg128(x + off) : u32x4_t{0, 0, 0, 0};
        }
#pragma unroll
        for (int tt = 0; tt < 16; ++tt) {
          uint32_t id[S];
#pragma unroll
          for (int s = 0; s < S; ++s) id[s] = min(extract_id<IdT>(ring[j][s], tt), kmax);
          // rows past the tile hold a zero scale; their products are not stored
          const u32x4_t w = make_wfrag<S, LMODE, SEM, XDT>(lds_cb, id, K, L.active_mask, rs);
          acc = mfma16<XDT>(xf[tt], w, acc);
        }
      }
      issue(ring[j]);  // refill this slot with the item PF ahead
      if (++ct_c == CPT) {
        // tile done: sum the NW partial accumulators, store M x 16 outputs
        ct_c = 0;
        float* rb = red + (size_t)buf * NW * 256 + wave * 256;
#pragma unroll
        for (int e = 0; e < 4; ++e) rb[(4 * q + e) * 16 + nl] = acc[e];  // lane holds D[4q + e][nl]
        __syncthreads();
        if (tid < M * 16) {
          const int m = tid >> 4;
          const int n = tid & 15;
          const float* rr = red + (size_t)buf * NW * 256 + tid;
          float v = 0.0f;
#pragma unroll
          for (int w = 0; w < NW; ++w) v += rr[w * 256];
          if (n < cti.rows) store_output(E, m, cti.out_row0 + n, v);
        }
        buf ^= 1;
        ++ct_t;
      }
    }
  }
}

template <int S, typename IdT, int LMODE, int SEM, int XDT>
static hipError_t decode_go(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, const void* x, int M,
                            int n_cu, hipStream_t st) {
  constexpr int kLdsMax = 160 * 1024;
  const bool xlds = decode_lds_bytes<LMODE>(S, L.codebook_size, true, M, L.in_features) <= (size_t)kLdsMax;
  const size_t lds = decode_lds_bytes<LMODE>(S, L.codebook_size, xlds, M, L.in_features);
  auto kern = xlds ? rvq_decode_kernel<S, IdT, LMODE, SEM, XDT, true> : rvq_decode_kernel<S, IdT, LMODE, SEM, XDT, false>;
  static bool attr_set[2] = {false, false};
  if (!attr_set[xlds]) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       kLdsMax);
    if (e != hipSuccess) return e;
    attr_set[xlds] = true;
  }
  int per_cu = (int)(kLdsMax / lds);
  if (per_cu > 4) per_cu = 4;
  if (per_cu < 1) per_cu = 1;
  int grid = n_cu * per_cu;
  if (grid > L.n_tiles) grid = L.n_tiles;
  if (grid < 1) return hipSuccess;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kDecodeThreads), lds, st, L, D, E, reinterpret_cast<const uint16_t*>(x), M);
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
