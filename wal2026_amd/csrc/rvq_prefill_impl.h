// rvq_prefill_impl.h -- Block-RVQ linear for large M (prefill), block_size 8.
//
// Workgroup tile: BM = 32 * TM activation rows x 256 weight rows (tile kind 2),
// k-step 32 columns (4 blocks).  512 threads = 8 waves in a 2 (M) x 4 (N)
// arrangement; a wave owns 16 TM x 64 outputs = TM x 4 tiles of
// v_mfma_f32_16x16x32_{bf16,f16}.  Per k-step every thread
//   * dequantises 2 blocks (16 weights) of one weight row from the LDS
//     codebooks with the reference's exact rounding (rvq_fragment.h) into the
//     W tile in LDS, in the MFMA input dtype, and
//   * copies one or two 16-byte pieces of x (the tile is BM rows x 64 bytes)
//     into the x tile in LDS.
// Pipeline (iteration k): the MFMAs of step k run on operand fragments
// already in registers while the fragments of step k + 1 are read from LDS
// buffer (k + 1) & 1 and step k + 2 is dequantised into buffer k & 1, whose
// fragments every wave read before the previous barrier; one barrier per
// step.  x is loaded four steps ahead, index bytes (16 blocks = 4 steps per
// load) a group ahead.  Loads are unconditional buffer loads (out-of-range
// offsets read zeros), so a step is one basic block and the compiler's load
// counters stay exact.
//
// LDS rows are 96 bytes apart: a 16 x 16 fragment read (lane l: row l % 16,
// 16-byte chunk l / 16) is then conflict-free on gfx950's 64-bank LDS, which
// serves lanes 0-7 with 16-23 (and so on) in one cycle; an 80-byte stride
// measures 2-way conflicted.  The codebook table is replicated (as many
// copies as LDS holds, up to 8) so lanes gathering in the same cycle mostly
// hit different copies.
//
// Measured on gfx950: the dequantisation arithmetic does not overlap the
// MFMAs of the same SIMD (their costs add), so the kernel's rate is set by
// the VALU work per weight (about four full-rate instructions per element)
// amortised over the BM rows that use it.
//
// Grid: the x-row tile index varies fastest, so consecutive workgroups (which
// the dispatcher deals round-robin to the XCDs) share one weight tile and each
// XCD keeps revisiting the same few x tiles in its L2.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <cstring>

#include "rvq_fragment.h"

namespace wal {

constexpr int kConsumerWaves = 8;   // MFMA waves
constexpr int kProducerWaves = 8;   // dequantisation and x-copy waves
constexpr int kPrefillThreads = (kConsumerWaves + kProducerWaves) * 64;
constexpr int kProducerThreads = kProducerWaves * 64;
constexpr int PBN = 256;        // weight rows per workgroup tile
constexpr int PBK = 32;         // k per step
constexpr int PSTR = PBK + 16;  // elements per LDS row (96 bytes; see below)

template <int TM>
constexpr int prefill_bm() { return 32 * TM; }

// Staged table entries: S tables of K entries back to back, plus, for 8-bit
// indices and K < 256, the 256 - K entries that keep any index byte of the
// last stage inside the allocation (8-bit ids are not clamped).
template <int S, typename IdT>
WAL_HOST_DEVICE int prefill_table_entries(int K) {
  return S * K + ((sizeof(IdT) == 1 && K < 256) ? 256 - K : 0);
}

template <int TM>
WAL_HOST_DEVICE size_t prefill_tile_bytes() {
  return (size_t)2 * (32 * TM + PBN) * PSTR * sizeof(uint16_t);
}

// LDS of a launch whose codebook table is replicated 1 << rshift times.
template <int S, typename IdT, int LMODE>
WAL_HOST_DEVICE size_t prefill_lds_bytes(int TM, int K, int rshift) {
  return (TM == 8 ? prefill_tile_bytes<8>() : prefill_tile_bytes<4>()) +
         ((size_t)prefill_table_entries<S, IdT>(K) * lds_entry_bytes<LMODE>() << rshift);
}


// Split-K: ksplit > 1 workgroups share one output tile, each over a slice of
// the k-steps (whole units of kSplitUnit steps, so that every slice starts on
// an index group and the register slots of the unrolled producer loop keep
// their compile-time indices), and write fp32 partial sums to part
// [ksplit][M][out_features]; rvq_splitk_reduce_kernel sums them in slice
// order (deterministic) and applies the epilogue.
constexpr int kSplitUnit = 8;

template <int S, typename IdT, int LMODE, int SEM, int XDT, int TM>
__global__ __launch_bounds__(kPrefillThreads) void rvq_prefill_kernel(LayerArgs L, DtypeArgs D, EpilogueArgs E,
                                                                      const uint16_t* __restrict__ x, int64_t M,
                                                                      int n_mt, int rshift, int ksplit,
                                                                      float* __restrict__ part) {
  constexpr int BM = prefill_bm<TM>();
  constexpr int XP = BM * 4 / kProducerThreads;  // 16-byte x pieces per producer thread per k-step
  constexpr int BPT = PBN * 4 / kProducerThreads;  // blocks each producer thread dequantises per k-step
  constexpr int NV = sizeof(IdT);                  // 16-byte index loads per stage per group of 4 k-steps
  static_assert(XP >= 1 && BM * 4 % kProducerThreads == 0, "x tile split");
  static_assert(BPT == 2, "two producer threads per weight row");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);  // [2][BM][PSTR]
  uint16_t* ws = xs + 2 * BM * PSTR;                 // [2][PBN][PSTR]
  uint8_t* lds_cb = reinterpret_cast<uint8_t*>(ws + 2 * PBN * PSTR);

  const int K = L.codebook_size;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int mt = (int)(blockIdx.x % (unsigned)n_mt);
  const int rest = (int)(blockIdx.x / (unsigned)n_mt);
  const int ks = rest % ksplit;  // k slice of this workgroup
  const int nt = rest / ksplit;
  const FragTile<S> ti = get_frag_tile<S>(L, nt);
  const int64_t m0 = (int64_t)mt * BM;
  const int B = L.blocks_per_row;
  const int in = L.in_features;
  const int nk_all = B / 4;  // B % 16 == 0 (host contract): whole k-steps, whole index groups
  // this slice's k-steps [kb, nk): the host gives every slice at least one unit
  const int nu = (nk_all + kSplitUnit - 1) / kSplitUnit;
  const int kb = kSplitUnit * (int)((int64_t)ks * nu / ksplit);
  const int nk = min(nk_all, kSplitUnit * (int)((int64_t)(ks + 1) * nu / ksplit));
  const uint32_t kmax = (uint32_t)(K - 1);

  // Codebook table, replicated 1 << rshift times (host choice: as many
  // copies, up to 8, as LDS holds): staged compactly into the idle W tile
  // area, then spread into the replicated layout.  All waves take part.
  constexpr int ESZ = lds_entry_bytes<LMODE>();
  if (rshift == 0) {
    stage_codebooks<S, LMODE, SEM, XDT>(lds_cb, ti.p, K, D);
  } else {
    uint8_t* compact = reinterpret_cast<uint8_t*>(ws);
    stage_codebooks<S, LMODE, SEM, XDT>(compact, ti.p, K, D);
    __syncthreads();
    const int n16 = prefill_table_entries<S, IdT>(K) * (ESZ / 16);  // 16-byte pieces
    const int nc = 1 << rshift;
    for (int i = tid; i < n16 * nc; i += kPrefillThreads) {
      const int piece = i >> rshift, c = i & (nc - 1);
      const int e = piece / (ESZ / 16), h = piece - e * (ESZ / 16);
      *reinterpret_cast<u32x4_t*>(lds_cb + (((e << rshift) + c) * ESZ) + 16 * h) =
          *reinterpret_cast<const u32x4_t*>(compact + (size_t)piece * 16);
    }
  }
  __syncthreads();  // table staged (and the compact copy in the W area read)

  if (wave < kConsumerWaves) {
    // ---- consumers: 8 waves (2 per SIMD, the pair that keeps the matrix
    // core busy), 2 (M) x 4 (N), each a 16 TM x 64 output tile ----
    const int wm = wave >> 2, wn = wave & 3;
    const int l16 = lane & 15, q = lane >> 4;
    const uint16_t* xa = xs + (wm * 16 * TM + l16) * PSTR + 8 * q;
    const uint16_t* wb = ws + (wn * 64 + l16) * PSTR + 8 * q;
    f32x4_t acc[TM][4];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    __syncthreads();  // step kb produced
    for (int k = kb; k < nk; ++k) {
      const int buf = k & 1;
      u32x4_t a[TM], b[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const u32x4_t*>(wb + (buf * PBN + j * 16) * PSTR);
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = *reinterpret_cast<const u32x4_t*>(xa + (buf * BM + i * 16) * PSTR);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<XDT>(a[i], b[j], acc[i][j]);
      __syncthreads();  // buffer buf read; step k + 1 produced
    }
    // lane holds D[m = 4q + e][n = l16] of each 16 x 16 tile.  (Two loops,
    // not a branch per element: a larger unrolled body would leave acc
    // dynamically indexed, in scratch memory.)
    if (ksplit > 1) {
      float* pk = part + (size_t)ks * (size_t)M * (size_t)E.ldy + ti.out_row0;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int nloc = wn * 64 + j * 16 + l16;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int64_t m = m0 + wm * 16 * TM + i * 16 + 4 * q + e;
            if (m < M && nloc < ti.rows) pk[m * E.ldy + nloc] = acc[i][j][e];
          }
        }
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int nloc = wn * 64 + j * 16 + l16;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t m = m0 + wm * 16 * TM + i * 16 + 4 * q + e;
          if (m < M && nloc < ti.rows) store_output(E, m, ti.out_row0 + nloc, acc[i][j][e]);
        }
      }
    }
    return;
  }

  // ---- producers: 8 waves (two per SIMD, running beside the MFMAs of the
  // two consumer waves there); threads pt = 2r, 2r + 1 own weight row r,
  // blocks 2 (pt & 1) + {0, 1} of every k-step ----
  const int pt = tid - kConsumerWaves * 64;
  const int prow = pt >> 1, ph = pt & 1;
  const uint8_t* lds_lane = lds_cb + (lane & ((1 << rshift) - 1)) * ESZ;  // this lane's table copy
  // Rows past the tile dequantise the tile's first row; their outputs are
  // never stored.
  const int64_t wr = ti.row0 + (prow < ti.rows ? prow : 0);
  const RowScale rs = make_row_scale<XDT>(load_f(ti.p.row_scale, D.sc_dtype, scale_index(L, wr)));
  // index planes: one descriptor per stage on the group's base (uniform; a
  // per-lane base would make the compiler loop over the lanes' descriptors),
  // the row in the per-lane offset (rows * B * sizeof(IdT) < 2^31, host check)
  bufrsrc_t idr[S];
#pragma unroll
  for (int s = 0; s < S; ++s) idr[s] = make_rsrc(ti.p.ids[s]);
  const uint32_t idrow = (uint32_t)(wr * B * (int64_t)sizeof(IdT));
  // x pieces p = pt + i * 256 -> row p / 4, 16-byte column p % 4, addressed
  // from the tile's first row (rows past M read zeros)
  const bufrsrc_t xr = make_rsrc(x + m0 * in);
  uint32_t xoff[XP];
#pragma unroll
  for (int i = 0; i < XP; ++i) {
    const int p = pt + i * kProducerThreads;
    xoff[i] = m0 + (p >> 2) < M ? (uint32_t)(((p >> 2) * in + 8 * (p & 3)) * 2) : kBufOOB;
  }
  // Loads are unconditional (a step or group past the end gets an
  // out-of-range offset and reads zeros), so a step is one basic block and
  // the compiler's load counters stay exact.
  auto load_x = [&](int k, u32x4_t (&dst)[XP]) {
    const uint32_t step = k < nk ? (uint32_t)(k * PBK * 2) : kBufOOB;
#pragma unroll
    for (int i = 0; i < XP; ++i) dst[i] = ldbuf128(xr, xoff[i] == kBufOOB ? kBufOOB : xoff[i] + step);
  };
  auto load_ids = [&](int grp, u32x4_t (&dst)[S][NV]) {
    const uint32_t off = grp * 4 < nk ? idrow + (uint32_t)(grp * 16 * NV) : kBufOOB;
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int v = 0; v < NV; ++v) dst[s][v] = ldbuf128(idr[s], off == kBufOOB ? kBufOOB : off + 16 * v);
  };
  // step k: the thread's 2 blocks into W buffer buf, x pieces into x buffer buf
  auto produce = [&](int k, int buf, const u32x4_t (&ids)[S][NV], const u32x4_t (&xv)[XP]) {
    WfragRaw<S, LMODE> raw[BPT];
#pragma unroll
    for (int b = 0; b < BPT; ++b) {
      const int t = 4 * (k & 3) + 2 * ph + b;  // block inside the 16-block index group
      uint32_t id[S];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        if constexpr (NV == 1) {
          id[s] = (ids[s][0][t >> 2] >> (8 * (t & 3))) & 0xffu;  // inside the allocation
        } else {
          id[s] = min((ids[s][t >> 3][(t >> 1) & 3] >> (16 * (t & 1))) & 0xffffu, kmax);
        }
      }
      raw[b] = gather_wfrag_rep<S, LMODE>(lds_lane, id, K, rshift);
    }
    uint16_t* wd = ws + (buf * PBN + prow) * PSTR + 16 * ph;
#pragma unroll
    for (int b = 0; b < BPT; ++b)
      *reinterpret_cast<u32x4_t*>(wd + 8 * b) = combine_wfrag<S, LMODE, SEM, XDT>(raw[b], L.active_mask, rs);
#pragma unroll
    for (int i = 0; i < XP; ++i) {
      const int p = pt + i * kProducerThreads;
      *reinterpret_cast<u32x4_t*>(xs + (buf * BM + (p >> 2)) * PSTR + 8 * (p & 3)) = xv[i];
    }
  };

  u32x4_t xq[4][XP];      // x pieces of steps k + 1 .. k + 4 (slot = step & 3)
  u32x4_t idq[2][S][NV];  // index bytes of two groups of 4 k-steps (slot = group & 1)
  // (kb is a multiple of 8: the slots below are those of steps 0 .. 4 of an
  // unsplit launch)
  load_ids(kb / 4, idq[0]);
  load_ids(kb / 4 + 1, idq[1]);
#pragma unroll
  for (int j = 0; j < 4; ++j) load_x(kb + j, xq[j]);
  produce(kb, 0, idq[0], xq[0]);
  load_x(kb + 4, xq[0]);
  __syncthreads();  // step kb produced
  // Iteration k produces step k + 1 into buffer (k + 1) & 1 (read by the
  // consumers in iteration k - 1, before the previous barrier).  Unrolled by
  // 8 so that register-array indices are compile-time constants (k0 is a
  // multiple of 8): step k + 1 uses x slot (u + 1) & 3 and index slot
  // ((u + 1) >> 2) & 1; x runs four steps ahead, index bytes a group ahead.
  for (int k0 = kb; k0 < nk; k0 += 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + u;
      if (k >= nk) break;  // uniform
      const int gs = ((u + 1) >> 2) & 1;
      produce(k + 1, (u + 1) & 1, idq[gs], xq[(u + 1) & 3]);  // past the end: harmless
      load_x(k + 5, xq[(u + 1) & 3]);
      // once the last step of a group is produced, the group two ahead goes
      // into its slot
      if (((u + 1) & 3) == 3) load_ids(((k + 1) >> 2) + 2, idq[gs]);
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------------------
// Tall tile: 256 x-rows x 256 weight rows, 8 waves (two per SIMD, up to 256
// registers per lane), every wave both dequantising and multiplying.
//
// Each dequantised weight feeds 256 MFMA rows, so the dequantisation work per
// flop is half that of a 128-row tile.  Per k-step (32 columns = 4 blocks):
//   * wave (wm, wn) of 2 (M) x 4 (N) multiplies its 128 x 64 output tile with
//     v_mfma_f32_32x32x16 products (4 row blocks x 2 column blocks per k
//     half): the four W fragments and eight x fragments come from LDS buffer
//     k & 1; all products of the first k half come before those of the
//     second, so the two that accumulate into one tile are 8 apart;
//   * thread t dequantises blocks 2 (t & 1) and 2 (t & 1) + 1 of weight row
//     t / 2 (bits 2 and 3 of t / 2 swapped, see the bank note below) for step
//     k + 1 into W buffer (k + 1) & 1, and copies 2 of the x tile's 1024
//     16-byte pieces.
// The two waves of a SIMD hide each other's LDS and global latencies.
// Measured on gfx950 against the alternatives: one dequantising wave beside
// two multiplying waves per SIMD left the multiplying waves at the barrier
// more than half the time (the dequantising wave's serial chain set the
// step); one wave per SIMD with the weights dequantised straight into MFMA
// registers (no W tile in LDS) lost more to exposed latency than it saved in
// LDS traffic.  The 32 x 32 product keeps the matrix core busy twice as long
// per operand read as the 16 x 16 one, and a VALU instruction of the same
// SIMD takes less of its time (about 1.3 cycles against 3, measured).
//
// LDS rows are 64 bytes (one k-step of 16-bit values) with the 16-byte chunk
// c of row r stored at chunk c ^ f(r), f(r) = bit 2 of r + 2 * bit 4 of r:
// the fragment reads (lane l: row l % 32, chunk 2 h + l / 32) then run at the
// rate of sequential reads (measured), and the W and x writes (2 and 4 lanes
// per row) at the rate of sequential writes.
// ---------------------------------------------------------------------------
constexpr int kTallWaves = 8;
constexpr int kTallThreads = kTallWaves * 64;
constexpr int TBM = 256;                  // x rows per workgroup tile
constexpr int kTallRowBytes = PBK * 2;    // 64
constexpr int kTallTileBytes = 256 * kTallRowBytes;  // one 256-row operand tile (16 KB)

WAL_HOST_DEVICE constexpr int tall_swz(int row, int chunk) { return (chunk ^ ((row >> 1) & 3)) * 16; }
WAL_HOST_DEVICE constexpr int tall_swz32(int row, int chunk) {
  return (chunk ^ (((row >> 2) & 1) | ((row >> 3) & 2))) * 16;
}

template <int S, typename IdT, int LMODE>
WAL_HOST_DEVICE size_t prefill_tall_lds_bytes(int K, int rshift) {
  return (size_t)4 * kTallTileBytes + ((size_t)prefill_table_entries<S, IdT>(K) * lds_entry_bytes<LMODE>() << rshift);
}

// Instances whose registers fit 256 per lane without scratch (checked with the
// compiler's resource report).
template <int S, typename IdT, int LMODE>
constexpr bool tall_supported() {
  return prefill_tall_ok(S, LMODE);
}

// One tall workgroup's k-loop and epilogue over NB * 128 weight rows of a
// tile (NB = 2: the whole 256-row tile; NB = 1: the half starting at row
// wrow0).  Wave (wm, wn) multiplies x rows 128 wm .. + 128 by weight rows
// 32 NB wn .. + 32 NB; thread t dequantises NB of the 4 blocks of one weight
// row per k-step.  The table is staged and smem holds [2][x tile] [2][W tile]
// [table].
template <int S, typename IdT, int LMODE, int SEM, int XDT, int NB>
WAL_DEVICE void tall_tile(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E,
                          const uint16_t* __restrict__ x, int64_t M, const FragTile<S>& ti, int64_t m0, int wrow0,
                          int rshift, uint8_t* smem) {
  constexpr int XP = TBM * 4 / kTallThreads;  // 2 x pieces per thread per k-step
  constexpr int NV = sizeof(IdT);             // 16-byte index loads per stage per group of 4 k-steps
  constexpr int TPR = 4 / NB;                 // threads per weight row
  uint8_t* xs = smem;                          // [2][256 rows][64 B]
  uint8_t* ws = smem + 2 * kTallTileBytes;     // [2][256 rows][64 B] (NB * 128 rows used)
  uint8_t* lds_cb = smem + 4 * kTallTileBytes;
  const int K = L.codebook_size;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int B = L.blocks_per_row;
  const int in = L.in_features;
  const int nk = B / 4;  // B % 16 == 0 (host contract): whole k-steps, whole index groups
  const uint32_t kmax = (uint32_t)(K - 1);
  constexpr int ESZ = lds_entry_bytes<LMODE>();

  // ---- dequantisation and x copy: thread tid, weight row pr, blocks
  // NB (tid % TPR) .. + NB of every k-step.  Lanes 0-7 and 16-23 (one LDS
  // write cycle) get rows r0 .. r0 + 3: bits 2 and 3 (NB = 2) or 1 and 2
  // (NB = 1) of the row index are swapped ----
  const int q2 = tid / TPR, ph = tid % TPR;
  const int pr = NB == 2 ? (q2 & ~12) | ((q2 & 4) << 1) | ((q2 & 8) >> 1) : (q2 & ~6) | ((q2 & 2) << 1) | ((q2 & 4) >> 1);
  const uint8_t* lds_lane = lds_cb + (lane & ((1 << rshift) - 1)) * ESZ;  // this lane's table copy
  // Rows past the tile dequantise the tile's first row; their outputs are
  // never stored.
  const int64_t wr = ti.row0 + (wrow0 + pr < ti.rows ? wrow0 + pr : 0);
  const RowScale rs = make_row_scale<XDT>(load_f(ti.p.row_scale, D.sc_dtype, scale_index(L, wr)));
  // index planes: one descriptor per stage on the group's base (uniform), the
  // row in the per-lane offset (rows * B * sizeof(IdT) < 2^31, host check)
  bufrsrc_t idr[S];
#pragma unroll
  for (int s = 0; s < S; ++s) idr[s] = make_rsrc(ti.p.ids[s]);
  const uint32_t idrow = (uint32_t)(wr * B * (int64_t)sizeof(IdT));
  // x piece p = tid + i * 512: 16-byte chunk p % 4 of row q = p / 4 with bits
  // 1 and 2 of q swapped; rows past M read zeros
  const bufrsrc_t xr = make_rsrc(x + m0 * in);
  uint32_t xoff[XP];
  int xdst[XP];
#pragma unroll
  for (int i = 0; i < XP; ++i) {
    const int p = tid + i * kTallThreads;
    const int q = p >> 2, c = p & 3;
    const int r = (q & ~6) | ((q & 2) << 1) | ((q & 4) >> 1);
    xoff[i] = m0 + r < M ? (uint32_t)((r * in + 8 * c) * 2) : kBufOOB;
    xdst[i] = r * kTallRowBytes + tall_swz32(r, c);
  }
  uint8_t* wd = ws + pr * kTallRowBytes;
  int wsw[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) wsw[b] = tall_swz32(pr, NB * ph + b);
  // Loads are unconditional (a step or group past the end gets an
  // out-of-range offset and reads zeros), so a step is one basic block.
  auto load_x = [&](int k, u32x4_t (&dst)[XP]) {
    const uint32_t step = k < nk ? (uint32_t)(k * PBK * 2) : kBufOOB;
#pragma unroll
    for (int i = 0; i < XP; ++i) dst[i] = ldbuf128(xr, xoff[i] == kBufOOB ? kBufOOB : xoff[i] + step);
  };
  auto load_ids = [&](int grp, u32x4_t (&dst)[S][NV]) {
    const uint32_t off = grp * 4 < nk ? idrow + (uint32_t)(grp * 16 * NV) : kBufOOB;
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int v = 0; v < NV; ++v) dst[s][v] = ldbuf128(idr[s], off == kBufOOB ? kBufOOB : off + 16 * v);
  };
  // the codewords of this thread's blocks of step k (index group ids)
  auto gather = [&](int k, const u32x4_t (&ids)[S][NV], WfragRaw<S, LMODE> (&raw)[NB]) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int t = 4 * (k & 3) + NB * ph + b;  // block inside the 16-block index group
      uint32_t id[S];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        if constexpr (NV == 1) {
          id[s] = (ids[s][0][t >> 2] >> (8 * (t & 3))) & 0xffu;  // inside the allocation
        } else {
          id[s] = min((ids[s][t >> 3][(t >> 1) & 3] >> (16 * (t & 1))) & 0xffffu, kmax);
        }
      }
      raw[b] = gather_wfrag_rep<S, LMODE>(lds_lane, id, K, rshift);
    }
  };
  // the weights of the thread's blocks and the x pieces of one step into buffer buf
  auto put = [&](int buf, const WfragRaw<S, LMODE> (&raw)[NB], const u32x4_t (&xv)[XP]) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
      *reinterpret_cast<u32x4_t*>(wd + buf * kTallTileBytes + wsw[b]) =
          combine_wfrag<S, LMODE, SEM, XDT>(raw[b], L.active_mask, rs);
#pragma unroll
    for (int i = 0; i < XP; ++i) *reinterpret_cast<u32x4_t*>(xs + buf * kTallTileBytes + xdst[i]) = xv[i];
  };

  // ---- multiplication: wave (wm, wn), a 128 x 32 NB output tile ----
  const int wm = wave >> 2, wn = wave & 3;
  const int l32 = lane & 31, hk = lane >> 5;
  // fragment rows start at multiples of 32, so the swizzle of row l32 is that
  // of every fragment's row
  const uint8_t* xa = xs + (wm * 128 + l32) * kTallRowBytes;
  const uint8_t* wb = ws + (wn * 32 * NB + l32) * kTallRowBytes;
  const int sw0 = tall_swz32(l32, hk), sw1 = tall_swz32(l32, 2 + hk);  // k halves 0 and 1
  f32x16_t acc[4][NB];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
  auto multiply = [&](int buf) {
    const int bo = buf * kTallTileBytes;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int sw = h ? sw1 : sw0;
      u32x4_t bw[NB];
#pragma unroll
      for (int j = 0; j < NB; ++j) bw[j] = *reinterpret_cast<const u32x4_t*>(wb + bo + j * 32 * kTallRowBytes + sw);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t*>(xa + bo + i * 32 * kTallRowBytes + sw);
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = mfma32<XDT>(a, bw[j], acc[i][j]);
      }
    }
  };

  // ---- pipeline: iteration k multiplies step k (buffer k & 1) and produces
  // step k + 1 into buffer (k + 1) & 1, which every wave finished reading in
  // iteration k - 1, before the previous barrier; one barrier per step.  x
  // runs four steps ahead (slot = step & 3), index bytes a group ahead (idc:
  // the group of the step being produced, idn: the next one).  The loop
  // takes one index group (4 steps) per trip, so every register-array index
  // is a constant. ----
  u32x4_t xq[4][XP];
  u32x4_t idc[S][NV], idn[S][NV];
  WfragRaw<S, LMODE> raw[NB];
  load_ids(0, idc);
  load_ids(1, idn);
#pragma unroll
  for (int j = 0; j < 4; ++j) load_x(j, xq[j]);
  gather(0, idc, raw);
  put(0, raw, xq[0]);
  load_x(4, xq[0]);
  __syncthreads();  // step 0 produced
  for (int g = 0; g < nk / 4; ++g) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int k = 4 * g + u;
      // step k + 1 is in group g (u < 3) or g + 1 (u == 3); past the end it
      // reads zeros and writes a buffer nobody reads
      if (u < 3) gather(k + 1, idc, raw);
      else gather(k + 1, idn, raw);
      multiply(u & 1);
      put((u + 1) & 1, raw, xq[(u + 1) & 3]);
      load_x(k + 5, xq[(u + 1) & 3]);
      if (u == 3) {
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
          for (int v = 0; v < NV; ++v) idc[s][v] = idn[s][v];
        load_ids(g + 2, idn);
      }
      __syncthreads();  // buffer k & 1 read; step k + 1 produced
    }
  }

  // Epilogue through LDS (the operand tiles are idle after the last barrier):
  // per 32-row slice the wave parks its 32 x 32 NB accumulators in a private
  // area and reads them back one output row per instruction.  The stores are
  // coalesced, and acc is indexed by constants only (a loop over it would put
  // the array in scratch memory).
  constexpr int WC = 32 * NB;  // output columns of a wave
  float* stage = reinterpret_cast<float*>(smem) + wave * 32 * WC;
  const int nloc = wrow0 + wn * WC + lane;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) stage[(8 * (e >> 2) + 4 * hk + (e & 3)) * WC + j * 32 + l32] = acc[i][j][e];
    // (one wave's LDS accesses run in order: the reads see these writes, and
    // the next slice's writes wait for these reads)
    if (lane < WC) {
      for (int r = 0; r < 32; ++r) {
        const int64_t m = m0 + wm * 128 + i * 32 + r;
        const float v = stage[r * WC + lane];
        if (m < M && nloc < ti.rows) store_output(E, m, ti.out_row0 + nloc, v);
      }
    }
  }
}

// Grid: blocks [0, n_full * n_mt) take whole 256 x 256 tiles (tile
// b / n_mt, x tile b % n_mt: the x-tile index fastest, so each XCD's L2 keeps
// revisiting the same x tiles); the blocks after them split each remaining
// tile into two 256 x 128 halves.  The host sizes n_full so that the whole
// tiles fill complete rounds of workgroups and the halves the last one,
// which whole tiles would leave partly empty.
template <int S, typename IdT, int LMODE, int SEM, int XDT>
__global__ __launch_bounds__(kTallThreads) void rvq_prefill_tall_kernel(LayerArgs L, DtypeArgs D, EpilogueArgs E,
                                                                        const uint16_t* __restrict__ x, int64_t M,
                                                                        int n_mt, int rshift, int n_full) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* ws = smem + 2 * kTallTileBytes;
  uint8_t* lds_cb = smem + 4 * kTallTileBytes;
  const int K = L.codebook_size;
  const int tid = threadIdx.x;
  const int bx = (int)blockIdx.x, nfb = n_full * n_mt;
  int mt, nt, half = -1;  // uniform: the whole workgroup
  if (bx < nfb) {
    mt = bx % n_mt;
    nt = bx / n_mt;
  } else {
    const int b2 = bx - nfb, h = b2 / n_mt;
    mt = b2 - h * n_mt;
    nt = n_full + (h >> 1);
    half = h & 1;
  }
  const FragTile<S> ti = get_frag_tile<S>(L, nt);
  if (half > 0 && ti.rows <= 128) return;  // uniform: a second half past the tile's rows
  const int64_t m0 = (int64_t)mt * TBM;

  constexpr int ESZ = lds_entry_bytes<LMODE>();
  if (rshift == 0) {
    stage_codebooks<S, LMODE, SEM, XDT>(lds_cb, ti.p, K, D);
  } else {
    uint8_t* compact = ws;  // the W tiles are idle until the first step
    stage_codebooks<S, LMODE, SEM, XDT>(compact, ti.p, K, D);
    __syncthreads();
    const int n16 = prefill_table_entries<S, IdT>(K) * (ESZ / 16);
    const int nc = 1 << rshift;
    for (int i = tid; i < n16 * nc; i += kTallThreads) {
      const int piece = i >> rshift, c = i & (nc - 1);
      const int e = piece / (ESZ / 16), h = piece - e * (ESZ / 16);
      *reinterpret_cast<u32x4_t*>(lds_cb + (((e << rshift) + c) * ESZ) + 16 * h) =
          *reinterpret_cast<const u32x4_t*>(compact + (size_t)piece * 16);
    }
  }
  __syncthreads();  // table staged (and the compact copy in the W area read)
  if (half < 0) tall_tile<S, IdT, LMODE, SEM, XDT, 2>(L, D, E, x, M, ti, m0, 0, rshift, smem);
  else tall_tile<S, IdT, LMODE, SEM, XDT, 1>(L, D, E, x, M, ti, m0, 128 * half, rshift, smem);
}

// How many of the n_tiles weight tiles run whole: those that fill complete
// rounds of workgroups (one per CU), when the rest, split into halves, fit one
// more round; otherwise all (a second round of halves would take as long as
// the partly empty round of whole tiles it replaces).
inline int tall_full_tiles(int64_t n_tiles, int n_mt, int n_cu) {
  const int64_t n_full = n_tiles * n_mt / n_cu * n_cu / n_mt;
  if (n_full < n_tiles && 2 * (n_tiles - n_full) * n_mt <= n_cu) return (int)n_full;
  return (int)n_tiles;
}

template <int S, typename IdT, int LMODE, int SEM, int XDT>
static hipError_t prefill_tall(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, const void* x,
                               int64_t M, hipStream_t st) {
  const size_t tbl = (size_t)prefill_table_entries<S, IdT>(L.codebook_size) * lds_entry_bytes<LMODE>();
  int rshift = 3;
  while (rshift > 0 && (prefill_tall_lds_bytes<S, IdT, LMODE>(L.codebook_size, rshift) > (size_t)160 * 1024 ||
                        tbl > (size_t)2 * kTallTileBytes))
    --rshift;
  const size_t lds = prefill_tall_lds_bytes<S, IdT, LMODE>(L.codebook_size, rshift);
  auto kern = rvq_prefill_tall_kernel<S, IdT, LMODE, SEM, XDT>;
  hipError_t e = allow_max_lds(reinterpret_cast<const void*>(kern));
  if (e != hipSuccess) return e;
  const int n_mt = (int)((M + TBM - 1) / TBM);
  const int n_full = tall_full_tiles(L.n_tiles, n_mt, device_cu_count());
  dim3 grid((unsigned)(((int64_t)n_full + 2 * (L.n_tiles - n_full)) * n_mt));
  hipLaunchKernelGGL(kern, grid, dim3(kTallThreads), lds, st, L, D, E, reinterpret_cast<const uint16_t*>(x), M, n_mt,
                     rshift, n_full);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Wide tile: 256 x-rows x 128 weight rows, 16 waves (four per SIMD, 128
// registers per lane).  Each dequantised weight feeds 256 MFMA rows, as in
// the tall tile, and the two waves of each role per SIMD keep both the
// matrix core and the VALU issuing (one wave alone issues VALU work at about
// half the SIMD's rate).  The workgroup takes one half of a 256-row weight
// tile (a half past the tile's rows exits at once).
//   * 8 consumer waves, 4 (M) x 2 (N), each a 64 x 64 output tile.
//   * 8 producer waves: thread pt dequantises block pt % 4 of weight row
//     pt / 4 per k-step and copies 2 of the x tile's 1024 16-byte pieces.
// LDS rows and swizzle as in the tall tile.
// ---------------------------------------------------------------------------
constexpr int kWideThreads = 1024;
constexpr int kWideProducerThreads = 512;
constexpr int WBN = 128;  // weight rows per workgroup
constexpr int kWideXBytes = TBM * kTallRowBytes;  // 16 KB
constexpr int kWideWBytes = WBN * kTallRowBytes;  // 8 KB

template <int S, typename IdT, int LMODE>
WAL_HOST_DEVICE size_t prefill_wide_lds_bytes(int K, int rshift) {
  return (size_t)2 * (kWideXBytes + kWideWBytes) +
         ((size_t)prefill_table_entries<S, IdT>(K) * lds_entry_bytes<LMODE>() << rshift);
}

// Instances that fit 128 registers per lane without scratch (compiler
// resource report).
template <int S, typename IdT, int LMODE>
constexpr bool wide_supported() {
  return prefill_wide_ok(S, LMODE, (int)sizeof(IdT));
}

template <int S, typename IdT, int LMODE, int SEM, int XDT>
__global__ __launch_bounds__(kWideThreads) void rvq_prefill_wide_kernel(LayerArgs L, DtypeArgs D, EpilogueArgs E,
                                                                        const uint16_t* __restrict__ x, int64_t M,
                                                                        int n_mt, int rshift) {
  constexpr int XP = TBM * 4 / kWideProducerThreads;  // 2 x pieces per producer thread per k-step
  constexpr int NV = sizeof(IdT);
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* xs = smem;                    // [2][256 rows][64 B]
  uint8_t* ws = smem + 2 * kWideXBytes;  // [2][128 rows][64 B]
  uint8_t* lds_cb = ws + 2 * kWideWBytes;

  const int K = L.codebook_size;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int mt = (int)(blockIdx.x % (unsigned)n_mt);
  const int nh = (int)(blockIdx.x / (unsigned)n_mt);
  const FragTile<S> ti = get_frag_tile<S>(L, nh >> 1);
  const int half = (nh & 1) * WBN;
  const int rows_here = min(WBN, ti.rows - half);
  if (rows_here <= 0) return;  // uniform: the whole workgroup
  const int64_t m0 = (int64_t)mt * TBM;
  const int B = L.blocks_per_row;
  const int in = L.in_features;
  const int nk = B / 4;
  const uint32_t kmax = (uint32_t)(K - 1);

  constexpr int ESZ = lds_entry_bytes<LMODE>();
  if (rshift == 0) {
    stage_codebooks<S, LMODE, SEM, XDT>(lds_cb, ti.p, K, D);
  } else {
    uint8_t* compact = xs;  // the x tiles are idle until the first step
    stage_codebooks<S, LMODE, SEM, XDT>(compact, ti.p, K, D);
    __syncthreads();
    const int n16 = prefill_table_entries<S, IdT>(K) * (ESZ / 16);
    const int nc = 1 << rshift;
    for (int i = tid; i < n16 * nc; i += kWideThreads) {
      const int piece = i >> rshift, c = i & (nc - 1);
      const int e = piece / (ESZ / 16), h = piece - e * (ESZ / 16);
      *reinterpret_cast<u32x4_t*>(lds_cb + (((e << rshift) + c) * ESZ) + 16 * h) =
          *reinterpret_cast<const u32x4_t*>(compact + (size_t)piece * 16);
    }
  }
  __syncthreads();

  if (wave < 8) {
    const int wm = wave >> 1, wn = wave & 1;
    const int l16 = lane & 15, q = lane >> 4;
    const int sw = tall_swz(l16, q);
    const uint8_t* xa = xs + (wm * 64 + l16) * kTallRowBytes + sw;
    const uint8_t* wb = ws + (wn * 64 + l16) * kTallRowBytes + sw;
    f32x4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    __syncthreads();  // step 0 produced
    for (int k = 0; k < nk; ++k) {
      const int bx = (k & 1) * kWideXBytes, bw = (k & 1) * kWideWBytes;
      u32x4_t a[4], b[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const u32x4_t*>(wb + bw + j * 16 * kTallRowBytes);
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const u32x4_t*>(xa + bx + i * 16 * kTallRowBytes);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16<XDT>(a[i], b[j], acc[i][j]);
      __syncthreads();  // buffer k & 1 read; step k + 1 produced
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int nloc = wn * 64 + j * 16 + l16;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t m = m0 + wm * 64 + i * 16 + 4 * q + e;
          if (m < M && nloc < rows_here) store_output(E, m, ti.out_row0 + half + nloc, acc[i][j][e]);
        }
      }
    }
    return;
  }

  // ---- producers: thread pt dequantises block pt % 4 of row pt / 4 ----
  const int pt = tid - 512;
  const int prow = pt >> 2, pb = pt & 3;
  const uint8_t* lds_lane = lds_cb + (lane & ((1 << rshift) - 1)) * ESZ;
  const int64_t wr = ti.row0 + half + (prow < rows_here ? prow : 0);  // rows past the tile: never stored
  const RowScale rs = make_row_scale<XDT>(load_f(ti.p.row_scale, D.sc_dtype, scale_index(L, wr)));
  bufrsrc_t idr[S];
#pragma unroll
  for (int s = 0; s < S; ++s) idr[s] = make_rsrc(ti.p.ids[s]);
  const uint32_t idrow = (uint32_t)(wr * B * (int64_t)sizeof(IdT));
  const bufrsrc_t xr = make_rsrc(x + m0 * in);
  uint32_t xoff[XP];
  int xdst[XP];
#pragma unroll
  for (int i = 0; i < XP; ++i) {
    const int p = pt + i * kWideProducerThreads;
    const int r = p >> 2, c = p & 3;
    xoff[i] = m0 + r < M ? (uint32_t)((r * in + 8 * c) * 2) : kBufOOB;
    xdst[i] = r * kTallRowBytes + tall_swz(r, c);
  }
  uint8_t* wd = ws + prow * kTallRowBytes + tall_swz(prow, pb);
  auto load_x = [&](int k, u32x4_t (&dst)[XP]) {
    const uint32_t step = k < nk ? (uint32_t)(k * PBK * 2) : kBufOOB;
#pragma unroll
    for (int i = 0; i < XP; ++i) dst[i] = ldbuf128(xr, xoff[i] == kBufOOB ? kBufOOB : xoff[i] + step);
  };
  auto load_ids = [&](int grp, u32x4_t (&dst)[S][NV]) {
    const uint32_t off = grp * 4 < nk ? idrow + (uint32_t)(grp * 16 * NV) : kBufOOB;
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int v = 0; v < NV; ++v) dst[s][v] = ldbuf128(idr[s], off == kBufOOB ? kBufOOB : off + 16 * v);
  };
  auto produce = [&](int k, int buf, const u32x4_t (&ids)[S][NV], const u32x4_t (&xv)[XP]) {
    // block 4 (k & 3) + pb of the 16-block index group; k & 3 is a constant
    // of the unrolled loop, pb is not, so the vector words are picked with
    // constant indices and a select (a register array indexed by a variable
    // would be copied to scratch memory)
    const int c = k & 3;
    uint32_t id[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if constexpr (NV == 1) {
        id[s] = (ids[s][0][c] >> (8 * pb)) & 0xffu;  // inside the allocation
      } else {
        const uint32_t lo = ids[s][c >> 1][(2 * c) & 3], hi = ids[s][c >> 1][(2 * c + 1) & 3];
        id[s] = min(((pb & 2 ? hi : lo) >> (16 * (pb & 1))) & 0xffffu, kmax);
      }
    }
    const WfragRaw<S, LMODE> raw = gather_wfrag_rep<S, LMODE>(lds_lane, id, K, rshift);
#pragma unroll
    for (int i = 0; i < XP; ++i) *reinterpret_cast<u32x4_t*>(xs + buf * kWideXBytes + xdst[i]) = xv[i];
    *reinterpret_cast<u32x4_t*>(wd + buf * kWideWBytes) = combine_wfrag<S, LMODE, SEM, XDT>(raw, L.active_mask, rs);
  };

  u32x4_t xq[4][XP];
  u32x4_t idq[2][S][NV];
  load_ids(0, idq[0]);
  load_ids(1, idq[1]);
#pragma unroll
  for (int j = 0; j < 4; ++j) load_x(j, xq[j]);
  produce(0, 0, idq[0], xq[0]);
  load_x(4, xq[0]);
  __syncthreads();  // step 0 produced
  for (int k0 = 0; k0 < nk; k0 += 8) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = k0 + u;
      if (k >= nk) break;  // uniform
      const int gs = ((u + 1) >> 2) & 1;
      produce(k + 1, (u + 1) & 1, idq[gs], xq[(u + 1) & 3]);
      load_x(k + 5, xq[(u + 1) & 3]);
      if (((u + 1) & 3) == 3) load_ids(((k + 1) >> 2) + 2, idq[gs]);
      __syncthreads();
    }
  }
}

template <int S, typename IdT, int LMODE, int SEM, int XDT>
static hipError_t prefill_wide(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, const void* x,
                               int64_t M, hipStream_t st) {
  const size_t tbl = (size_t)prefill_table_entries<S, IdT>(L.codebook_size) * lds_entry_bytes<LMODE>();
  int rshift = 3;
  while (rshift > 0 && (prefill_wide_lds_bytes<S, IdT, LMODE>(L.codebook_size, rshift) > (size_t)160 * 1024 ||
                        tbl > (size_t)2 * kWideXBytes))
    --rshift;
  const size_t lds = prefill_wide_lds_bytes<S, IdT, LMODE>(L.codebook_size, rshift);
  auto kern = rvq_prefill_wide_kernel<S, IdT, LMODE, SEM, XDT>;
  hipError_t e = allow_max_lds(reinterpret_cast<const void*>(kern));
  if (e != hipSuccess) return e;
  const int n_mt = (int)((M + TBM - 1) / TBM);
  dim3 grid((unsigned)(L.n_tiles * (int64_t)2 * n_mt));
  hipLaunchKernelGGL(kern, grid, dim3(kWideThreads), lds, st, L, D, E, reinterpret_cast<const uint16_t*>(x), M, n_mt,
                     rshift);
  return hipGetLastError();
}

template <int S, typename IdT, int LMODE, int SEM, int XDT, int TM>
static hipError_t prefill_tm(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, const void* x,
                             int64_t M, const PrefillSplit& sp, hipStream_t st) {
  // as many table copies (up to 8) as fit; the compact table is staged in
  // the W tile area first, so replication needs it to fit there
  const size_t tbl = (size_t)prefill_table_entries<S, IdT>(L.codebook_size) * lds_entry_bytes<LMODE>();
  int rshift = 3;
  while (rshift > 0 && (prefill_lds_bytes<S, IdT, LMODE>(TM, L.codebook_size, rshift) > (size_t)160 * 1024 ||
                        tbl > (size_t)2 * PBN * PSTR * sizeof(uint16_t)))
    --rshift;
  const size_t lds = prefill_lds_bytes<S, IdT, LMODE>(TM, L.codebook_size, rshift);
  auto kern = rvq_prefill_kernel<S, IdT, LMODE, SEM, XDT, TM>;
  hipError_t e = allow_max_lds(reinterpret_cast<const void*>(kern));
  if (e != hipSuccess) return e;
  const int n_mt = (int)((M + prefill_bm<TM>() - 1) / prefill_bm<TM>());
  const int ksplit = sp.part != nullptr && sp.ksplit > 1 ? sp.ksplit : 1;
  dim3 grid((unsigned)(L.n_tiles * (int64_t)n_mt * ksplit));
  hipLaunchKernelGGL(kern, grid, dim3(kPrefillThreads), lds, st, L, D, E, reinterpret_cast<const uint16_t*>(x), M,
                     n_mt, rshift, ksplit, sp.part);
  e = hipGetLastError();
  if (e != hipSuccess || ksplit == 1) return e;
  return launch_splitk_reduce(sp.part, ksplit, M, E, st);
}

// shape: the tile shape from plan_prefill_shape (PS_SHORT when the instance
// has no kernel of the requested shape).  Short is 128 x-rows x 256 weight
// rows (TM = 4, a 64 x 64 tile per wave).
template <int S, typename IdT, int LMODE, int SEM, int XDT>
static hipError_t prefill_go(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, const void* x,
                             int64_t M, int shape, const PrefillSplit& sp, hipStream_t st) {
  constexpr bool can_tall = tall_supported<S, IdT, LMODE>(), can_wide = wide_supported<S, IdT, LMODE>();
  if constexpr (can_tall)
    if (shape == PS_TALL) return prefill_tall<S, IdT, LMODE, SEM, XDT>(L, D, E, x, M, st);
  if constexpr (can_wide)
    if (shape == PS_WIDE) return prefill_wide<S, IdT, LMODE, SEM, XDT>(L, D, E, x, M, st);
  return prefill_tm<S, IdT, LMODE, SEM, XDT, 4>(L, D, E, x, M, sp, st);
}

template <int S, typename IdT, int XDT>
static hipError_t prefill_sem(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, int sem, int lmode,
                              const void* x, int64_t M, int shape, const PrefillSplit& sp, hipStream_t st) {
  if (sem == SEM_FAST) return prefill_go<S, IdT, LM_A16, SEM_FAST, XDT>(L, D, E, x, M, shape, sp, st);
  if constexpr (S == 1) {
    return prefill_go<S, IdT, LM_A16, SEM_RECON, XDT>(L, D, E, x, M, shape, sp, st);
  } else {
    if (lmode == LM_H16) return prefill_go<S, IdT, LM_H16, SEM_RECON, XDT>(L, D, E, x, M, shape, sp, st);
    return prefill_go<S, IdT, LM_F32, SEM_RECON, XDT>(L, D, E, x, M, shape, sp, st);
  }
}

// Entry for one (activation dtype, index width); explicitly instantiated in
// rvq_prefill_<x>_<ids>.hip.
template <int XDT, typename IdT>
hipError_t prefill_entry(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, int sem, int lmode,
                         const void* x, int64_t M, int shape, const PrefillSplit& sp, hipStream_t st) {
  switch (L.num_stages) {
    case 1: return prefill_sem<1, IdT, XDT>(L, D, E, sem, lmode, x, M, shape, sp, st);
    case 2: return prefill_sem<2, IdT, XDT>(L, D, E, sem, lmode, x, M, shape, sp, st);
    case 3: return prefill_sem<3, IdT, XDT>(L, D, E, sem, lmode, x, M, shape, sp, st);
    default: return prefill_sem<4, IdT, XDT>(L, D, E, sem, lmode, x, M, shape, sp, st);
  }
}

}  // namespace wal
