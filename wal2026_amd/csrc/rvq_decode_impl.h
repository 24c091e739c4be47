// rvq_decode_impl.h -- Block-RVQ linear for M <= 16 (decode), block_size 8.
//
// The weight is never written to memory.  Layout of the work:
//   * A workgroup of NW = blockDim.x / 64 waves takes a contiguous range of
//     16-row tiles.  It keeps the codebooks of the current row group in LDS
//     (restaged only when the tile's group changes) and, when it fits, the
//     activation rows x[0..M) as well.
//   * Within a tile the row's 64-block chunks are dealt to the waves: wave w
//     takes chunks w, w + NW, ...; every wave takes the same number CPT of
//     chunk slots per tile (a slot past the last chunk contributes nothing),
//     so the per-tile barriers are uniform.
//   * Lane l covers weight row n = l % 16 and the 16 consecutive blocks
//     [64c + 16q, 64c + 16q + 16), q = l / 16: one 128-bit load per stage for
//     8-bit ids, two for 16-bit ids.
//   * Software pipeline: the index loads (and the lane's row-scale load) of
//     the item PF slots ahead (decode_prefetch) are issued as an item is
//     taken from the ring, before its compute, as straight-line code, so
//     the only memory waits in the loop are the in-order ones for the slot
//     being consumed.  Loads past the end of the range get an out-of-range
//     buffer offset and read zeros without touching memory.  Per-tile
//     metadata comes from the plan through the scalar cache.
//   * For each block the lane gathers the S codewords from LDS, rebuilds the 8
//     weights exactly as the reference's dequantisation does (rvq_fragment.h)
//     and feeds them as the B operand of v_mfma_f32_16x16x32_{bf16,f16}; the A
//     operand is x[min(l % 16, M - 1)] at the same 8 columns (rows m >= M of
//     the product are never stored).
//   * SCALED (one stage, every 16-row tile under a single row-scale value):
//     the codebook is staged already multiplied by the tile's scale with the
//     reference's rounding, so the hot loop is gather + MFMA only; the staged
//     table is rebuilt when the scale changes.
//   * No barrier and no global store per tile: each wave parks its partial
//     16x16 accumulator of a tile in LDS; after the last tile of the range the
//     workgroup sums the NW partials and writes the M x 16 outputs of every
//     tile.  (A global store pending beside the index loads would make the
//     compiler's in-order load waits fall back to full drains.)
#pragma once

#include <type_traits>

#include "rvq_fragment.h"

namespace wal {

// Items of index loads in flight per wave.  Measured on gfx950 at every
// benchmark shape (c2, c3, c5): one item ahead is fastest.  The loop is bound
// by the LDS codeword gathers and the dequantisation arithmetic, not by HBM
// latency, and every deeper ring slot adds straight-line code and prologue
// loads (PF 4 -> 1: c3 +4 %, c5 +8 %, c2 +5 % tokens/s; with the refill
// issued before the compute, PF 2 -> 1: c3 +4 %, c5 +7 %).
template <int S, typename IdT>
constexpr int decode_prefetch() {
  return 1;
}

// Fragments whose codeword gathers are issued ahead of the one being combined
// in the pipelined item loop (multi-stage or per-row-scaled tables): two, or
// one when a fragment's codewords take more than 24 VGPRs.  Measured on
// gfx950 (decode M = 1, tokens/s): c5 442 -> 475, c2 1850 -> 2031 against
// gathering all 16 fragments before combining any; 1 and 2 ahead are equal,
// 4 and 6 ahead are slower (register pressure).
template <int S, int LMODE>
constexpr int decode_gather_ahead() {
  return S * lds_entry_bytes<LMODE>() / 4 > 24 ? 1 : 2;
}

// Each lane gets the value of lane TT of its 16-lane row (DPP row_newbcast).
template <int TT>
WAL_DEVICE uint32_t row_bcast_dw(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x150 + TT, 0xf, 0xf, false);
}
template <int TT>
WAL_DEVICE u32x4_t row_bcast_t(const u32x4_t& v) {
  return u32x4_t{row_bcast_dw<TT>(v[0]), row_bcast_dw<TT>(v[1]), row_bcast_dw<TT>(v[2]), row_bcast_dw<TT>(v[3])};
}
// row_bcast_t<tt> for a tt known after unrolling.
WAL_DEVICE u32x4_t row_bcast(const u32x4_t& v, int tt) {
  switch (tt) {
    case 0: return row_bcast_t<0>(v);
    case 1: return row_bcast_t<1>(v);
    case 2: return row_bcast_t<2>(v);
    case 3: return row_bcast_t<3>(v);
    case 4: return row_bcast_t<4>(v);
    case 5: return row_bcast_t<5>(v);
    case 6: return row_bcast_t<6>(v);
    case 7: return row_bcast_t<7>(v);
    case 8: return row_bcast_t<8>(v);
    case 9: return row_bcast_t<9>(v);
    case 10: return row_bcast_t<10>(v);
    case 11: return row_bcast_t<11>(v);
    case 12: return row_bcast_t<12>(v);
    case 13: return row_bcast_t<13>(v);
    case 14: return row_bcast_t<14>(v);
    default: return row_bcast_t<15>(v);
  }
}

template <typename IdT>
WAL_DEVICE uint32_t extract_id(const u32x4_t (&v)[sizeof(IdT)], int t) {
  if constexpr (sizeof(IdT) == 1) {
    return (v[0][t >> 2] >> (8 * (t & 3))) & 0xffu;
  } else {
    return (v[t >> 3][(t >> 1) & 3] >> (16 * (t & 1))) & 0xffffu;
  }
}

// Tile metadata through the scalar cache (uniform t): no vector-memory
// instruction, so reading it never waits on the index loads in flight.
template <int S>
WAL_DEVICE FragTile<S> tile_at(const LayerArgs& L, int t) {
  FragTile<S> f;
  if (L.plan == nullptr) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      f.p.ids[s] = L.g0.stage_ids[s];
      f.p.cb[s] = L.g0.codebooks[s];
    }
    f.p.row_scale = L.g0.row_scale;
    f.p.stage_scales = L.g0.stage_scales;
    f.group = 0;
    f.row0 = t * 16;
    f.out_row0 = L.g0.row0 + f.row0;
    f.grows = L.g0.rows;
  } else {
    typedef const __attribute__((address_space(4))) PlanTile c_tile_t;
    typedef const __attribute__((address_space(4))) wal_rvq_group c_group_t;
    c_tile_t* pt = (c_tile_t*)(L.plan_tiles) + t;
    c_group_t* G = (c_group_t*)(L.plan_groups) + pt->group;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      f.p.ids[s] = G->stage_ids[s];
      f.p.cb[s] = G->codebooks[s];
    }
    f.p.row_scale = G->row_scale;
    f.p.stage_scales = G->stage_scales;
    f.group = pt->group;
    f.row0 = pt->row0;
    f.out_row0 = pt->out_row0;
    f.grows = G->rows;
  }
  return f;
}

// Rows of a decode tile: its 16-row slice of the group, shorter at the
// group's end.  (Derived, not kept in the tile: a field that only some paths
// update makes the compiler keep the tile in scratch memory.)
template <int S>
WAL_DEVICE int tile_rows(const FragTile<S>& f) {
  return min(16, f.grows - f.row0);
}

// Tile t + 1 from tile t (f).  A group's tiles are consecutive 16-row tiles
// of the plan, so only the first tile of the next group is read from the
// plan: inside the loop a plan read is a dependent scalar-memory round trip
// (cold in L2 when the step streams more bytes than the caches hold) that
// every wave of the workgroup would wait for.
template <int S>
WAL_DEVICE FragTile<S> next_tile(const LayerArgs& L, const FragTile<S>& f, int t_next) {
  if (f.row0 + 16 < f.grows) {
    FragTile<S> n = f;
    n.row0 += 16;
    n.out_row0 += 16;
    return n;
  }
  return tile_at<S>(L, t_next);
}

// Staged-table key of a tile: its group, and for scaled tables its scale run.
template <int S, bool SCALED>
WAL_DEVICE int table_key(const LayerArgs& L, const FragTile<S>& f) {
  return SCALED ? (f.group << 16) ^ (int)scale_index(L, f.row0) : f.group;
}

WAL_DEVICE float scale_bits_to_f32(uint32_t h, int dt) { return dt == WAL_F16 ? f16_to_f32(h) : bf16_to_f32(h); }

// Stage one table (a group's codebooks, scaled by rs for SCALE_TABLE) from
// the image when there is one, else from the raw codebooks.  Inlined: an
// out-of-line call would give the kernel a call frame and a private (scratch)
// segment that every launch has to set up.
extern __shared__ __attribute__((aligned(16))) uint8_t decode_smem[];

template <int S, int LMODE, int SEM, int XDT, bool SCALE_TABLE>
WAL_DEVICE void stage_table(uint32_t dst_off, const uint8_t* img, const GroupPtrs<S>& p, int K, const DtypeArgs& D,
                            const RowScale& rs) {
  uint8_t* dst = decode_smem + dst_off;
  if (img != nullptr) stage_image<XDT, SCALE_TABLE>(dst, img, S * K * lds_entry_bytes<LMODE>() / 16, rs);
  else stage_codebooks<S, LMODE, SEM, XDT, SCALE_TABLE>(dst, p, K, D, rs);
}

template <int S, typename IdT, int LMODE, int SEM, int XDT, int XMODE, bool SCALED, int G>
__global__ __launch_bounds__(kDecodeMaxThreads) void rvq_decode_kernel(LayerArgs L, DtypeArgs D, EpilogueArgs E,
                                                                       const uint16_t* __restrict__ x, int M,
                                                                       int max_tiles, int nslots) {
  static_assert(!SCALED || LMODE == LM_A16, "scaled tables hold one 16-bit value per element");
  static_assert(G == 1 || XMODE == XM_REG, "wave groups: one chunk per wave, x fragments in registers");
  // Touch every cache line of the kernel arguments at once: otherwise the
  // compiler loads each field where it is first used, and every first touch
  // of a line is its own dependent scalar-memory round trip.
  asm volatile("" ::"s"(L.in_features), "s"(L.plan_tiles), "s"(L.plan_groups), "s"(L.g0.stage_ids[0]), "s"(L.g0.codebooks[4]),
               "s"(L.g0.row_scale), "s"(L.image), "s"(D.x_dtype), "s"(E.y), "s"(E.bias_mode), "s"(x), "s"(nslots));
  constexpr bool XLDS = XMODE == XM_LDS || XMODE == XM_REG;
  constexpr bool XREG = XMODE == XM_REG || XMODE == XM_GREG;
  constexpr int PF = decode_prefetch<S, IdT>(), NV = sizeof(IdT);
  constexpr int ESZ = lds_entry_bytes<LMODE>();
  constexpr int XR = 4;  // 16-byte x loads per thread kept in registers across the codebook staging
  uint8_t* smem = decode_smem;
  constexpr int NW = kDecodeMaxWaves;  // launched with exactly NW waves
  const int K = L.codebook_size;
  const int B = L.blocks_per_row;
  const int in = L.in_features;
  const int M16 = M * 16;
  const int tbl_bytes = S * K * ESZ;  // one staged table (all stages of a group)
  uint8_t* lds_cb = smem;             // nslots (1 or 2) table slots
  float* part = reinterpret_cast<float*>(smem + (size_t)nslots * tbl_bytes);  // [max_tiles][NW][M * 16]
  int* tmeta = reinterpret_cast<int*>(part + (size_t)max_tiles * NW * M16);      // [max_tiles][4]
  uint8_t* zrow = reinterpret_cast<uint8_t*>(tmeta + (size_t)max_tiles * 4);   // 256 zero bytes
  uint16_t* xs = reinterpret_cast<uint16_t*>(zrow + 256);                    // [M][in] when XLDS
  uint8_t* xscr = zrow + 256;  // XM_GTR: [NW][8 rows][1 KB] transpose scratch

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nl = lane & 15;
  const int q = lane >> 4;
  const int nchunk = (B + 63) >> 6;
  // G wave groups (G > 1 when a row has at most NW / G chunks): group g =
  // wave / NWG computes the range's tiles j with j % G == g, wave w taking
  // chunk w % NWG of them, so no wave idles for want of a chunk.  Every wave
  // still walks every tile (table slots, restages and partial parking stay
  // in lockstep); a wave's partial for a tile it does not compute is the
  // zero it started the tile with, so the sums are those of G == 1.
  constexpr int NWG = NW / G;
  const int wch = G == 1 ? wave : wave % NWG;  // this wave's chunk (first of CPT)
  const int wgr = G == 1 ? 0 : wave / NWG;    // this wave's group
  const int CPT = (nchunk + NWG - 1) / NWG;
  // tiles [t_begin, t_begin + n_tiles_wg): T split as evenly as possible
  const int T = L.n_tiles;
  const int tq = T / (int)gridDim.x, tr = T % (int)gridDim.x, bx = blockIdx.x;
  const int t_begin = bx * tq + min(bx, tr);
  const int n_tiles_wg = tq + (bx < tr ? 1 : 0);
  const int t_end = t_begin + n_tiles_wg;
  const int n_items = n_tiles_wg * CPT;
  const int xm = min(nl, M - 1);  // x row this lane feeds to the MFMA
  // Ids are validated against K by the caller; one past the range is clamped
  // to the last entry, as every kernel of the library does, so it never reads
  // outside the staged table.
  const uint32_t kmax = (uint32_t)(K - 1);

  // ---- prologue, part 1: loads of the activations and tables ---------------
  // The range's tiles fall in one or two table segments (same group and, for
  // scaled tables, same scale run): the segment boundary is where the first
  // tile's group or scale run ends.  Both segments' tables are staged into
  // slots 0 and 1 (when the launch has two); any other segment (a range
  // longer than a group, or a single slot) is restaged in the loop.  These
  // loads are issued before the index ring, so waiting for them (vmcnt is
  // in order) does not wait for the cold index loads behind them.
  FragTile<S> cti = tile_at<S>(L, t_begin);
  const int gseg = t_begin + (cti.grows - cti.row0 + 15) / 16;  // first tile of the next group
  int seg1 = gseg;
  if constexpr (SCALED) {
    const int run_left = L.scale_rows - (cti.row0 & (L.scale_rows - 1));  // scale_rows: power of two >= 16
    seg1 = min(seg1, t_begin + run_left / 16);
  }
  const bool two = seg1 < t_end && nslots == 2;
  FragTile<S> sti = cti;
  if (two) {
    if (seg1 < gseg) {
      // a scale-run boundary inside the group: the group's tiles are
      // consecutive 16-row tiles, so no table read is needed
      const int dr = (seg1 - t_begin) * 16;
      sti.row0 += dr;
      sti.out_row0 += dr;
    } else {
      sti = tile_at<S>(L, seg1);
    }
  }
  // keys of the tables in slots 0 and 1 (two scalars: a dynamically indexed
  // array would live in scratch memory)
  int key0 = table_key<S, SCALED>(L, cti), key1 = two ? table_key<S, SCALED>(L, sti) : -1;
  const bool have_image = L.image != nullptr;
  const uint8_t* img0 = have_image ? L.image + (size_t)cti.group * tbl_bytes : nullptr;
  const uint8_t* img1 = have_image ? L.image + (size_t)sti.group * tbl_bytes : nullptr;
  const bool same_img = sti.group == cti.group;
  const int n16 = XLDS ? M * in / 8 : 0;  // 16-byte pieces of x (in % 128 == 0)
  const int t16 = tbl_bytes / 16;
  u32x4_t xr[XR];
#pragma unroll
  for (int u = 0; u < XR; ++u) {
    // (uniform: n16 is a multiple of 64) no load for pieces past x, which
    // would only take load-issue bandwidth from the table loads behind them
    if (u == 0 || u * (int)blockDim.x < n16)
      xr[u] = ldg128(x + (size_t)min(tid + u * (int)blockDim.x, max(n16 - 1, 0)) * 8);
  }
  // XM_REG / XM_GREG: this wave's chunk is the same for every tile, so its 16
  // x fragments (zero past the row) are read once: XM_GREG here, from global
  // memory, XM_REG after the barrier, from the x rows staged in LDS.
  u32x4_t xreg[XREG ? 16 : 1];
  // XM_GREG with room in the table slots (uniform): each load reads one
  // contiguous 1 KB run of an x row (lane = block of the wave's chunk), and
  // the fragments are transposed through the table slots' LDS before the
  // tables are staged.  A lane's own fragments are 16-byte pieces of one row,
  // so loading them directly touches 64 cache lines per instruction.
  const bool xt = XMODE == XM_GREG && M > 4 && (size_t)nslots * tbl_bytes >= (size_t)NW * 16 * 1024;
  if constexpr (XMODE == XM_GREG) {
    if (xt) {
      const int blk = wave * 64 + lane;
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (u < M) xreg[u] = blk < B ? ldg128(x + (size_t)u * in + (size_t)blk * 8) : u32x4_t{0, 0, 0, 0};
    } else {
      const int base = wave * 64 + 16 * q;
#pragma unroll
      for (int tt = 0; tt < 16; ++tt)
        xreg[tt] = base < B ? ldg128(x + (size_t)xm * in + (size_t)(base + tt) * 8) : u32x4_t{0, 0, 0, 0};
    }
  }
  u32x4_t b0[kImageBatch], b1[kImageBatch];
  if (have_image) {
    load_image_batch(b0, img0, t16, tid, blockDim.x);
    // both slots of one group (two scale runs) stage from the same image:
    // load it once (per-CU load bandwidth bounds this prologue)
    if (two && !same_img) load_image_batch(b1, img1, t16, tid, blockDim.x);
  }
  uint32_t sc0 = 0, sc1 = 0;  // scales of the two segments (scaled tables)
  if constexpr (SCALED) {
    sc0 = ldg<uint16_t>(cti.p.row_scale, scale_index(L, cti.row0));
    sc1 = ldg<uint16_t>(sti.p.row_scale, scale_index(L, sti.row0));
  }

  // ---- index ring: issue cursor runs PF items ahead of the compute cursor ----
  u32x4_t ring[PF][S][NV];
  uint32_t rsr[PF];  // raw bits of the lane's row scale for the slot's tile
  int is_t = 0, is_c = 0;
  FragTile<S> iti = cti;
  auto issue = [&](int j) {
    // Always issues the same buffer loads (straight-line code); a slot past
    // the range, or a chunk past the row, gets an out-of-range offset and
    // reads zeros without touching memory.  Rows past the tile re-read its
    // last row (outputs of those rows are never stored).
    const int c = wch + NWG * is_c;
    const bool ok = is_t < n_tiles_wg && c < nchunk && (G == 1 || is_t % G == wgr);  // uniform
    const int base = min(c * 64 + 16 * q, B - 16);
    const int r = iti.row0 + min(nl, tile_rows<S>(iti) - 1);
    const uint32_t off = ok ? (uint32_t)((r * B + base) * (int)sizeof(IdT)) : kBufOOB;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const bufrsrc_t rs_ids = make_rsrc(iti.p.ids[s]);
#pragma unroll
      for (int v = 0; v < NV; ++v) ring[j][s][v] = ldbuf128_stream(rs_ids, off + v * 16);
    }
    // 16-bit scale buffers only (the host routes fp32 scales elsewhere)
    const int si = (int)scale_index(L, SCALED ? iti.row0 : r);
    rsr[j] = ldbuf16(make_rsrc(iti.p.row_scale), is_t < n_tiles_wg ? (uint32_t)si * 2u : kBufOOB);
    if (++is_c == CPT) {
      is_c = 0;
      if (++is_t < n_tiles_wg) iti = next_tile<S>(L, iti, t_begin + is_t);
    }
  };
#pragma unroll
  for (int j = 0; j < PF; ++j) issue(j);

  // ---- prologue, part 2: stage the tables and x while the ring loads fly ---
  if constexpr (XMODE == XM_GREG) {
    if (xt) {
      // this wave's rows of its chunk, 1 KB per row, piece p of row u at
      // p ^ u: conflict-free writes, and conflict-free reads for the 16
      // lanes (16 rows) of each read pass
      uint8_t* xw = lds_cb + (size_t)wave * 16 * 1024;
#pragma unroll
      for (int u = 0; u < 16; ++u)
        if (u < M) *reinterpret_cast<u32x4_t*>(xw + u * 1024 + ((lane ^ u) & 63) * 16) = xreg[u];
      // (a wave reads back only what it wrote)
#pragma unroll
      for (int tt = 0; tt < 16; ++tt)
        xreg[tt] = *reinterpret_cast<const u32x4_t*>(xw + xm * 1024 + (((16 * q + tt) ^ xm) & 63) * 16);
      __syncthreads();  // every wave holds its fragments before the tables overwrite the slots
    }
  }
  if (tid < 16) reinterpret_cast<u32x4_t*>(zrow)[tid] = u32x4_t{0, 0, 0, 0};
  RowScale r0 = make_row_scale<XDT>(0.0f), r1 = r0;
  if constexpr (SCALED) {
    r0 = make_row_scale<XDT>(scale_bits_to_f32(__builtin_amdgcn_readfirstlane(sc0), D.sc_dtype));
    r1 = make_row_scale<XDT>(scale_bits_to_f32(__builtin_amdgcn_readfirstlane(sc1), D.sc_dtype));
  }
  if (have_image) {
    stage_image<XDT, SCALED>(lds_cb, img0, t16, r0, &b0);
    if (two) {
      // (a register copy: selecting between the two arrays by pointer would
      // put both in scratch memory)
      if (same_img) {
#pragma unroll
        for (int u = 0; u < kImageBatch; ++u) b1[u] = b0[u];
      }
      stage_image<XDT, SCALED>(lds_cb + tbl_bytes, img1, t16, r1, &b1);
    }
  } else {
    // no image: convert the raw codebooks here (out of line)
    stage_table<S, LMODE, SEM, XDT, SCALED>(0u, nullptr, cti.p, K, D, r0);
    if (two) stage_table<S, LMODE, SEM, XDT, SCALED>((uint32_t)tbl_bytes, nullptr, sti.p, K, D, r1);
  }
  if constexpr (XLDS) {
#pragma unroll
    for (int u = 0; u < XR; ++u)
      if (tid + u * (int)blockDim.x < n16) reinterpret_cast<u32x4_t*>(xs)[tid + u * blockDim.x] = xr[u];
    for (int i = tid + XR * blockDim.x; i < n16; i += blockDim.x)
      reinterpret_cast<u32x4_t*>(xs)[i] = ldg128(x + (size_t)i * 8);
  }
  __syncthreads();

  if constexpr (XMODE == XM_REG) {
    const int base = wch * 64 + 16 * q;
    const uint8_t* xp = base < B ? reinterpret_cast<const uint8_t*>(xs + (size_t)xm * in + (size_t)base * 8) : zrow;
#pragma unroll
    for (int tt = 0; tt < 16; ++tt) xreg[tt] = *reinterpret_cast<const u32x4_t*>(xp + tt * 16);
  }
  if constexpr (XREG) {
    // Opaque to the compiler, so it keeps them in registers instead of
    // re-reading them next to each MFMA (waiting on the newest LDS read is a
    // full lgkmcnt(0) wait, which would serialise the gathers).
#pragma unroll
    for (int tt = 0; tt < 16; ++tt) asm volatile("" : "+v"(xreg[tt]));
  }

  // ---- compute ----------------------------------------------------------------
  int ct_t = 0, ct_c = 0;  // compute cursor
  int slot = 0;            // table slot of the current tile
  RowScale rs = make_row_scale<XDT>(0.0f);
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int i0 = 0; i0 < n_items; i0 += PF) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const bool live = i0 + j < n_items;  // uniform
      if (live && ct_c == 0) {
        // first item of a tile: pick its table slot
        if (ct_t > 0) cti = next_tile<S>(L, cti, t_begin + ct_t);  // tile t_begin: the prologue's
        // the epilogue's output rows of this tile (no plan read there)
        if (tid == 0) reinterpret_cast<int2*>(tmeta)[2 * ct_t] = make_int2(cti.out_row0, tile_rows<S>(cti));
        const int k = table_key<S, SCALED>(L, cti);
        if (k == key0) {
          slot = 0;
        } else if (k == key1) {
          slot = 1;
        } else {
          // a segment no slot holds: restage into the slot the previous tile
          // did not use (the only slot when there is one)
          slot = nslots == 2 ? slot ^ 1 : 0;
          __syncthreads();  // every wave is done with that slot
          RowScale r = make_row_scale<XDT>(0.0f);
          if constexpr (SCALED) r = make_row_scale<XDT>(scale_bits_to_f32(__builtin_amdgcn_readfirstlane(rsr[j]), D.sc_dtype));
          stage_table<S, LMODE, SEM, XDT, SCALED>((uint32_t)(slot * tbl_bytes),
                                                  L.image != nullptr ? L.image + (size_t)cti.group * tbl_bytes : nullptr,
                                                  cti.p, K, D, r);
          __syncthreads();
          if (slot == 0) key0 = k;
          else key1 = k;
        }
        if constexpr (!SCALED) rs = make_row_scale<XDT>(scale_bits_to_f32(rsr[j], D.sc_dtype));
        acc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      }
      // Take this item's indices out of the ring and refill the slot with the
      // item PF ahead (uniform) before computing, so that load's latency runs
      // under this item's gathers and MFMAs (c3 +5 %, c5 +4 % tokens/s
      // against a refill after the compute).
      u32x4_t cur[S][NV];
#pragma unroll
      for (int s = 0; s < S; ++s)
#pragma unroll
        for (int v = 0; v < NV; ++v) cur[s][v] = ring[j][s][v];
      if (i0 + j + PF < n_items) issue(j);
      const int c = wch + NWG * ct_c;
      if (live && c < nchunk && (G == 1 || ct_t % G == wgr)) {  // uniform across the wave
        const int base = c * 64 + 16 * q;
        const bool seg_ok = base < B;  // lanes past the row read zero activations
        // lanes past the row read the 256-byte zero row instead
        const uint8_t* xp = XLDS && seg_ok ? reinterpret_cast<const uint8_t*>(xs + (size_t)xm * in + (size_t)base * 8)
                                           : zrow;
        // The item's compute.  xb (M = 1, x in LDS): each lane reads one
        // 16-byte piece of the chunk's x row (the 16 lanes of a row hold the
        // segment's 16 fragments, one conflict-free read), and fragment tt is
        // broadcast from lane tt of each row with DPP instead of 16 LDS reads.
        auto item = [&](auto xb) {
          u32x4_t xpiece = {0, 0, 0, 0};
          if constexpr (decltype(xb)::value) {
            if (seg_ok) xpiece = *reinterpret_cast<const u32x4_t*>(xs + (size_t)(base + nl) * 8);
          }
          const uint8_t* tbl = lds_cb + (size_t)slot * tbl_bytes;
          // XM_GTR: the rows' runs of this chunk, issued before the gathers so
          // their latency runs under them
          u32x4_t xv[XMODE == XM_GTR ? 16 : 1];
          if constexpr (XMODE == XM_GTR) {
            const int blk = c * 64 + lane;
  #pragma unroll
            for (int u = 0; u < 16; ++u)
              if (u < M) xv[u] = blk < B ? ldg128(x + (size_t)u * in + (size_t)blk * 8) : u32x4_t{0, 0, 0, 0};
          }
          // The activation fragment of block slot tt of the item.
          auto x_frag = [&](int tt, const u32x4_t (&xt)[XMODE == XM_GTR ? 16 : 1]) -> u32x4_t {
            if constexpr (XREG) {
              return xreg[tt];
            } else if constexpr (XMODE == XM_GTR) {
              return xt[tt];
            } else if constexpr (decltype(xb)::value) {
              return row_bcast(xpiece, tt);
            } else if constexpr (XMODE == XM_LDS) {
              return *reinterpret_cast<const u32x4_t*>(xp + tt * 16);
            } else {
              const u32x4_t xf = ldg128(x + (size_t)xm * in + (size_t)min(base + tt, B - 1) * 8);
              return seg_ok ? xf : u32x4_t{0, 0, 0, 0};
            }
          };
          auto ids_of = [&](int tt, uint32_t (&id)[S]) {
  #pragma unroll
            for (int s = 0; s < S; ++s) id[s] = min(extract_id<IdT>(cur[s], tt), kmax);
          };
          if constexpr (!SCALED && XMODE != XM_GTR) {
            // Software pipeline over the item's 16 fragments: the codeword
            // gathers of fragment tt + GA are issued before fragment tt is
            // combined (stage sums, roundings and the row-scale product on the
            // VALU), so each wave's LDS gathers run under its own VALU work
            // instead of after it.
            constexpr int GA = decode_gather_ahead<S, LMODE>();
            const u32x4_t xt_unused[1] = {u32x4_t{0, 0, 0, 0}};
            WfragRaw<S, LMODE> raw[GA];
  #pragma unroll
            for (int tt = 0; tt < GA; ++tt) {
              uint32_t id[S];
              ids_of(tt, id);
              raw[tt] = gather_wfrag<S, LMODE>(tbl, id, K);
            }
  #pragma unroll
            for (int tt = 0; tt < 16; ++tt) {
              WfragRaw<S, LMODE> nxt;
              if (tt + GA < 16) {
                uint32_t id[S];
                ids_of(tt + GA, id);
                nxt = gather_wfrag<S, LMODE>(tbl, id, K);
              }
              // keep the next gathers ahead of this fragment's VALU work
              __builtin_amdgcn_sched_barrier(0);
              const u32x4_t w = combine_wfrag<S, LMODE, SEM, XDT>(raw[tt % GA], L.active_mask, rs);
              acc = mfma16<XDT>(x_frag(tt, xt_unused), w, acc);
              if (tt + GA < 16) raw[tt % GA] = nxt;
            }
          } else {
            // All 16 fragments of the item are gathered before the first MFMA
            // consumes one, so the LDS latency is paid once per item instead of
            // once per block.
            u32x4_t wf[16];
  #pragma unroll
            for (int tt = 0; tt < 16; ++tt) {
              uint32_t id[S];
              ids_of(tt, id);
              if constexpr (SCALED) wf[tt] = *reinterpret_cast<const u32x4_t*>(tbl + (size_t)id[0] * 16);
              else wf[tt] = make_wfrag<S, LMODE, SEM, XDT>(tbl, id, K, L.active_mask, rs);
            }
            // keep the scheduler from sinking the gathers back next to their MFMAs
            __builtin_amdgcn_sched_barrier(0);
            // XM_GTR: rows 0-7, then 8-15, through this wave's 8 KB scratch (piece
            // p of row r at p ^ r: conflict-free writes, and conflict-free reads
            // for the 16 lanes of a read pass); each lane reads in the half that
            // holds its row.  LDS operations of one wave complete in order, so
            // the second half's writes do not overtake the first half's reads.
            u32x4_t xt[XMODE == XM_GTR ? 16 : 1];
            if constexpr (XMODE == XM_GTR) {
              uint8_t* sw = xscr + (size_t)wave * kDecodeXScratchBytes;
  #pragma unroll
              for (int h = 0; h < 2; ++h) {
                if (8 * h < M) {
  #pragma unroll
                  for (int u = 0; u < 8; ++u)
                    if (8 * h + u < M)
                      *reinterpret_cast<u32x4_t*>(sw + u * 1024 + ((lane ^ (8 * h + u)) & 63) * 16) = xv[8 * h + u];
                  if ((xm >> 3) == h) {
  #pragma unroll
                    for (int tt = 0; tt < 16; ++tt)
                      xt[tt] = *reinterpret_cast<const u32x4_t*>(sw + (xm - 8 * h) * 1024 + (((16 * q + tt) ^ xm) & 63) * 16);
                  }
                }
              }
            }
  #pragma unroll
            for (int tt = 0; tt < 16; ++tt) acc = mfma16<XDT>(x_frag(tt, xt), wf[tt], acc);
          }
        };
        // (scale-folded tables only: there the item loop has almost no VALU
        // work, c3 down_proj 12.9 -> 12.0 us; the multi-stage combine is
        // VALU-bound and the broadcasts made it slower)
        if constexpr (XMODE == XM_LDS && SCALED) {
          if (M == 1) item(std::true_type{});
          else item(std::false_type{});
        } else {
          item(std::false_type{});
        }
      }
      if (live && ++ct_c == CPT) {
        // tile done: park this wave's partial (rows m < M) in LDS
        ct_c = 0;
        float* pb = part + ((size_t)ct_t * NW + wave) * M16;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (4 * q + e < M) pb[(4 * q + e) * 16 + nl] = acc[e];  // lane holds D[4q + e][nl]
        ++ct_t;
      }
    }
  }

  // ---- epilogue: sum the NW partials of every tile, store M x 16 outputs ----
  // The only global stores of the kernel: none is pending while index loads
  // are in flight, so the loads' waits stay in-order partial waits.
  __syncthreads();
  for (int e = tid; e < n_tiles_wg * M16; e += blockDim.x) {
    const int k = e / M16;
    const int o = e - k * M16;
    const int m = o >> 4;
    const int nn = o & 15;
    const int2 orow = reinterpret_cast<const int2*>(tmeta)[2 * k];  // {first output row, rows}
    const float* pp = part + (size_t)k * NW * M16 + o;
    float v = 0.0f;
    for (int w = 0; w < NW; ++w) v += pp[w * M16];
    if (nn < orow.y) store_output(E, m, orow.x + nn, v);
  }
}

template <int S, typename IdT, int LMODE, int SEM, int XDT, bool SCALED>
static hipError_t decode_go(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, const void* x, int M,
                            const DecodePlan& P, hipStream_t st) {
  if (P.grid < 1) return hipSuccess;
  auto kern = P.xmode == XM_REG    ? rvq_decode_kernel<S, IdT, LMODE, SEM, XDT, XM_REG, SCALED, 1>
              : P.xmode == XM_LDS  ? rvq_decode_kernel<S, IdT, LMODE, SEM, XDT, XM_LDS, SCALED, 1>
              : P.xmode == XM_GREG ? rvq_decode_kernel<S, IdT, LMODE, SEM, XDT, XM_GREG, SCALED, 1>
              : P.xmode == XM_GTR  ? rvq_decode_kernel<S, IdT, LMODE, SEM, XDT, XM_GTR, SCALED, 1>
                                   : rvq_decode_kernel<S, IdT, LMODE, SEM, XDT, XM_GLOBAL, SCALED, 1>;
  if constexpr (!SCALED) {
    if (P.xmode == XM_REG && P.groups == 2) kern = rvq_decode_kernel<S, IdT, LMODE, SEM, XDT, XM_REG, false, 2>;
  }
  hipError_t e = allow_max_lds(reinterpret_cast<const void*>(kern));
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(P.grid), dim3(kDecodeMaxThreads), P.lds, st, L, D, E,
                     reinterpret_cast<const uint16_t*>(x), M, P.share, P.nslots);
  return hipGetLastError();
}

template <int S, typename IdT, int XDT>
static hipError_t decode_sem(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, int sem, int lmode,
                             const void* x, int M, const DecodePlan& P, hipStream_t st) {
  if constexpr (S == 1) {
    // one stage: the row-scale product is folded into the staged table when
    // every 16-row tile has a single scale value (decode_scaled_tables)
    const bool scaled = decode_scaled_tables(L.num_stages, L.scale_rows);
    if (sem == SEM_FAST)
      return scaled ? decode_go<S, IdT, LM_A16, SEM_FAST, XDT, true>(L, D, E, x, M, P, st)
                    : decode_go<S, IdT, LM_A16, SEM_FAST, XDT, false>(L, D, E, x, M, P, st);
    return scaled ? decode_go<S, IdT, LM_A16, SEM_RECON, XDT, true>(L, D, E, x, M, P, st)
                  : decode_go<S, IdT, LM_A16, SEM_RECON, XDT, false>(L, D, E, x, M, P, st);
  } else {
    if (sem == SEM_FAST) return decode_go<S, IdT, LM_A16, SEM_FAST, XDT, false>(L, D, E, x, M, P, st);
    if (lmode == LM_H16) return decode_go<S, IdT, LM_H16, SEM_RECON, XDT, false>(L, D, E, x, M, P, st);
    return decode_go<S, IdT, LM_F32, SEM_RECON, XDT, false>(L, D, E, x, M, P, st);
  }
}

// Entry for one (activation dtype, index width); explicitly instantiated in
// rvq_decode_<x>_<ids>.hip so the variants compile in parallel.
template <int XDT, typename IdT>
hipError_t decode_entry(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, int sem, int lmode,
                        const void* x, int M, const DecodePlan& P, hipStream_t st) {
  switch (L.num_stages) {
    case 1: return decode_sem<1, IdT, XDT>(L, D, E, sem, lmode, x, M, P, st);
    case 2: return decode_sem<2, IdT, XDT>(L, D, E, sem, lmode, x, M, P, st);
    case 3: return decode_sem<3, IdT, XDT>(L, D, E, sem, lmode, x, M, P, st);
    default: return decode_sem<4, IdT, XDT>(L, D, E, sem, lmode, x, M, P, st);
  }
}

}  // namespace wal
