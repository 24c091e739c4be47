// rvq_plan.h -- launch planning for the block-size-8 MFMA kernels, on the host.
//
// wal_rvq_linear and wal_rvq_linear_info run the same planner, so what the
// query reports is what a call launches.  The decode planner picks where the
// MFMA's activation fragments come from (XMode), how many codebook table slots
// a workgroup keeps in LDS, and the grid; the prefill planner picks the tile
// shape.  Both honour an environment override for tests and tuning:
//   WAL2026_DECODE_XMODE = reg | lds | greg | gtr | global
//   WAL2026_PREFILL_TILE = short | tall | wide
#pragma once

#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "wal2026_amd.h"

namespace wal {

constexpr int kLdsMaxBytes = 160 * 1024;  // LDS per workgroup on gfx950

// ---- decode (M <= 16) ------------------------------------------------------
constexpr int kDecodeMaxWaves = 8;
constexpr int kDecodeMaxThreads = kDecodeMaxWaves * 64;
constexpr int kDecodeTileMetaBytes = 16;         // {out_row0, rows, -, -} per tile
constexpr int kDecodeXScratchBytes = 8 * 1024;   // XM_GTR transpose scratch per wave (8 rows x 1 KB)

// Where the decode kernel's activation fragments come from.
enum XMode : int {
  XM_GLOBAL = WAL_XMODE_GLOBAL,  // read per item from global memory (L2)
  XM_LDS = WAL_XMODE_LDS,        // x staged in LDS, fragments read per item
  XM_REG = WAL_XMODE_REG,        // x staged in LDS; each wave owns one chunk (CPT == 1), so its
                                 // 16 fragments are read once and kept in registers
  XM_GREG = WAL_XMODE_GREG,      // as XM_REG, but the 16 fragments come straight from global
                                 // memory (large M: x beside two tables would not fit LDS)
  XM_GTR = WAL_XMODE_GTR         // x too large for LDS: per item, each load reads one contiguous
                                 // 1 KB run of an x row and the fragments are transposed
                                 // through a per-wave LDS scratch
};

// Bytes of LDS a decode launch needs: nslots staged tables (the codebooks of
// up to two groups / scale runs, esz bytes per entry), the per-tile partial
// sums of every wave and the output rows of every tile (max_tiles tiles per
// workgroup), a 256-byte zero row, (xlds) the activation rows and (xscr) the
// XM_GTR transpose scratch.
inline __host__ __device__ size_t decode_lds_bytes(int esz, int S, int K, bool xlds, int M, int in, int nw,
                                                   int max_tiles, int nslots, bool xscr) {
  return (size_t)nslots * S * K * esz + (size_t)max_tiles * ((size_t)nw * M * 16 * sizeof(float) + kDecodeTileMetaBytes) +
         256 + (xlds ? (size_t)M * in * sizeof(uint16_t) : 0) + (xscr ? (size_t)nw * kDecodeXScratchBytes : 0);
}

struct DecodePlan {
  int xmode;
  int nslots;
  int grid;
  int share;  // tiles of the largest workgroup share
  size_t lds;
  int groups;  // wave groups (2: two halves of the waves take alternate tiles)
};

// WAL2026_DECODE_XMODE, or -1 (planner's choice); -2 for an unknown value.
inline int decode_xmode_override() {
  const char* f = getenv("WAL2026_DECODE_XMODE");
  if (f == nullptr || *f == 0) return -1;
  if (strcmp(f, "global") == 0) return XM_GLOBAL;
  if (strcmp(f, "lds") == 0) return XM_LDS;
  if (strcmp(f, "reg") == 0) return XM_REG;
  if (strcmp(f, "greg") == 0) return XM_GREG;
  if (strcmp(f, "gtr") == 0) return XM_GTR;
  return -2;
}

// Plan a decode launch of n_tiles 16-row tiles over n_cu CUs.  esz: bytes per
// staged codebook entry; S, K: stages and entries per table; B: blocks per
// row (a multiple of 16); segments: a workgroup's tiles can need two tables
// (several groups, or scale-folded tables with more than one scale run).
// force: an XMode, or -1 for the planner's choice.  Returns false when no
// layout fits (or the forced one does not apply).
//
// Each workgroup takes an equal share of the tiles and keeps the partial sums
// of its whole share in LDS; when a share does not fit, the grid grows until
// it does.  Candidate layouts in order of preference; the first whose grid
// fits one round of workgroups (one per CU) wins, else the one with the
// fewest rounds: x in LDS (in registers when each wave owns one chunk), x
// straight from global memory into registers (one chunk per wave), x row runs
// transposed per item (M > 4), fragments from global memory per item.  Two
// table slots before one.
inline bool plan_decode(int esz, int S, int K, int M, int in, int B, int n_tiles, int n_cu, bool segments, int force,
                        DecodePlan* out) {
  const int nw = kDecodeMaxWaves;
  if (n_cu < 1) n_cu = 256;
  const int nchunk = (B + 63) / 64;
  const bool one_chunk = nchunk <= nw;
  struct Cand { int xmode, nslots; };
  const Cand cands[] = {{one_chunk ? XM_REG : XM_LDS, 2}, {XM_GREG, 2}, {one_chunk ? XM_REG : XM_LDS, 1},
                        {XM_GREG, 1}, {XM_GTR, 2}, {XM_GTR, 1}, {XM_GLOBAL, 2}, {XM_GLOBAL, 1}};
  const Cand forced[] = {{force, 2}, {force, 1}};
  const Cand* list = force >= 0 ? forced : cands;
  const int n = force >= 0 ? 2 : (int)(sizeof(cands) / sizeof(cands[0]));
  if (force >= 0 && (force == XM_REG || force == XM_GREG) && !one_chunk) return false;
  if (force < -1 || force > XM_GTR) return false;
  int best_rounds = 1 << 30;
  bool found = false;
  for (int i = 0; i < n; ++i) {
    const Cand& c = list[i];
    if (c.nslots == 2 && !segments) continue;
    if (force < 0) {
      if (c.xmode == XM_GREG && !one_chunk) continue;
      if (c.xmode == XM_GTR && M <= 4) continue;  // up to 4 rows, direct loads touch at most 16 lines
    }
    const bool xlds = c.xmode == XM_REG || c.xmode == XM_LDS;
    const bool xscr = c.xmode == XM_GTR;
    const size_t fixed = decode_lds_bytes(esz, S, K, xlds, M, in, nw, 0, c.nslots, xscr);
    const size_t per_tile = (size_t)nw * M * 16 * sizeof(float) + kDecodeTileMetaBytes;
    if (fixed + per_tile > (size_t)kLdsMaxBytes) continue;
    const int fit = (int)(((size_t)kLdsMaxBytes - fixed) / per_tile);
    int g = n_cu < n_tiles ? n_cu : n_tiles;
    const int min_grid = (n_tiles + fit - 1) / fit;
    if (g < min_grid) g = min_grid;
    if (g < 1) g = 1;
    const int rounds = (g + n_cu - 1) / n_cu;
    if (rounds < best_rounds) {
      best_rounds = rounds;
      out->xmode = c.xmode;
      out->nslots = c.nslots;
      out->grid = g;
      out->share = (n_tiles + g - 1) / g;
      out->lds = decode_lds_bytes(esz, S, K, xlds, M, in, nw, out->share, c.nslots, xscr);
      // x in registers with at most half as many chunks per row as waves
      // (in_features <= 2048): two wave groups on alternate tiles, when a
      // workgroup holds more than one tile
      out->groups = c.xmode == XM_REG && 2 * nchunk <= nw && out->share > 1 ? 2 : 1;
      found = true;
    }
    if (rounds <= 1) break;
  }
  return found;
}

// ---- prefill (M > 16) ------------------------------------------------------
enum PrefillShape : int { PS_SHORT = WAL_TILE_SHORT, PS_TALL = WAL_TILE_TALL, PS_WIDE = WAL_TILE_WIDE };

// Shapes whose kernels exist for an instance (their producer registers fit
// beside the pipeline without scratch, checked with the compiler's resource
// report).  lmode: LdsMode of rvq_kernels.h (2 = fp32 entries).
constexpr bool prefill_tall_ok(int S, int lmode) { return S <= 2 && lmode != 2; }
constexpr bool prefill_wide_ok(int S, int lmode, int id_bytes) { return !(S >= 4 && lmode == 2 && id_bytes == 2); }

// WAL2026_PREFILL_TILE, or -1; -2 for an unknown value.
inline int prefill_tile_override() {
  const char* f = getenv("WAL2026_PREFILL_TILE");
  if (f == nullptr || *f == 0) return -1;
  if (strcmp(f, "short") == 0) return PS_SHORT;
  if (strcmp(f, "tall") == 0) return PS_TALL;
  if (strcmp(f, "wide") == 0) return PS_WIDE;
  return -2;
}

// Split-K of the short tile: at most this many slices, each at least one
// unit of 8 k-steps (the kernel's kSplitUnit).
constexpr int kMaxKSplit = 32;
constexpr int kKSplitUnit = 8;

// WAL2026_PREFILL_KSPLIT (a slice count for every split-capable call, 1 = no
// split), or 0 (planner's choice); -1 for a bad value.
inline int prefill_ksplit_override() {
  const char* f = getenv("WAL2026_PREFILL_KSPLIT");
  if (f == nullptr || *f == 0) return 0;
  const int v = atoi(f);
  return v >= 1 && v <= kMaxKSplit ? v : -1;
}

struct PrefillPlan {
  int shape;   // PrefillShape
  int ksplit;  // k slices of the short tile (1: none)
  int grid;    // workgroups of the prefill kernel
  int ksteps;  // k-steps of the largest workgroup
};

// Tile shape (and split) of a prefill launch: 128 x 256 (short), 256 x 256
// (tall) or 256 x 128 (wide) x rows by weight rows, one workgroup per CU.
// Cost = rounds of workgroups x k-steps per workgroup x time per k-step,
// measured at c4 (gfx950) as 0.84 (short), 1.22 (tall), 0.76 (wide) us.  With
// split (a caller workspace), the short tile's output tiles can share their
// k-steps among ksplit workgroups when the tiles alone leave CUs idle (a
// 4096-row layer at M <= 128 is 16 workgroups), adding one pass that sums the
// fp32 partials (read at about 3 TB/s).  A forced shape the instance lacks
// falls back to short; force_ks > 0 forces the slice count of a short tile.
inline PrefillPlan plan_prefill(int S, int lmode, int id_bytes, int64_t M, int64_t N, int n_tiles256,
                                int blocks_per_row, int n_cu, int force, bool allow_split, int force_ks) {
  const bool can_tall = prefill_tall_ok(S, lmode), can_wide = prefill_wide_ok(S, lmode, id_bytes);
  const int64_t cu = n_cu > 0 ? n_cu : 256;
  const int nk = blocks_per_row / 4;
  const int nu = (nk + kKSplitUnit - 1) / kKSplitUnit;
  const int64_t mt128 = (M + 127) / 128, mt256 = (M + 255) / 256;
  const int64_t wg_short = (int64_t)n_tiles256 * mt128;
  // the short tile's slice count and cost
  int ks = 1;
  if (allow_split) {
    if (force_ks > 0) {
      ks = force_ks;
    } else if (wg_short < cu) {
      ks = (int)(cu / wg_short);
    }
    ks = ks > nu ? nu : ks;
    ks = ks > kMaxKSplit ? kMaxKSplit : ks;
    ks = ks < 1 ? 1 : ks;
  }
  auto short_cost = [&](int k) -> double {
    const double steps = k == 1 ? nk : (double)kKSplitUnit * ((nu + k - 1) / k);
    const double red = k == 1 ? 0.0 : ((double)k * M * N * 4.0 + (double)M * N * 2.0) / 3.0e6 + 2.0;
    return (double)((wg_short * k + cu - 1) / cu) * steps * 0.84 + red;
  };
  // a planned (not forced) split is kept only where it is cheaper
  if (ks > 1 && force_ks <= 0 && short_cost(ks) >= short_cost(1)) ks = 1;
  PrefillPlan p{PS_SHORT, ks, (int)(wg_short * ks), ks == 1 ? nk : kKSplitUnit * ((nu + ks - 1) / ks)};
  auto as_tall = [&]() { return PrefillPlan{PS_TALL, 1, (int)(n_tiles256 * mt256), nk}; };
  auto as_wide = [&]() { return PrefillPlan{PS_WIDE, 1, (int)(n_tiles256 * 2 * mt256), nk}; };
  if (force == PS_SHORT) return p;
  if (force == PS_TALL) return can_tall ? as_tall() : p;
  if (force == PS_WIDE) return can_wide ? as_wide() : p;
  if (M <= 128) return p;
  const double c_short = short_cost(ks);
  const double c_tall = can_tall ? (double)((n_tiles256 * mt256 + cu - 1) / cu) * nk * 1.22 : 1e300;
  const double c_wide = can_wide ? (double)((n_tiles256 * 2 * mt256 + cu - 1) / cu) * nk * 0.76 : 1e300;
  if (c_tall <= c_wide && c_tall < c_short) return as_tall();
  if (c_wide < c_short) return as_wide();
  return p;
}

}  // namespace wal
