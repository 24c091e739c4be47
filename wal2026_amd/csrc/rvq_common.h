// rvq_common.h -- shared device code for the gfx950 Block-RVQ kernels.
//
// Every kernel reproduces the reference's dequantisation of one weight element
// (src/runtime.py:379-414 for RECONSTRUCT, :568-598 for RECONSTRUCT_FAST):
//
//   RECONSTRUCT, output dtype dt:
//     t  = ((0 + v_0) + v_1) + ... + v_{S-1}    fp32, v_s = f32(cb_s[id_s][j]) [* f32(stage_scale_s)]
//     t  = t * f32(block_scale[r, b])            (if present)
//     W  = rne_dt(rne_dt(t) * rne_dt(row_scale[r]))     (dt = f32: W = t * f32(row_scale))
//   RECONSTRUCT_FAST, over the active stages s_0 < s_1 < ...:
//     c_s = rne_dt(cb_s[id_s][j]) [then rne_dt(c_s * rne_dt(stage_scale_s))]
//     a   = c_{s_0};  a = rne_dt(a + c_{s_k}) for k >= 1
//     W   = rne_dt(a * rne_dt(row_scale[r]))
//
// Products of two values that are each exact in bf16/fp16 are exact in fp32,
// so "round the fp32 product" equals torch's bf16/fp16 multiply.  The library
// is compiled with -ffp-contract=off so no add/multiply pair is fused.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wal2026_amd.h"

// Device helpers are force-inlined: a call boundary turns LDS pointers into
// flat pointers and by-value structs into stack traffic.
#define WAL_DEVICE __device__ __attribute__((always_inline)) inline
#define WAL_HOST_DEVICE __host__ __device__ __attribute__((always_inline)) inline

namespace wal {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) u32x4_t g_u32x4_t;

// 128-bit loads from the global address space.  Buffers reach the kernels as
// plain (flat) pointers; a flat load may alias LDS, which serialises it
// against LDS stores and makes every LDS wait also wait for it.  Casting to
// address space 1 gives global_load instructions with their own counter.
WAL_DEVICE u32x4_t ldg128(const void* p) { return *(g_u32x4_t*)(p); }
// Streaming variant (non-temporal): data read exactly once, kept out of the
// way of the small tables and activations that are reused.
WAL_DEVICE u32x4_t ldg128_stream(const void* p) { return __builtin_nontemporal_load((g_u32x4_t*)(p)); }
// Raw buffer loads through a resource descriptor covering [p, p + 2 GiB):
// an offset at or past kBufOOB is out of range, and the hardware returns
// zeros without a memory access (used for pipeline slots past the end of the
// work).  Dword 3 of the descriptor: 32-bit raw data format.
typedef __amdgpu_buffer_rsrc_t bufrsrc_t;
constexpr uint32_t kBufOOB = 0x80000000u;
WAL_DEVICE bufrsrc_t make_rsrc(const void* p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)kBufOOB, 0x00020000);
}
// 16 bytes at byte offset off, non-temporal (streamed once).
WAL_DEVICE u32x4_t ldbuf128_stream(bufrsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
}
WAL_DEVICE uint32_t ldbuf16(bufrsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0); }
// 16 bytes at byte offset off, cached (data other workgroups read again).
WAL_DEVICE u32x4_t ldbuf128(bufrsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Scalar element of a global buffer.
template <typename T>
WAL_DEVICE T ldg(const void* p, int64_t i) { return ((const __attribute__((address_space(1))) T*)(p))[i]; }

// ---------------------------------------------------------------------------
// Plan image (built on the host by wal_rvq_plan_build, read by kernels).
// ---------------------------------------------------------------------------
constexpr int kPlanMagic = 0x57524c31;  // "WRL1"
constexpr int kNumTileKinds = 3;
constexpr int kTileRows[kNumTileKinds] = {16, 64, 256};

struct PlanTile {
  int32_t group;
  int32_t row0;  // first row inside the group
  int32_t rows;  // rows in this tile (<= tile size)
  int32_t out_row0;  // first output row (group row0 + row0)
};

struct PlanHeader {
  int32_t magic;
  int32_t n_groups;
  int32_t groups_offset;  // bytes from the header start
  int32_t pad;
  int32_t tiles_offset[kNumTileKinds];
  int32_t n_tiles[kNumTileKinds];
};

// Kernel-side constants of one layer (passed by value).
struct LayerArgs {
  int32_t in_features;
  int32_t out_features;
  int32_t block_size;
  int32_t blocks_per_row;
  int32_t codebook_size;
  int32_t num_stages;
  int32_t scale_rows;
  int32_t n_tiles;       // for the kernel's tile kind
  int32_t tile_rows;     // rows per tile for the kernel's tile kind
  int32_t tile_kind;
  uint32_t active_mask;  // RECONSTRUCT_FAST active stages
  int32_t scale_shift;   // log2(scale_rows) when it is a power of two, else -1
  const PlanHeader* plan;  // NULL -> single group g0
  wal_rvq_group g0;
  const uint8_t* image;    // codebook image (per group: S x K staged entries) or NULL
  int32_t n_groups;
  int32_t pad2;
  // The plan's tile table for this launch's tile kind and its group table
  // (NULL without a plan): a kernel reads them without first reading the
  // plan header.
  const PlanTile* plan_tiles;
  const wal_rvq_group* plan_groups;
};

// row_scale entry of row r (inside its group): r / scale_rows, a shift when
// scale_rows is a power of two.
WAL_HOST_DEVICE int64_t scale_index(const LayerArgs& L, int64_t r) {
  return L.scale_shift >= 0 ? (r >> L.scale_shift) : r / L.scale_rows;
}

struct TileInfo {
  wal_rvq_group g;  // by value: no pointer into the kernel-argument segment
  int32_t group;
  int32_t row0;      // first row inside the group
  int32_t rows;
  int32_t out_row0;  // first output row
};

WAL_DEVICE TileInfo get_tile(const LayerArgs& L, int t) {
  TileInfo ti;
  if (L.plan == nullptr) {
    ti.g = L.g0;
    ti.group = 0;
    ti.row0 = t * L.tile_rows;
    ti.rows = min(L.tile_rows, L.g0.rows - ti.row0);
    ti.out_row0 = L.g0.row0 + ti.row0;
  } else {
    typedef const __attribute__((address_space(1))) PlanHeader g_header_t;
    typedef const __attribute__((address_space(1))) PlanTile g_tile_t;
    typedef const __attribute__((address_space(1))) wal_rvq_group g_group_t;
    const __attribute__((address_space(1))) char* base = (const __attribute__((address_space(1))) char*)(L.plan);
    g_header_t* H = (g_header_t*)base;
    g_tile_t* tiles = (g_tile_t*)(base + H->tiles_offset[L.tile_kind]);
    g_group_t* groups = (g_group_t*)(base + H->groups_offset);
    g_tile_t* pt = tiles + t;
    g_group_t* G = groups + pt->group;
    for (int s = 0; s < WAL_RVQ_MAX_STAGES; ++s) {
      ti.g.stage_ids[s] = G->stage_ids[s];
      ti.g.codebooks[s] = G->codebooks[s];
    }
    ti.g.stage_scales = G->stage_scales;
    ti.g.row_scale = G->row_scale;
    ti.g.block_scale = G->block_scale;
    ti.g.row0 = G->row0;
    ti.g.rows = G->rows;
    ti.group = pt->group;
    ti.row0 = pt->row0;
    ti.rows = pt->rows;
    ti.out_row0 = pt->out_row0;
  }
  return ti;
}

// ---------------------------------------------------------------------------
// Scalar conversions.
// ---------------------------------------------------------------------------
WAL_DEVICE float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

WAL_DEVICE float f16_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// fp32 -> bf16 round-to-nearest-even; NaN -> 0x7fc0 (torch's scalar rule).
WAL_DEVICE uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// fp32 -> fp16 round-to-nearest-even, subnormals and overflow per IEEE-754;
// NaN -> sign | 0x7e00 (torch's scalar rule).
WAL_DEVICE uint32_t f32_to_f16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7e00u;
  if (a >= 0x477ff000u) return sign | 0x7c00u;
  int e = (int)(a >> 23) - 127;
  if (e >= -14) {
    uint32_t man = a & 0x7fffffu;
    uint32_t h = ((uint32_t)(e + 15) << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return sign | h;
  }
  if (e < -25) return sign;
  uint32_t sig = (a & 0x7fffffu) | 0x800000u;
  int s = -(e + 1);
  uint32_t q = sig >> s;
  uint32_t rem = sig & ((1u << s) - 1u);
  uint32_t half = 1u << (s - 1);
  if (rem > half || (rem == half && (q & 1u))) q++;
  return sign | q;
}

template <int DT>
WAL_DEVICE float round_dt(float v) {
  if constexpr (DT == WAL_BF16) return bf16_to_f32(f32_to_bf16_rne(v));
  else if constexpr (DT == WAL_F16) return f16_to_f32(f32_to_f16_rne(v));
  else return v;
}

template <int DT>
WAL_DEVICE uint32_t to_bits16(float v) {
  if constexpr (DT == WAL_BF16) return f32_to_bf16_rne(v);
  else return f32_to_f16_rne(v);
}

// Load element i of a float buffer of runtime dtype dt as fp32 (exact).
WAL_DEVICE float load_f(const void* p, int dt, int64_t i) {
  if (dt == WAL_F16) return f16_to_f32(ldg<uint16_t>(p, i));
  if (dt == WAL_BF16) return bf16_to_f32(ldg<uint16_t>(p, i));
  return ldg<float>(p, i);
}

WAL_DEVICE int64_t load_id(const void* p, int dt, int64_t i) {
  if (dt == WAL_U8) return ldg<uint8_t>(p, i);
  if (dt == WAL_I16) return ldg<int16_t>(p, i);
  if (dt == WAL_U16) return ldg<uint16_t>(p, i);
  return ldg<int32_t>(p, i);
}

// Hardware packed conversions (round-to-nearest-even for finite inputs).
WAL_DEVICE uint32_t pack_bf16(float lo, float hi) {
  bf16x2_t r = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, r);
}
WAL_DEVICE uint32_t pack_f16(float lo, float hi) {
  f16x2_t r = {(_Float16)lo, (_Float16)hi};
  return __builtin_bit_cast(uint32_t, r);
}
WAL_DEVICE float lo_bf16(uint32_t p) { return __uint_as_float(p << 16); }
WAL_DEVICE float hi_bf16(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }
WAL_DEVICE float lo_f16(uint32_t p) { return f16_to_f32(p & 0xffffu); }
WAL_DEVICE float hi_f16(uint32_t p) { return f16_to_f32(p >> 16); }

// f32(a.lo) + f32(b.lo) / f32(a.hi) + f32(b.hi) for packed fp16 pairs: one
// v_fma_mix_f32 each (a * 1.0 + b, a single fp32 rounding == the fp32 add).
WAL_DEVICE float mix_add_lo(uint32_t a, uint32_t b) {
  float r;
  asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,1]" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
WAL_DEVICE float mix_add_hi(uint32_t a, uint32_t b) {
  float r;
  asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,1] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// t + f32(a.lo) / t + f32(a.hi) for an fp32 t and a packed fp16 pair.
WAL_DEVICE float mix_acc_lo(float t, uint32_t a) {
  float r;
  asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(a), "v"(t));
  return r;
}
WAL_DEVICE float mix_acc_hi(float t, uint32_t a) {
  float r;
  asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(a), "v"(t));
  return r;
}

}  // namespace wal
