// rvq_fragment.h -- codebook staging and exact 8-weight fragment dequantisation
// for the MFMA kernels (block_size 8, 1..4 stages).
//
// LDS holds every stage's codebook in one of three forms (LdsMode):
//   LM_A16: one 16-bit value per element, already the per-stage term the
//           weight formula starts from:
//             RECON, S = 1: a = rne_x(0 + v)           (v = f32(cb) [* f32(ss)])
//             FAST        : c = rne_x(rne_x(cb) [* rne_x(ss)])
//   LM_H16: the raw fp16 codebook (RECON, S >= 2, fp16 codebooks, no stage
//           scales); stages are summed in fp32 with v_fma_mix_f32.
//   LM_F32: fp32 stage values v (RECON, S >= 2, any other codebook/scales).
// A fragment is the 8 weights W[r, 8b .. 8b+7] of one block, packed as the
// 4-dword B operand of v_mfma_f32_16x16x32_{bf16,f16}.
#pragma once

#include "rvq_kernels.h"

namespace wal {

template <int LMODE>
__host__ __device__ constexpr int lds_entry_bytes() { return LMODE == LM_F32 ? 32 : 16; }

// The buffers of one row group that the fragment kernels read, with the stage
// count fixed at compile time so every per-stage pointer has a static index.
template <int S>
struct GroupPtrs {
  const void* ids[S];
  const void* cb[S];
  const void* row_scale;
  const void* stage_scales;
};

template <int S>
struct FragTile {
  GroupPtrs<S> p;
  int32_t group;
  int32_t row0;      // first row inside the group
  int32_t rows;
  int32_t out_row0;  // first output row
  int32_t grows;     // rows of the group
};

template <int S>
WAL_DEVICE FragTile<S> get_frag_tile(const LayerArgs& L, int t) {
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
    f.row0 = t * L.tile_rows;
    f.rows = min(L.tile_rows, L.g0.rows - f.row0);
    f.out_row0 = L.g0.row0 + f.row0;
    f.grows = L.g0.rows;
  } else {
    typedef const __attribute__((address_space(1))) PlanHeader g_header_t;
    typedef const __attribute__((address_space(1))) PlanTile g_tile_t;
    typedef const __attribute__((address_space(1))) wal_rvq_group g_group_t;
    const __attribute__((address_space(1))) char* base = (const __attribute__((address_space(1))) char*)(L.plan);
    g_header_t* H = (g_header_t*)base;
    g_tile_t* tiles = (g_tile_t*)(base + H->tiles_offset[L.tile_kind]);
    g_tile_t* pt = tiles + t;
    g_group_t* G = (g_group_t*)(base + H->groups_offset) + pt->group;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      f.p.ids[s] = G->stage_ids[s];
      f.p.cb[s] = G->codebooks[s];
    }
    f.p.row_scale = G->row_scale;
    f.p.stage_scales = G->stage_scales;
    f.group = pt->group;
    f.row0 = pt->row0;
    f.rows = pt->rows;
    f.out_row0 = pt->out_row0;
    f.grows = G->rows;
  }
  return f;
}

// Row-scale operand: rf = rne_x(row_scale) as fp32.  For fp16 x, r2 is that
// value as a packed fp16 pair; for bf16 x, r2 = (rf, 0) and r3 = (0, rf) as
// packed bf16 pairs, the second operands of v_dot2_f32_bf16 below.
struct RowScale {
  float rf;
  uint32_t r2;
  uint32_t r3;
};

template <int XDT>
WAL_DEVICE RowScale make_row_scale(float rs) {
  RowScale r;
  r.rf = round_dt<XDT>(rs);
  if constexpr (XDT == WAL_F16) {
    const uint32_t h = f32_to_f16_rne(rs);
    r.r2 = h | (h << 16);
    r.r3 = 0;
  } else {
    const uint32_t h = f32_to_bf16_rne(rs);
    r.r2 = h;
    r.r3 = h << 16;
  }
  return r;
}

WAL_DEVICE uint32_t pk_mul_f16(uint32_t a, uint32_t b) {
  f16x2_t r = __builtin_bit_cast(f16x2_t, a) * __builtin_bit_cast(f16x2_t, b);
  return __builtin_bit_cast(uint32_t, r);
}
WAL_DEVICE uint32_t pk_add_f16(uint32_t a, uint32_t b) {
  f16x2_t r = __builtin_bit_cast(f16x2_t, a) + __builtin_bit_cast(f16x2_t, b);
  return __builtin_bit_cast(uint32_t, r);
}

// rne_bf16(a_i * s) for the 8 bf16 values a of one fragment (4 packed pairs),
// s = rne_bf16(row_scale): per pair, v_dot2_f32_bf16 against (s, 0) and
// (0, s) gives the exact fp32 products a.lo * s and a.hi * s (a product of two
// bf16 values has at most 16 significant bits; the other term is +-0 and the
// addend 0, so only the sign of a zero product can differ from a plain
// multiply, which no fp32 sum that starts at +0 can observe), and
// v_cvt_pk_bf16_f32 rounds the pair to nearest-even.  Finite inputs only.
//
// One asm block: a dot result must be three wait states old before a VALU
// reads it, which the compiler cannot see through inline asm.  The order
// below leaves at least three instructions between each dot and the pack
// that reads it; the closing s_nop gives the two wait states a VALU result
// needs before an MFMA reads it.
WAL_DEVICE u32x4_t scale_frag_bf16(const u32x4_t& a, uint32_t slo, uint32_t shi) {
  u32x4_t w;
  float t0, t1, t2, t3, t4, t5, t6, t7;
  asm("v_dot2_f32_bf16 %4, %12, %16, 0\n\t"
      "v_dot2_f32_bf16 %5, %12, %17, 0\n\t"
      "v_dot2_f32_bf16 %6, %13, %16, 0\n\t"
      "v_dot2_f32_bf16 %7, %13, %17, 0\n\t"
      "v_dot2_f32_bf16 %8, %14, %16, 0\n\t"
      "v_dot2_f32_bf16 %9, %14, %17, 0\n\t"
      "v_dot2_f32_bf16 %10, %15, %16, 0\n\t"
      "v_dot2_f32_bf16 %11, %15, %17, 0\n\t"
      "v_cvt_pk_bf16_f32 %0, %4, %5\n\t"
      "v_cvt_pk_bf16_f32 %1, %6, %7\n\t"
      "v_cvt_pk_bf16_f32 %2, %8, %9\n\t"
      "v_cvt_pk_bf16_f32 %3, %10, %11\n\t"
      "s_nop 1"
      : "=&v"(w[0]), "=&v"(w[1]), "=&v"(w[2]), "=&v"(w[3]), "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3),
        "=&v"(t4), "=&v"(t5), "=&v"(t6), "=&v"(t7)
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(slo), "v"(shi));
  return w;
}

// rne_bf16(a_i * rf) with the sign of every product kept: each bf16 value is
// widened to fp32 and multiplied (exact: at most 16 significant bits), then
// the pair is rounded to nearest-even.  For a dense weight, where a -0
// (a -0 codeword under FAST semantics, or a negative scale) is observable.
WAL_DEVICE u32x4_t scale_frag_bf16_signed(const u32x4_t& a, float rf) {
  u32x4_t w;
#pragma unroll
  for (int pr = 0; pr < 4; ++pr)
    w[pr] = pack_bf16(__uint_as_float(a[pr] << 16) * rf, __uint_as_float(a[pr] & 0xffff0000u) * rf);
  return w;
}

// rne_x(a * rf) for the 8 x-dtype values of a fragment (finite).  SIGNED_ZERO:
// keep the sign of a zero product (dense weights); a product's zero sign
// cannot change a matrix product whose sums start at +0, so the MFMA kernels
// take the cheaper bf16 form.
template <int XDT, bool SIGNED_ZERO = false>
WAL_DEVICE u32x4_t scale_frag(const u32x4_t& a, const RowScale& rs) {
  if constexpr (XDT == WAL_F16) {
    u32x4_t w;
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) w[pr] = pk_mul_f16(a[pr], rs.r2);
    return w;
  } else if constexpr (SIGNED_ZERO) {
    return scale_frag_bf16_signed(a, rs.rf);
  } else {
    return scale_frag_bf16(a, rs.r2, rs.r3);
  }
}

// Round a pair to x dtype (nearest-even) and pack it: the hardware conversion,
// exact for finite values.
template <int XDT>
WAL_DEVICE uint32_t pack_x(float lo, float hi) {
  if constexpr (XDT == WAL_F16) return pack_f16(lo, hi);
  else return pack_bf16(lo, hi);
}

// Convert one raw codebook entry (8 values; fp32 codebooks use both halves of
// raw) of stage s into its LDS form at entry e.
template <int LMODE, int SEM, int XDT, bool SCALE_TABLE>
WAL_DEVICE void store_codebook_entry(uint8_t* lds, int e, int s, const u32x4_t (&raw)[2], int cb_dtype,
                                     bool has_ss, float ss, const RowScale& rs) {
  if constexpr (LMODE == LM_H16) {
    // fp16 copy.  Stage 0 is stored as 0 + v (-0 becomes +0), the first add
    // of the reference's zero-initialised fp32 sum, so the fragment code can
    // sum the stages without a leading zero.
    u32x4_t a = raw[0];
    if (s == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t w = a[j];
        if ((w & 0xffffu) == 0x8000u) w &= 0xffff0000u;
        if ((w >> 16) == 0x8000u) w &= 0x0000ffffu;
        a[j] = w;
      }
    }
    *reinterpret_cast<u32x4_t*>(lds + (size_t)e * 16) = a;
  } else if (LMODE == LM_A16 && SEM == SEM_RECON && cb_dtype == WAL_F16 && !has_ss) {
    // The common case in one exact op per value: v_fma_mix_f32 converts the
    // fp16 value and adds it to +0 (the reference's zero-initialised fp32
    // sum), then a hardware nearest-even pack rounds the pair to x dtype.
    u32x4_t o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = pack_x<XDT>(mix_acc_lo(0.0f, raw[0][j]), mix_acc_hi(0.0f, raw[0][j]));
    if constexpr (SCALE_TABLE) o = scale_frag<XDT>(o, rs);
    *reinterpret_cast<u32x4_t*>(lds + (size_t)e * 16) = o;
  } else {
    float v[8];
    if (cb_dtype == WAL_F32) {
#pragma unroll
      for (int j = 0; j < 4; ++j) { v[j] = __uint_as_float(raw[0][j]); v[4 + j] = __uint_as_float(raw[1][j]); }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t w = raw[0][j];
        if (cb_dtype == WAL_F16) { v[2 * j] = f16_to_f32(w & 0xffffu); v[2 * j + 1] = f16_to_f32(w >> 16); }
        else { v[2 * j] = bf16_to_f32(w & 0xffffu); v[2 * j + 1] = bf16_to_f32(w >> 16); }
      }
    }
    if constexpr (LMODE == LM_F32) {
      // Stage 0 is stored as 0 + v (the reference's zero-initialised sum);
      // -0 + u == u for every u, so other stages are stored unchanged.
      const float z = s == 0 ? 0.0f : -0.0f;
      u32x4_t a, b;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        a[j] = __float_as_uint(z + (has_ss ? v[j] * ss : v[j]));
        b[j] = __float_as_uint(z + (has_ss ? v[4 + j] * ss : v[4 + j]));
      }
      u32x4_t* dst = reinterpret_cast<u32x4_t*>(lds + (size_t)e * 32);
      dst[0] = a;
      dst[1] = b;
    } else {  // LM_A16
      // hardware round-to-nearest-even packs (finite codebooks)
      u32x4_t o;
      if constexpr (SEM == SEM_FAST) {
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = pack_x<XDT>(v[2 * j], v[2 * j + 1]);  // c = rne_x(cb)
        if (has_ss) o = scale_frag<XDT, true>(o, make_row_scale<XDT>(ss));      // rne_x(c * rne_x(ss))
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float a0 = has_ss ? v[2 * j] * ss : v[2 * j];
          const float a1 = has_ss ? v[2 * j + 1] * ss : v[2 * j + 1];
          o[j] = pack_x<XDT>(0.0f + a0, 0.0f + a1);  // rne_x(0 + v), the zero-initialised fp32 sum
        }
      }
      if constexpr (SCALE_TABLE) o = scale_frag<XDT>(o, rs);
      *reinterpret_cast<u32x4_t*>(lds + (size_t)e * 16) = o;
    }
  }
}

// Codebook staging.  16-bit codebooks go in batches: every thread issues the
// loads of U entries per stage (entries k0 + u * nt) before converting and
// storing any, so one batch costs one memory round trip; the loads are
// straight-line (indices past K are clamped and their results dropped), so
// callers can issue a batch early and store it later.
template <int S>
__host__ __device__ constexpr int stage_batch() { return S >= 8 ? 1 : 8 / S; }

template <int S>
WAL_DEVICE void load_codebook_batch(u32x4_t (&raw)[S][stage_batch<S>()], const GroupPtrs<S>& g, int K, int k0,
                                    int nt) {
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const char* cb = static_cast<const char*>(g.cb[s]);
#pragma unroll
    for (int u = 0; u < stage_batch<S>(); ++u) raw[s][u] = ldg128(cb + (size_t)min(k0 + u * nt, K - 1) * 16);
  }
}

// Stage scales of a group as fp32 (1.0 when absent).
template <int S>
WAL_DEVICE void load_stage_scales(float (&ssv)[S], const GroupPtrs<S>& g, const DtypeArgs& D) {
#pragma unroll
  for (int s = 0; s < S; ++s) ssv[s] = g.stage_scales != nullptr ? load_f(g.stage_scales, D.sc_dtype, s) : 1.0f;
}

template <int S, int LMODE, int SEM, int XDT, bool SCALE_TABLE>
WAL_DEVICE void store_codebook_batch(uint8_t* lds, const u32x4_t (&raw)[S][stage_batch<S>()], int K, int k0, int nt,
                                     const DtypeArgs& D, bool has_ss, const float (&ssv)[S], const RowScale& rs) {
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int u = 0; u < stage_batch<S>(); ++u) {
      const int k = k0 + u * nt;
      if (k < K) {
        const u32x4_t r2[2] = {raw[s][u], u32x4_t{0, 0, 0, 0}};
        store_codebook_entry<LMODE, SEM, XDT, SCALE_TABLE>(lds, s * K + k, s, r2, D.cb_dtype, has_ss, ssv[s], rs);
      }
    }
}

// Fill LDS with the codebooks of one group (all threads of the block take
// part), 16-bit codebooks batch by batch; fp32 codebooks (rare) take a plain
// loop.  SCALE_TABLE (LM_A16 only): every staged value is replaced by its
// product with the row scale rs, rounded as the reference rounds
// W = rne_x(a * rne_x(row_scale)).  first_batch_loaded: the caller already
// issued the first batch into raw (load_codebook_batch with k0 = threadIdx.x).
template <int S, int LMODE, int SEM, int XDT, bool SCALE_TABLE = false>
WAL_DEVICE void stage_codebooks(uint8_t* lds, const GroupPtrs<S>& g, int K, const DtypeArgs& D,
                                const RowScale& rs = RowScale{0.0f, 0u, 0u},
                                const u32x4_t (*first)[S][stage_batch<S>()] = nullptr) {
  static_assert(!SCALE_TABLE || LMODE == LM_A16, "scaled tables are 16-bit");
  constexpr int U = stage_batch<S>();
  const int nt = blockDim.x;
  const bool has_ss = g.stage_scales != nullptr;
  float ssv[S];
  load_stage_scales<S>(ssv, g, D);
  if (D.cb_dtype == WAL_F32) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const char* cb = static_cast<const char*>(g.cb[s]);
      for (int k = threadIdx.x; k < K; k += nt) {
        const u32x4_t raw[2] = {ldg128(cb + (size_t)k * 32), ldg128(cb + (size_t)k * 32 + 16)};
        store_codebook_entry<LMODE, SEM, XDT, SCALE_TABLE>(lds, s * K + k, s, raw, WAL_F32, has_ss, ssv[s], rs);
      }
    }
    return;
  }
  int k0 = threadIdx.x;
  if (first != nullptr) {
    store_codebook_batch<S, LMODE, SEM, XDT, SCALE_TABLE>(lds, *first, K, k0, nt, D, has_ss, ssv, rs);
    k0 += U * nt;
  }
  for (; k0 < K; k0 += U * nt) {
    u32x4_t raw[S][U];
    load_codebook_batch<S>(raw, g, K, k0, nt);
    store_codebook_batch<S, LMODE, SEM, XDT, SCALE_TABLE>(lds, raw, K, k0, nt, D, has_ss, ssv, rs);
  }
}


// 8-weight fragment for stage ids id[0..S-1]: the pre-scale values in x
// dtype (RECON: rne_x of the fp32 stage sum; FAST: the x-dtype stage sum),
// then the row-scale product.
// The LDS entries of one block's S codewords (gather_wfrag), and the 8
// weights made from them (combine_wfrag); split so that a caller can issue the
// gathers of several blocks before it waits for the first.
template <int S, int LMODE>
struct WfragRaw {
  u32x4_t c[S][LMODE == LM_F32 ? 2 : 1];
};

template <int S, int LMODE>
WAL_DEVICE WfragRaw<S, LMODE> gather_wfrag(const uint8_t* lds, const uint32_t (&id)[S], int K) {
  WfragRaw<S, LMODE> r;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    if constexpr (LMODE == LM_F32) {
      const u32x4_t* p = reinterpret_cast<const u32x4_t*>(lds + ((size_t)s * K + id[s]) * 32);
      r.c[s][0] = p[0];
      r.c[s][1] = p[1];
    } else {
      r.c[s][0] = *reinterpret_cast<const u32x4_t*>(lds + ((size_t)s * K + id[s]) * 16);
    }
  }
  return r;
}

// gather_wfrag from a table replicated 1 << rshift times entry by entry
// (entry e, copy c at ((e << rshift) + c) * ESZ); lds_lane already points at
// this lane's copy.  Lanes that read in the same LDS cycle use different
// copies, which sit in different banks, so random codewords do not conflict.
template <int S, int LMODE>
WAL_DEVICE WfragRaw<S, LMODE> gather_wfrag_rep(const uint8_t* lds_lane, const uint32_t (&id)[S], int K, int rshift) {
  constexpr int ESZ = LMODE == LM_F32 ? 32 : 16;
  WfragRaw<S, LMODE> r;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const uint8_t* p = lds_lane + ((uint32_t)((s * K + (int)id[s]) * ESZ) << rshift);
    r.c[s][0] = *reinterpret_cast<const u32x4_t*>(p);
    if constexpr (LMODE == LM_F32) r.c[s][1] = *reinterpret_cast<const u32x4_t*>(p + 16);
  }
  return r;
}

template <int S, int LMODE, int SEM, int XDT, bool SIGNED_ZERO = false>
WAL_DEVICE u32x4_t combine_wfrag(const WfragRaw<S, LMODE>& raw, uint32_t active, const RowScale& rs) {
  u32x4_t a;
  if constexpr (LMODE == LM_F32) {
    const auto& c = raw.c;
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) {
      const int h = pr >> 1, o = (pr & 1) * 2;
      float tl = __uint_as_float(c[0][h][o]);  // staged as 0 + v
      float th = __uint_as_float(c[0][h][o + 1]);
#pragma unroll
      for (int s = 1; s < S; ++s) {
        tl = tl + __uint_as_float(c[s][h][o]);
        th = th + __uint_as_float(c[s][h][o + 1]);
      }
      a[pr] = pack_x<XDT>(tl, th);
    }
  } else {
    u32x4_t c[S];
#pragma unroll
    for (int s = 0; s < S; ++s) c[s] = raw.c[s][0];
    if constexpr (LMODE == LM_H16) {
      // stage 0 is staged as 0 + v, so c0 + c1 + ... equals the reference's
      // ((0 + c0) + c1) + ... bit for bit, signed zeros included
#pragma unroll
      for (int pr = 0; pr < 4; ++pr) {
        float tl = mix_add_lo(c[0][pr], c[1][pr]);
        float th = mix_add_hi(c[0][pr], c[1][pr]);
#pragma unroll
        for (int s = 2; s < S; ++s) {
          tl = mix_acc_lo(tl, c[s][pr]);
          th = mix_acc_hi(th, c[s][pr]);
        }
        a[pr] = pack_x<XDT>(tl, th);
      }
    } else if constexpr (SEM == SEM_RECON) {  // LM_A16, S == 1
      a = c[0];
    } else {  // LM_A16, FAST
#pragma unroll
      for (int pr = 0; pr < 4; ++pr) {
        uint32_t v = 0;
        bool first = true;
#pragma unroll
        for (int s = 0; s < S; ++s) {
          if (!(active & (1u << s))) continue;
          if (first) {
            v = c[s][pr];
            first = false;
          } else if constexpr (XDT == WAL_F16) {
            v = pk_add_f16(v, c[s][pr]);
          } else {
            v = pack_bf16(lo_bf16(v) + lo_bf16(c[s][pr]), hi_bf16(v) + hi_bf16(c[s][pr]));
          }
        }
        a[pr] = v;
      }
    }
  }
  return scale_frag<XDT, SIGNED_ZERO>(a, rs);
}

// The 8 weights of one block: gather the S codewords from the staged table,
// rebuild the reference's dequantised values, apply the row scale.
template <int S, int LMODE, int SEM, int XDT>
WAL_DEVICE u32x4_t make_wfrag(const uint8_t* lds, const uint32_t (&id)[S], int K, uint32_t active,
                              const RowScale& rs) {
  return combine_wfrag<S, LMODE, SEM, XDT>(gather_wfrag<S, LMODE>(lds, id, K), active, rs);
}

template <int XDT>
WAL_DEVICE f32x4_t mfma16(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  if constexpr (XDT == WAL_F16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  }
}


// 32 x 32 x 16 product: lane l holds A row l % 32 and B column l % 32, k
// elements 8 (l / 32) .. + 8 of each; D[i][j] is element
// (i % 4) + 4 (i / 8) of lane j + 32 ((i / 4) % 2).  Same operand registers
// as mfma16 for twice the flops: measured on gfx950, a VALU instruction of
// another wave (or of the same one) takes about 1.3 cycles from a stream of
// these against about 3 from a stream of 16 x 16 x 32 products.
template <int XDT>
WAL_DEVICE f32x16_t mfma32(const u32x4_t& a, const u32x4_t& b, const f32x16_t& c) {
  if constexpr (XDT == WAL_F16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  }
}

// ---- staging from a codebook image ------------------------------------------
// An image holds, per group, the S x K entries already in their LDS form (the
// same bytes store_codebook_entry writes), so staging a group is a copy of
// S * K * entry_bytes bytes in 16-byte pieces, batch by batch (8 pieces per
// thread); SCALE_TABLE (16-bit entries) multiplies every staged fragment by
// the row scale with the reference's rounding on the way.
constexpr int kImageBatch = 8;

WAL_DEVICE void load_image_batch(u32x4_t (&r)[kImageBatch], const uint8_t* img, int n16, int i0, int nt) {
#pragma unroll
  for (int u = 0; u < kImageBatch; ++u) r[u] = ldg128(img + (size_t)min(i0 + u * nt, n16 - 1) * 16);
}

template <int XDT, bool SCALE_TABLE>
WAL_DEVICE void store_image_batch(uint8_t* lds, const u32x4_t (&r)[kImageBatch], int n16, int i0, int nt,
                                  const RowScale& rs) {
#pragma unroll
  for (int u = 0; u < kImageBatch; ++u) {
    const int i = i0 + u * nt;
    if (i < n16) {
      u32x4_t v = r[u];
      if constexpr (SCALE_TABLE) v = scale_frag<XDT>(v, rs);
      *reinterpret_cast<u32x4_t*>(lds + (size_t)i * 16) = v;
    }
  }
}

// Stage n16 pieces of an image into LDS; the first batch may already be in
// `first` (issued early by the caller with i0 = threadIdx.x).
template <int XDT, bool SCALE_TABLE>
WAL_DEVICE void stage_image(uint8_t* lds, const uint8_t* img, int n16, const RowScale& rs,
                            const u32x4_t (*first)[kImageBatch] = nullptr) {
  const int nt = blockDim.x;
  int i0 = threadIdx.x;
  if (first != nullptr) {
    store_image_batch<XDT, SCALE_TABLE>(lds, *first, n16, i0, nt, rs);
    i0 += kImageBatch * nt;
  }
  for (; i0 < n16; i0 += kImageBatch * nt) {
    u32x4_t r[kImageBatch];
    load_image_batch(r, img, n16, i0, nt);
    store_image_batch<XDT, SCALE_TABLE>(lds, r, n16, i0, nt, rs);
  }
}

}  // namespace wal
