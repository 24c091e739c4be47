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

// Fill LDS with the codebooks of group g (all threads of the block take part).
template <int S, int LMODE, int SEM, int XDT>
__device__ inline void stage_codebooks(uint8_t* lds, const wal_rvq_group& g, int K, const DtypeArgs& D) {
  const int total = S * K;
  for (int e = threadIdx.x; e < total; e += blockDim.x) {
    const int s = e / K;
    const int k = e - s * K;
    const void* cb = nullptr;
#pragma unroll
    for (int ss = 0; ss < S; ++ss)
      if (ss == s) cb = g.codebooks[ss];
    float v[8];
    if (D.cb_dtype == WAL_F32) {
      const u32x4_t* p = reinterpret_cast<const u32x4_t*>(reinterpret_cast<const float*>(cb) + (int64_t)k * 8);
      u32x4_t a = p[0], b = p[1];
#pragma unroll
      for (int j = 0; j < 4; ++j) { v[j] = __uint_as_float(a[j]); v[4 + j] = __uint_as_float(b[j]); }
    } else {
      u32x4_t a = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint16_t*>(cb) + (int64_t)k * 8);
      if (LMODE == LM_H16) {
        // fp16 copy.  Stage 0 is stored as 0 + v (-0 becomes +0), the first
        // add of the reference's zero-initialised fp32 sum, so the fragment
        // code can sum the stages without a leading zero.
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
        continue;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t w = a[j];
        if (D.cb_dtype == WAL_F16) { v[2 * j] = f16_to_f32(w & 0xffffu); v[2 * j + 1] = f16_to_f32(w >> 16); }
        else { v[2 * j] = bf16_to_f32(w & 0xffffu); v[2 * j + 1] = bf16_to_f32(w >> 16); }
      }
    }
    const bool has_ss = g.stage_scales != nullptr;
    const float ss = has_ss ? load_f(g.stage_scales, D.sc_dtype, s) : 1.0f;
    if constexpr (LMODE == LM_F32) {
      // Stage 0 is stored as 0 + v (the reference's zero-initialised sum).
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
    } else if constexpr (LMODE == LM_A16) {
      u32x4_t o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t h[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const float x = v[2 * j + u];
          float c;
          if constexpr (SEM == SEM_FAST) {
            c = round_dt<XDT>(x);
            if (has_ss) c = round_dt<XDT>(c * round_dt<XDT>(ss));
          } else {
            c = 0.0f + (has_ss ? x * ss : x);
          }
          h[u] = to_bits16<XDT>(c);
        }
        o[j] = h[0] | (h[1] << 16);
      }
      *reinterpret_cast<u32x4_t*>(lds + (size_t)e * 16) = o;
    }
  }
}

// Row-scale operand: rf = rne_x(row_scale) as fp32; r2 = that value as a
// packed fp16 pair (used only when x is fp16).
struct RowScale {
  float rf;
  uint32_t r2;
};

template <int XDT>
__device__ inline RowScale make_row_scale(float rs) {
  RowScale r;
  r.rf = round_dt<XDT>(rs);
  if constexpr (XDT == WAL_F16) {
    const uint32_t h = f32_to_f16_rne(rs);
    r.r2 = h | (h << 16);
  } else {
    r.r2 = 0;
  }
  return r;
}

__device__ inline uint32_t pk_mul_f16(uint32_t a, uint32_t b) {
  f16x2_t r = __builtin_bit_cast(f16x2_t, a) * __builtin_bit_cast(f16x2_t, b);
  return __builtin_bit_cast(uint32_t, r);
}
__device__ inline uint32_t pk_add_f16(uint32_t a, uint32_t b) {
  f16x2_t r = __builtin_bit_cast(f16x2_t, a) + __builtin_bit_cast(f16x2_t, b);
  return __builtin_bit_cast(uint32_t, r);
}

// rne_x(a * rf) for a packed pair a of x-dtype values.
template <int XDT>
__device__ inline uint32_t scale_pair(uint32_t a, const RowScale& rs) {
  if constexpr (XDT == WAL_F16) {
    return pk_mul_f16(a, rs.r2);
  } else {
    return pack_bf16(lo_bf16(a) * rs.rf, hi_bf16(a) * rs.rf);
  }
}

template <int XDT>
__device__ inline uint32_t pack_x(float lo, float hi) {
  if constexpr (XDT == WAL_F16) return pack_f16(lo, hi);
  else return pack_bf16(lo, hi);
}

// 8-weight fragment for stage ids id[0..S-1].
template <int S, int LMODE, int SEM, int XDT>
__device__ inline u32x4_t make_wfrag(const uint8_t* lds, const uint32_t (&id)[S], int K, uint32_t active,
                                     const RowScale& rs) {
  u32x4_t w;
  if constexpr (LMODE == LM_F32) {
    u32x4_t c[S][2];
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const u32x4_t* p = reinterpret_cast<const u32x4_t*>(lds + ((size_t)s * K + id[s]) * 32);
      c[s][0] = p[0];
      c[s][1] = p[1];
    }
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
      w[pr] = scale_pair<XDT>(pack_x<XDT>(tl, th), rs);
    }
  } else {
    u32x4_t c[S];
#pragma unroll
    for (int s = 0; s < S; ++s) c[s] = *reinterpret_cast<const u32x4_t*>(lds + ((size_t)s * K + id[s]) * 16);
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
        w[pr] = scale_pair<XDT>(pack_x<XDT>(tl, th), rs);
      }
    } else if constexpr (SEM == SEM_RECON) {  // LM_A16, S == 1
#pragma unroll
      for (int pr = 0; pr < 4; ++pr) w[pr] = scale_pair<XDT>(c[0][pr], rs);
    } else {  // LM_A16, FAST
#pragma unroll
      for (int pr = 0; pr < 4; ++pr) {
        uint32_t a = 0;
        bool first = true;
#pragma unroll
        for (int s = 0; s < S; ++s) {
          if (!(active & (1u << s))) continue;
          if (first) {
            a = c[s][pr];
            first = false;
          } else if constexpr (XDT == WAL_F16) {
            a = pk_add_f16(a, c[s][pr]);
          } else {
            a = pack_bf16(lo_bf16(a) + lo_bf16(c[s][pr]), hi_bf16(a) + hi_bf16(c[s][pr]));
          }
        }
        w[pr] = scale_pair<XDT>(a, rs);
      }
    }
  }
  return w;
}

template <int XDT>
__device__ inline f32x4_t mfma16(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
  if constexpr (XDT == WAL_F16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  }
}

}  // namespace wal
