/*
 * rvq_oracle.c -- CPU restatement of the reference's Block-RVQ arithmetic.
 * TEST INFRASTRUCTURE ONLY (see rvq_oracle.h).  Built with
 * -ffp-contract=off so that every fp32 multiply and add rounds separately,
 * as the reference's torch ops do.
 */
#include "rvq_oracle.h"

#include <math.h>
#include <string.h>

static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* binary16 -> binary32, exact for every input (subnormals, inf, nan). */
float or_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if (exp == 0x1fu) return bits_f32(sign | 0x7f800000u | (man << 13));
  if (exp == 0) {
    if (man == 0) return bits_f32(sign);
    /* subnormal: man * 2^-24, exactly representable in binary32 */
    float v = (float)man * 0x1p-24f;
    return sign ? -v : v;
  }
  return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

float or_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

/* binary32 -> binary16, round to nearest, ties to even.  Overflow -> inf,
 * NaN -> sign | 0x7e00 (the value torch's scalar c10::Half conversion gives). */
uint16_t or_f32_to_f16(float f) {
  uint32_t u = f32_bits(f);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  /* 65520 = 0x477ff000 is the midpoint between 65504 (odd mantissa) and
   * 2^16: ties-to-even rounds it, and anything larger, to infinity. */
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  int e = (int)(a >> 23) - 127;
  if (e >= -14) {
    uint32_t man = a & 0x7fffffu;
    uint32_t h = ((uint32_t)(e + 15) << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
  }
  if (e < -25) return (uint16_t)sign;       /* below half of the smallest subnormal */
  /* subnormal result, unit 2^-24: value / 2^-24 = sig * 2^(e+1) */
  uint32_t sig = (a & 0x7fffffu) | 0x800000u;
  int s = -(e + 1);                          /* 14 .. 24 */
  uint32_t q = sig >> s;
  uint32_t rem = sig & ((1u << s) - 1u);
  uint32_t half = 1u << (s - 1);
  if (rem > half || (rem == half && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}

/* binary32 -> bfloat16, round to nearest, ties to even; NaN -> 0x7fc0 (the
 * value torch's scalar c10::BFloat16 conversion gives). */
uint16_t or_f32_to_bf16(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  uint32_t bias = 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)((u + bias) >> 16);
}

float or_load_f32(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case OR_F16: return or_f16_to_f32(((const uint16_t*)p)[i]);
    case OR_BF16: return or_bf16_to_f32(((const uint16_t*)p)[i]);
    default: return ((const float*)p)[i];
  }
}

float or_round(float v, int dtype) {
  switch (dtype) {
    case OR_F16: return or_f16_to_f32(or_f32_to_f16(v));
    case OR_BF16: return or_bf16_to_f32(or_f32_to_bf16(v));
    default: return v;
  }
}

static void store_out(void* out, int dtype, int64_t i, float v) {
  switch (dtype) {
    case OR_F16: ((uint16_t*)out)[i] = or_f32_to_f16(v); break;
    case OR_BF16: ((uint16_t*)out)[i] = or_f32_to_bf16(v); break;
    default: ((float*)out)[i] = v; break;
  }
}

static int64_t load_id(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case OR_U8: return ((const uint8_t*)p)[i];
    case OR_I16: return ((const int16_t*)p)[i];
    case OR_U16: return ((const uint16_t*)p)[i];
    default: return ((const int32_t*)p)[i];
  }
}

static int check_group(const or_group* g) {
  if (g->num_stages < 1 || g->num_stages > OR_MAX_STAGES) return -1;
  if (g->block_size < 1 || g->blocks_per_row * g->block_size < g->in_features) return -1;
  if (g->scale_rows < 1) return -1;
  return 0;
}

/* Restates src/runtime.py:379-414 for groups with no residual correction and
 * no transform (the fields those steps read are None):
 *   recon = zeros fp32                                  :382
 *   for s: stage = codebook_s[ids_s].float()            :384-385
 *          stage = stage * stage_scales[s].float()      :386-387 (if present)
 *          recon += stage                               :388
 *   recon = recon * block_scale.float()                 :398-399 (if present)
 *   W = recon[:, :in].to(dt) * row_scale.to(dt)         :413-414
 * Out-of-range ids make the function return -2 (torch raises IndexError). */
int or_reconstruct_weight(const or_group* g, int out_dtype, void* out) {
  if (check_group(g)) return -1;
  const int64_t B = g->blocks_per_row, d = g->block_size, in = g->in_features;
  for (int64_t r = 0; r < g->rows; ++r) {
    const float rs = or_load_f32(g->row_scale, g->rs_dtype, r / g->scale_rows);
    const float rs_dt = or_round(rs, out_dtype);
    for (int64_t b = 0; b < B; ++b) {
      int64_t ids[OR_MAX_STAGES];
      for (int s = 0; s < g->num_stages; ++s) {
        ids[s] = load_id(g->stage_ids[s], g->id_dtype, r * B + b);
        if (ids[s] < 0 || ids[s] >= g->codebook_size) return -2;
      }
      const float bs = g->block_scale ? or_load_f32(g->block_scale, g->bs_dtype, r * B + b) : 1.0f;
      for (int64_t j = 0; j < d; ++j) {
        const int64_t col = b * d + j;
        if (col >= in) break;
        float acc = 0.0f;
        for (int s = 0; s < g->num_stages; ++s) {
          float v = or_load_f32(g->codebooks[s], g->cb_dtype, ids[s] * d + j);
          if (g->stage_scales) v = v * or_load_f32(g->stage_scales, g->ss_dtype, s);
          acc = acc + v;
        }
        if (g->block_scale) acc = acc * bs;
        float w;
        if (out_dtype == OR_F32) {
          w = acc * rs;
        } else {
          w = or_round(or_round(acc, out_dtype) * rs_dt, out_dtype);
        }
        store_out(out, out_dtype, r * in + col, w);
      }
    }
  }
  return 0;
}

/* Restates src/runtime.py:568-598 (plain groups, :416-429) with the cache of
 * :431-448:
 *   cb_dt[s] = codebook_s.to(dt) [* stage_scales[s].to(dt)]   :441-444
 *   recon = cb_dt[first][ids_first]                            :590-591
 *   for idx in active[1:]: recon.add_(cb_dt[idx][ids_idx])     :592-594
 *   W = recon[:, :in].mul_(row_scale.to(dt))                   :595-597
 * Every op rounds to dt.  A group with block_scale is not "plain"; the
 * reference then calls reconstruct_weight with all stages (:579-580). */
int or_reconstruct_weight_fast(const or_group* g, uint32_t active_mask,
                               int out_dtype, void* out) {
  if (check_group(g)) return -1;
  if (g->block_scale) return or_reconstruct_weight(g, out_dtype, out);
  if ((active_mask & ((1u << g->num_stages) - 1u)) == 0) active_mask = 1u;
  const int64_t B = g->blocks_per_row, d = g->block_size, in = g->in_features;
  for (int64_t r = 0; r < g->rows; ++r) {
    const float rs_dt = or_round(or_load_f32(g->row_scale, g->rs_dtype, r / g->scale_rows), out_dtype);
    for (int64_t b = 0; b < B; ++b) {
      for (int64_t j = 0; j < d; ++j) {
        const int64_t col = b * d + j;
        if (col >= in) break;
        int first = 1;
        float recon = 0.0f;
        for (int s = 0; s < g->num_stages; ++s) {
          if (!(active_mask & (1u << s))) continue;
          const int64_t id = load_id(g->stage_ids[s], g->id_dtype, r * B + b);
          if (id < 0 || id >= g->codebook_size) return -2;
          float c = or_round(or_load_f32(g->codebooks[s], g->cb_dtype, id * d + j), out_dtype);
          if (g->stage_scales) {
            const float ss = or_round(or_load_f32(g->stage_scales, g->ss_dtype, s), out_dtype);
            c = or_round(c * ss, out_dtype);
          }
          recon = first ? c : or_round(recon + c, out_dtype);
          first = 0;
        }
        store_out(out, out_dtype, r * in + col, or_round(recon * rs_dt, out_dtype));
      }
    }
  }
  return 0;
}

int or_stagewise_linear(const or_group* g, const void* x, int x_dtype, int64_t m, void* y) {
  if (check_group(g)) return -1;
  if (g->block_scale) return -3;
  const int64_t B = g->blocks_per_row, d = g->block_size, in = g->in_features;
  for (int64_t i = 0; i < m; ++i) {
    for (int64_t r = 0; r < g->rows; ++r) {
      float out = 0.0f;
      for (int s = 0; s < g->num_stages; ++s) {
        const float ss = g->stage_scales ? or_round(or_load_f32(g->stage_scales, g->ss_dtype, s), x_dtype) : 1.0f;
        double acc = 0.0;
        for (int64_t b = 0; b < B; ++b) {
          const int64_t id = load_id(g->stage_ids[s], g->id_dtype, r * B + b);
          if (id < 0 || id >= g->codebook_size) return -2;
          for (int64_t j = 0; j < d; ++j) {
            const int64_t col = b * d + j;
            if (col >= in) break;  /* zero padding of x (:883-885) */
            float w = or_round(or_load_f32(g->codebooks[s], g->cb_dtype, id * d + j), x_dtype);
            if (g->stage_scales) w = or_round(w * ss, x_dtype);
            acc += (double)or_load_f32(x, x_dtype, i * in + col) * (double)w;
          }
        }
        out = or_round(out + or_round((float)acc, x_dtype), x_dtype);
      }
      const float rs = or_round(or_load_f32(g->row_scale, g->rs_dtype, r / g->scale_rows), x_dtype);
      store_out(y, x_dtype, i * g->rows + r, or_round(out * rs, x_dtype));
    }
  }
  return 0;
}

void or_linear_f64(const void* x, int x_dtype, int64_t m, int64_t k,
                   const void* w, int w_dtype, int64_t n_rows,
                   const void* bias, int bias_dtype, double* y) {
  for (int64_t i = 0; i < m; ++i) {
    for (int64_t n = 0; n < n_rows; ++n) {
      double acc = 0.0;
      for (int64_t c = 0; c < k; ++c)
        acc += (double)or_load_f32(x, x_dtype, i * k + c) * (double)or_load_f32(w, w_dtype, n * k + c);
      if (bias) acc += (double)or_load_f32(bias, bias_dtype, n);
      y[i * n_rows + n] = acc;
    }
  }
}

/* src/triton_id_matmul.py:186-216: weight_block = sum_s float(cb[s, id]) from
 * 0 (:195-207), cast to x.dtype (:208), acc += x @ w^T in fp32 (restated in
 * double here), out = acc * float(rho) (:210) stored in x.dtype. */
void or_triton_rvq_matmul(const void* x, int x_dtype, int64_t m, int64_t in_features,
                          const void* ids, int id_dtype, int32_t num_stages,
                          int64_t n_rows, int64_t blocks_per_row,
                          const void* codebooks, int cb_dtype, int64_t codebook_size,
                          int32_t block_size, const void* row_scale, int rs_dtype,
                          int out_dtype, void* out) {
  const int64_t d = block_size;
  for (int64_t n = 0; n < n_rows; ++n) {
    const float rho = or_load_f32(row_scale, rs_dtype, n);
    for (int64_t i = 0; i < m; ++i) {
      double acc = 0.0;
      for (int64_t b = 0; b < blocks_per_row; ++b) {
        for (int64_t j = 0; j < d; ++j) {
          const int64_t col = b * d + j;
          if (col >= in_features) break;
          float wsum = 0.0f;
          for (int s = 0; s < num_stages; ++s) {
            const int64_t id = load_id(ids, id_dtype, ((int64_t)s * n_rows + n) * blocks_per_row + b);
            wsum = wsum + or_load_f32(codebooks, cb_dtype, ((int64_t)s * codebook_size + id) * d + j);
          }
          acc += (double)or_load_f32(x, x_dtype, i * in_features + col) * (double)or_round(wsum, x_dtype);
        }
      }
      store_out(out, out_dtype, i * n_rows + n, (float)acc * rho);
    }
  }
}

void or_id_route_weight(const void* ids, int id_dtype, int64_t n_rows, int64_t k,
                        const void* codebook_sum, int cs_dtype,
                        const void* row_scale, int rs_dtype,
                        int mode, int x_dtype, uint16_t* w_out) {
  for (int64_t n = 0; n < n_rows; ++n) {
    const float rs = or_load_f32(row_scale, rs_dtype, n);
    for (int64_t c = 0; c < k; ++c) {
      const int64_t id = load_id(ids, id_dtype, n * k + c);
      const float cs = or_load_f32(codebook_sum, cs_dtype, id);
      float w;
      if (mode == 0) {
        /* product in the buffers' dtype (fp16 as registered, :65-67), then
         * .to(x.dtype) in forward (:97) */
        w = or_round(or_round(cs * rs, cs_dtype), x_dtype);
      } else {
        w = or_round(or_round(cs, x_dtype) * or_round(rs, x_dtype), x_dtype);
      }
      w_out[n * k + c] = (x_dtype == OR_F16) ? or_f32_to_f16(w) : or_f32_to_bf16(w);
    }
  }
}

/* _assign_to_codebook, src/block_vq.py:180-196 (see rvq_oracle.h). */
static float or_sq_norm(const float* v, int d) {
  float s = v[0] * v[0];
  for (int j = 1; j < d; ++j) s = fmaf(v[j], v[j], s);
  return s;
}

void or_assign(const float* blocks, int64_t n, int d, const float* codebook, int64_t k_cb,
               int64_t* ids, float* min_dist) {
  for (int64_t i = 0; i < n; ++i) {
    const float* b = blocks + i * d;
    const float bsq = or_sq_norm(b, d);
    int64_t best = 0;
    float best_d = INFINITY;
    for (int64_t k = 0; k < k_cb; ++k) {
      const float* c = codebook + k * d;
      float dot = b[0] * c[0];
      for (int j = 1; j < d; ++j) dot = fmaf(b[j], c[j], dot);
      const float dist = (bsq + or_sq_norm(c, d)) - 2.0f * dot;
      if (dist < best_d) {
        best = k;
        best_d = dist;
      }
    }
    ids[i] = best;
    min_dist[i] = best_d;
  }
}

/* _fit_kmeans centroid reductions, src/block_vq.py:216-218 (see rvq_oracle.h). */
int or_centroid_sums(const int64_t* ids, int64_t n, const float* blocks, int d, int64_t k_cb,
                     float* sums, int64_t* counts) {
  for (int64_t i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= k_cb) return -1;
  for (int64_t k = 0; k < k_cb; ++k) {
    counts[k] = 0;
    for (int j = 0; j < d; ++j) sums[k * d + j] = 0.0f;
  }
  for (int64_t i = 0; i < n; ++i) {
    const int64_t k = ids[i];
    counts[k] += 1;
    for (int j = 0; j < d; ++j) sums[k * d + j] = sums[k * d + j] + blocks[i * d + j];
  }
  return 0;
}
