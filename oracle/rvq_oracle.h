/*
 * rvq_oracle.h -- CPU restatement of the reference's Block-RVQ / route-codebook
 * arithmetic.  TEST INFRASTRUCTURE ONLY: this code is the checker that the HIP
 * library is compared against.  It is never linked into, loaded by, or called
 * from the product path (wal2026_amd/), which fails loudly without its HIP
 * library instead of falling back here.
 *
 * Every function cites the reference file:line whose arithmetic it restates
 * (paths relative to the reference repository root).
 *
 * How each function is pinned (tests/test_oracle.py, tests/test_assign_oracle.py):
 *   conversions          every fp16 pattern; random and special fp32 patterns
 *                        against numpy and torch casts
 *   reconstruct_weight   hand-derived golden bits (tests/golden), closed forms
 *                        (one constant stage, a zero stage, all-zero ids), a
 *                        float64 bound, the one-hot readout, torch's op sequence
 *   reconstruct_fast     torch's op sequence, active-stage fixtures
 *   linear_f64           numpy float64, linearity, the one-hot readout
 *   triton_rvq_matmul    float64 closed form; power-of-two row scales exact; a
 *                        planted per-weight scale and a dropped scale caught
 *   stagewise_linear     torch's op sequence; one-stage closed form
 *   id_route_weight      hand-derived golden bits (double-rounding ties, an fp16
 *                        overflow, a subnormal tie); torch's op sequence
 *   assign               float64 brute force, exact ties, a planted sign error
 *   centroid_sums        bincount / index_add_ bit for bit; float64 sums
 *
 * Numbers are passed as raw bit patterns: 16-bit floats as uint16_t, with a
 * dtype tag (OR_F16 / OR_BF16 / OR_F32) saying how to read them.
 */
#ifndef WAL_RVQ_ORACLE_H
#define WAL_RVQ_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  OR_U8 = 0, OR_I16 = 1, OR_U16 = 2, OR_I32 = 3,
  OR_F16 = 10, OR_BF16 = 11, OR_F32 = 12
};

#define OR_MAX_STAGES 8

/* One PackedBlockRVQGroup's buffers (src/runtime.py:249-290), host memory. */
typedef struct or_group {
  int32_t rows;            /* stage_ids_i.shape[0] */
  int32_t in_features;     /* original_shape[1] */
  int32_t block_size;      /* d */
  int32_t blocks_per_row;  /* padded_cols / d */
  int32_t codebook_size;   /* K */
  int32_t num_stages;      /* S */
  int32_t id_dtype;        /* OR_U8 / OR_I16 / OR_U16 / OR_I32 */
  int32_t cb_dtype;        /* OR_F16 / OR_BF16 / OR_F32 (all codebooks) */
  int32_t rs_dtype;        /* row_scale dtype */
  int32_t ss_dtype;        /* stage_scales dtype (if present) */
  int32_t bs_dtype;        /* block_scale dtype (if present) */
  int32_t scale_rows;      /* rows sharing one row_scale entry (1 = per row) */
  const void* stage_ids[OR_MAX_STAGES];  /* [rows, blocks_per_row] */
  const void* codebooks[OR_MAX_STAGES];  /* [codebook_size, block_size] */
  const void* stage_scales;              /* [num_stages] or NULL */
  const void* row_scale;                 /* [ceil(rows/scale_rows)] */
  const void* block_scale;               /* [rows, blocks_per_row] or NULL */
} or_group;

/* Scalar conversions (IEEE-754 binary16 / bfloat16, round-to-nearest-even). */
float    or_f16_to_f32(uint16_t h);
float    or_bf16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
uint16_t or_f32_to_bf16(float f);
/* Read element i of a float buffer tagged with dtype as an fp32 value. */
float    or_load_f32(const void* p, int dtype, int64_t i);
/* Round fp32 to dtype and return the rounded value as fp32. */
float    or_round(float v, int dtype);

/* reconstruct_weight: src/runtime.py:379-414 (== src/block_vq.py:259-289). */
int or_reconstruct_weight(const or_group* g, int out_dtype, void* out);

/* reconstruct_weight_fast: src/runtime.py:568-598 with the cache of :431-448.
 * active_mask bit s set <=> stage s is in _compute_active_stage_indices()
 * (src/runtime.py:352-377); stages are visited in increasing index order. */
int or_reconstruct_weight_fast(const or_group* g, uint32_t active_mask,
                               int out_dtype, void* out);

/* y[m, n] = sum_k x[m, k] * W[n, k] (+ bias[n]) in double, the contraction of
 * F.linear (src/runtime.py:1501-1507).  W is [n_rows, k] tagged w_dtype, x is
 * [m, k] tagged x_dtype, bias may be NULL. */
void or_linear_f64(const void* x, int x_dtype, int64_t m, int64_t k,
                   const void* w, int w_dtype, int64_t n_rows,
                   const void* bias, int bias_dtype, double* y);

/* rvq_group_linear_matmul semantics (src/triton_id_matmul.py:143-217): per
 * block the fp32 sum of all stages is cast to x_dtype, contracted in double
 * (the kernel accumulates in fp32), then acc * float(row_scale) is rounded to
 * out_dtype.  ids [S, N, B], codebooks [S, K, d] fp16/bf16, row_scale [N]. */
void or_triton_rvq_matmul(const void* x, int x_dtype, int64_t m, int64_t in_features,
                          const void* ids, int id_dtype, int32_t num_stages,
                          int64_t n_rows, int64_t blocks_per_row,
                          const void* codebooks, int cb_dtype, int64_t codebook_size,
                          int32_t block_size, const void* row_scale, int rs_dtype,
                          int out_dtype, void* out);

/* stagewise_block_matmul (src/runtime.py:878-894), one group:
 *   out = 0 (x dtype)                                                 :886
 *   for every stage s: W_s = x_dtype(cb_s[id]) [* x_dtype(ss[s])]     :889-891
 *                      out = x_dtype(out + x_dtype(x . W_s^T))         :892
 *   y = x_dtype(out * x_dtype(row_scale))                              :894
 * The per-stage dot is taken in double and rounded once to x dtype (torch's
 * einsum accumulates in fp32 in an unspecified order).  x [m, in_features],
 * y [m, rows] in x dtype bits.  Groups with block_scale are refused (-3). */
int or_stagewise_linear(const or_group* g, const void* x, int x_dtype, int64_t m, void* y);

/* Scalar route codebook, d = 1.
 * mode 0 = PackedIDRouteLinear.forward (src/runtime.py:89-97):
 *   W16 = f16(codebook_sum[id] * row_scale) then W16.to(x_dtype).
 * mode 1 = FusedIDRouteLinear / id_route_linear_matmul (src/triton_id_matmul.py:55-62):
 *   w = x_dtype(lut[id]) * x_dtype(rho), product rounded to x_dtype.
 * Writes the dense weight [n_rows, k] in x_dtype bits (uint16). */
void or_id_route_weight(const void* ids, int id_dtype, int64_t n_rows, int64_t k,
                        const void* codebook_sum, int cs_dtype,
                        const void* row_scale, int rs_dtype,
                        int mode, int x_dtype, uint16_t* w_out);

/* _assign_to_codebook (src/block_vq.py:180-196): nearest codeword of every
 * block, fp32 throughout.
 *   code_sq[k] = sum_j c[k][j]^2, chunk_sq[i] = sum_j b[i][j]^2 and
 *   dot[i][k] = sum_j b[i][j] * c[k][j]: first product, then fused
 *   multiply-adds for j = 1..d-1 in order (as BLAS sgemm kernels accumulate);
 *   dist[i][k] = (chunk_sq[i] + code_sq[k]) - 2 * dot[i][k]   (:192);
 *   ids[i] = the first k of minimal dist[i][k] (strict <, from +inf:
 *   torch.min's tie rule, :193), min_dist[i] = that distance.
 * The reference leaves the order of its two sums and of the matmul to torch
 * (oneDNN/BLAS); the order above is this build's canonical one, and the HIP
 * kernel follows it exactly.  Finite inputs only. */
void or_assign(const float* blocks, int64_t n, int d, const float* codebook, int64_t k_cb,
               int64_t* ids, float* min_dist);

/* The centroid update's reductions in _fit_kmeans (src/block_vq.py:216-218):
 *   counts = bincount(ids, minlength=k_cb);
 *   sums = zeros(k_cb, d).index_add_(0, ids, blocks)
 * with torch's CPU order: for i = 0..n-1 ascending, sums[ids[i]][j] += blocks[i][j]
 * in fp32 from +0.  ids must lie in [0, k_cb) (returns -1 otherwise, like
 * index_add_ raising). */
int or_centroid_sums(const int64_t* ids, int64_t n, const float* blocks, int d, int64_t k_cb,
                     float* sums, int64_t* counts);

#ifdef __cplusplus
}
#endif
#endif
