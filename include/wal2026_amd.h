/*
 * wal2026_amd.h -- C ABI of the MI355X (gfx950) Block-RVQ / route-codebook
 * linear library (libwal2026_amd.so).
 *
 * This is the drop-in boundary for the reference's DRL-runtime compressed
 * linear forward.  The reference is pure Python (PyTorch + Triton); these entry
 * points are what its Python layer binds (through ctypes, or through the
 * torch operator library built beside this one) in place of the torch/Triton
 * calls cited on each declaration.  Paths are relative to the reference
 * repository root.
 *
 * Conventions
 *  - Plain C types only: device pointers are `const void*`, the HIP stream is
 *    passed as `void*` (a hipStream_t; NULL = the null stream).
 *  - Every entry point returns WAL_OK (0) or a negative wal_status.  On error
 *    wal_last_error() returns a message (thread-local).  Argument errors are
 *    found on the host before any launch; launches are checked with
 *    hipGetLastError().
 *  - Nothing here allocates device memory or synchronises the stream.
 *  - Tensors are dense and row-major.  Element types are given by wal_dtype
 *    tags.
 *  - Index values are NOT range-checked on the device: every id must lie in
 *    [0, codebook_size) (the reference's gather would raise on a bad id).
 *    Checking them needs a pass over the index planes, so the library leaves
 *    it to the caller (the Python layer checks once per module).  An id at or
 *    past codebook_size is clamped to codebook_size - 1 by every kernel, so a
 *    bad id gives a wrong but deterministic result, the same at every m;
 *    it never reads outside the codebook.
 */
#ifndef WAL2026_AMD_H
#define WAL2026_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WAL_RVQ_MAX_STAGES 8
#define WAL_ABI_VERSION 4

typedef enum wal_dtype {
  WAL_U8 = 0,   /* index planes, codebook_size <= 256 (src/block_vq.py:160-165) */
  WAL_I16 = 1,  /* index planes, codebook_size <= 32767 */
  WAL_U16 = 2,  /* index planes, codebook_size <= 65536 */
  WAL_I32 = 3,  /* index planes, larger codebooks */
  WAL_F16 = 10,
  WAL_BF16 = 11,
  WAL_F32 = 12
} wal_dtype;

typedef enum wal_status {
  WAL_OK = 0,
  WAL_EINVAL = -1,       /* bad argument (shape, dtype, null pointer) */
  WAL_EUNSUPPORTED = -2, /* valid input this library does not handle */
  WAL_EHIP = -3,         /* HIP runtime error (launch failure etc.) */
  WAL_ESIZE = -4         /* caller buffer too small */
} wal_status;

/* Which of the reference's dequantisation semantics a call reproduces. */
typedef enum wal_rvq_semantics {
  /* PackedBlockRVQGroup.reconstruct_weight (src/runtime.py:379-414): fp32 sum
   * of all stages, round to the output dtype, times row_scale rounded to it.
   * Used by strategies per_group / full_weight / chunked_weight /
   * stacked_matmul (src/runtime.py:1365-1370, :1501-1507). */
  WAL_RVQ_RECONSTRUCT = 0,
  /* PackedBlockRVQGroup.reconstruct_weight_fast (src/runtime.py:568-598):
   * arithmetic in the output dtype over the active stages only.  Used by
   * per_group_fast / full_weight_fast (:1371-1376, :1491-1500). */
  WAL_RVQ_RECONSTRUCT_FAST = 1,
  /* PackedBlockRVQGroup.stagewise_block_matmul (src/runtime.py:878-894),
   * strategy stagewise_einsum (:1466-1475): per stage, codewords cast to the
   * x dtype (times the stage scale cast to it), contracted and rounded to the
   * x dtype, the stage results summed in the x dtype from +0 over all stages,
   * then times row_scale cast to the x dtype; a bias is added to that rounded
   * result.  wal_rvq_linear only (there is no dense weight); groups with a
   * block_scale are refused (src/runtime.py:837-846). */
  WAL_RVQ_STAGEWISE = 2
} wal_rvq_semantics;

/* The buffers of one PackedBlockRVQGroup (src/runtime.py:249-290), device
 * pointers.  The group produces output rows [row0, row0 + rows). */
typedef struct wal_rvq_group {
  const void* stage_ids[WAL_RVQ_MAX_STAGES]; /* [rows, blocks_per_row], id dtype */
  const void* codebooks[WAL_RVQ_MAX_STAGES]; /* [codebook_size, block_size] */
  const void* stage_scales;                  /* [num_stages] or NULL */
  const void* row_scale;                     /* [ceil(rows / scale_rows)] */
  const void* block_scale;                   /* [rows, blocks_per_row] or NULL */
  int32_t row0;
  int32_t rows;
} wal_rvq_group;

/* One PackedGroupedBlockRVQLinear (src/runtime.py:1175-1232): G groups that
 * share the layer-wide constants below. */
typedef struct wal_rvq_layer {
  int32_t in_features;
  int32_t out_features;
  int32_t block_size;       /* d */
  int32_t blocks_per_row;   /* B = padded_cols / d */
  int32_t codebook_size;    /* K */
  int32_t num_stages;       /* S, 1..WAL_RVQ_MAX_STAGES */
  int32_t id_dtype;         /* WAL_U8 / WAL_I16 / WAL_U16 / WAL_I32 */
  int32_t codebook_dtype;   /* WAL_F16 / WAL_BF16 / WAL_F32 */
  int32_t scale_dtype;      /* row_scale, stage_scales and block_scale dtype */
  int32_t scale_rows;       /* rows per row_scale entry; 1 = per row */
  int32_t n_groups;
  int32_t image_tag;        /* WAL_RVQ_IMAGE_TAG the image was built for; 0 = no image */
  const wal_rvq_group* groups;  /* host array [n_groups]; groups[g].row0 ascending, contiguous */
  const void* plan;             /* device copy of the plan (see wal_rvq_plan_build),
                                   required when n_groups > 1, else may be NULL */
  const void* image;            /* device codebook image (wal_rvq_image_build) or NULL */
} wal_rvq_layer;

/* ---- plan: device-side group and tile tables ---------------------------- */

/* Bytes of the plan image for this layer.  No reference counterpart: the
 * reference walks its groups in a Python loop (src/runtime.py:1502-1506);
 * here one launch covers every group and reads them from this table. */
int wal_rvq_plan_size(const wal_rvq_layer* layer, size_t* bytes);

/* Write the plan image into host memory `dst` (`bytes` from
 * wal_rvq_plan_size).  The caller copies it to device memory and stores the
 * device pointer in layer->plan.  The image embeds the group device pointers,
 * so it must be rebuilt if any buffer moves. */
int wal_rvq_plan_build(const wal_rvq_layer* layer, void* dst, size_t bytes);

/* ---- codebook images ------------------------------------------------------ */

/* Tag of an image built for calls with this semantics and activation dtype. */
#define WAL_RVQ_IMAGE_TAG(semantics, x_dtype) (0x1000 | ((semantics) & 0xf) | (((x_dtype) & 0xff) << 4))

/* Bytes of the codebook image of this layer for calls with the given
 * semantics (wal_rvq_semantics) and activation dtype.  No reference
 * counterpart as an entry point: it is the device-side form of the derived
 * codebook caches the reference keeps on its modules (the out_dtype copies of
 * _build_fast_cache, src/runtime.py:431-448; the stage-scale-folded stack of
 * _triton_state, src/runtime.py:855-876). */
int wal_rvq_image_size(const wal_rvq_layer* layer, int semantics, int x_dtype, size_t* bytes);

/* Convert every group's codebooks, once, into the form the fused kernels
 * stage in LDS (per-stage values already rounded as the reference's
 * dequantisation rounds them before the row scale) and write it to device
 * memory dst (16-byte aligned, `bytes` from wal_rvq_image_size).  To use it,
 * store dst in layer->image and WAL_RVQ_IMAGE_TAG(semantics, x_dtype) in
 * layer->image_tag; wal_rvq_linear refuses a call whose semantics or x dtype
 * differ from the tag.  Rebuild it when a codebook or stage scale changes.
 * Finite codebooks and scales (the fused kernels' contract). */
int wal_rvq_image_build(const wal_rvq_layer* layer, int semantics, int x_dtype, void* dst, size_t bytes,
                        void* stream);

/* ---- Block-RVQ entry points --------------------------------------------- */

/* Dense weight [out_features, in_features] in out_dtype (F16/BF16/F32).
 * Replaces PackedGroupedBlockRVQLinear.reconstruct_weight /
 * reconstruct_weight_fast (src/runtime.py:1234-1240), i.e. the per-group
 * PackedBlockRVQGroup.reconstruct_weight (src/runtime.py:379-414) or
 * reconstruct_weight_fast (:568-598) concatenated on rows.  Bit-exact with
 * the reference for every finite result.  active_stage_mask (FAST only): bit
 * s set = stage s active (src/runtime.py:352-377); 0 means all stages. */
int wal_rvq_reconstruct(const wal_rvq_layer* layer, int semantics,
                        uint32_t active_stage_mask, void* w_out, int out_dtype,
                        void* stream);

/* y[m, n] = sum_k x[m, k] * W[n, k] + bias[n], W as wal_rvq_reconstruct would
 * produce it in x_dtype, accumulated in fp32 and rounded once to y_dtype.
 * Replaces PackedGroupedBlockRVQLinear.forward (src/runtime.py:1362-1507) for
 * the dequantise-then-F.linear strategies.  x [m, in_features] F16/BF16, y
 * [m, out_features] F16/BF16/F32, bias [out_features] or NULL (its dtype is
 * bias_dtype; the reference keeps a bf16 buffer, :1229-1230, and casts it to
 * x.dtype, which this call reproduces).  m >= 1; m <= 16 runs the decode
 * kernel, larger m the prefill kernel. */
int wal_rvq_linear(const wal_rvq_layer* layer, int semantics,
                   uint32_t active_stage_mask, const void* x, int64_t m,
                   int x_dtype, const void* bias, int bias_dtype, void* y,
                   int y_dtype, void* stream);

/* wal_rvq_linear with a caller workspace (device memory, 16-byte aligned) of
 * at least wal_rvq_linear_workspace_size bytes (WAL_ESIZE otherwise; NULL
 * with 0 bytes is wal_rvq_linear).  With it, a prefill call whose output
 * tiles alone would leave CUs idle (few weight rows at small m: a 4096-row
 * layer is 16 workgroups at m <= 128) shares each tile's k-steps among
 * several workgroups, which write fp32 partial sums there; a second launch
 * adds them in a fixed order, so the result is deterministic (it may differ
 * from wal_rvq_linear's in the last bits: another fp32 summation order).
 * Same replacement as wal_rvq_linear (src/runtime.py:1362-1507); the
 * workspace has no reference counterpart (torch's F.linear sizes its own). */
int wal_rvq_linear_ws(const wal_rvq_layer* layer, int semantics,
                      uint32_t active_stage_mask, const void* x, int64_t m,
                      int x_dtype, const void* bias, int bias_dtype, void* y,
                      int y_dtype, void* workspace, size_t workspace_bytes,
                      void* stream);

/* wal_rvq_linear_ws for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc):
 * the split-K partials go to a scratch array the library holds in device
 * memory, 64 MiB per GPU (kept until the process ends; its device address is
 * looked up once per device on the first call that needs it).  A call whose
 * partials would exceed 64 MiB (wal_rvq_linear_workspace_size) returns
 * WAL_ESIZE.  Calls that overlap on one GPU share the array and race: issue
 * them on one stream.  No counterpart in the reference: an entry point for
 * callers that cannot allocate. */
int wal_rvq_linear_noalloc(const wal_rvq_layer* layer, int semantics,
                           uint32_t active_stage_mask, const void* x, int64_t m,
                           int x_dtype, const void* bias, int bias_dtype, void* y,
                           int y_dtype, void* stream);

/* Bytes of workspace wal_rvq_linear_ws uses for these arguments (0: no split;
 * x is only checked for alignment).  No reference counterpart. */
int wal_rvq_linear_workspace_size(const wal_rvq_layer* layer, int semantics, const void* x,
                                  int64_t m, int x_dtype, size_t* bytes);

/* The fused Triton kernel's arithmetic: per block the fp32 sum of all stages
 * is cast to x_dtype, contracted in fp32, and the row scale is applied to the
 * accumulator (not per weight).  Replaces rvq_group_linear_matmul
 * (src/triton_id_matmul.py:220-306); unlike it, any block_size and U8/I16/
 * U16/I32 ids are accepted.  stage_ids [S, n, blocks_per_row], codebooks
 * [S, codebook_size, block_size] (F16/BF16, stage scales already folded as
 * in src/runtime.py:867-873), row_scale [n], x [m, k_in], out [m, n]. */
int wal_rvq_group_linear_matmul(const void* x, int64_t m, int64_t k_in, int x_dtype,
                                const void* stage_ids, int id_dtype, int32_t num_stages,
                                int64_t n, int64_t blocks_per_row,
                                const void* codebooks, int cb_dtype, int64_t codebook_size,
                                int32_t block_size, const void* row_scale, int rs_dtype,
                                void* out, int out_dtype, void* stream);

/* ---- scalar route codebook (d = 1) ---------------------------------------- */

/* Route-codebook linear: y = x @ W^T (+ bias), W[n, k] = f(codebook_sum[ids[n, k]],
 * row_scale[n]).  mode 0 reproduces PackedIDRouteLinear.forward
 * (src/runtime.py:89-97: product in the buffers' dtype, then cast to x
 * dtype; bias cast to x dtype before F.linear); mode 1 reproduces
 * FusedIDRouteLinear.forward / id_route_linear_matmul
 * (src/runtime.py:100-105, src/triton_id_matmul.py:55-62: each operand cast to
 * x dtype, product in x dtype; bias added to the rounded output).
 * ids [n, k] I16/U16/I32, codebook_sum [routes] and row_scale [n] F16/BF16
 * (same dtype), bias [n] (bias_dtype) or NULL. */
int wal_id_route_linear(const void* x, int64_t m, int64_t k, int x_dtype,
                        const void* ids, int id_dtype, int64_t n,
                        const void* codebook_sum, int64_t routes, int cs_dtype,
                        const void* row_scale, const void* bias, int bias_dtype,
                        int mode, void* y, int y_dtype, void* stream);

/* Dense route-codebook weight [n, k] in out_dtype.  mode 0 reproduces
 * PackedIDRouteLinear.reconstruct_weight (src/runtime.py:89-93: the product
 * codebook_sum[id] * row_scale in the buffers' dtype), then the cast to
 * out_dtype that forward applies (:97); mode 1 the per-weight value of
 * id_route_linear_matmul (src/triton_id_matmul.py:59-60). */
int wal_id_route_reconstruct(const void* ids, int id_dtype, int64_t n, int64_t k,
                             const void* codebook_sum, int64_t routes, int cs_dtype,
                             const void* row_scale, int mode, int out_dtype, void* w_out,
                             void* stream);

/* ---- encoder ------------------------------------------------------------- */

/* Nearest codeword of every block: replaces _assign_to_codebook
 * (src/block_vq.py:180-196), the assignment step of the reference's k-means
 * encoder (_fit_kmeans :199-227, encode_block_residual_vq).
 * blocks [n, d] and codebook [k_cb, d] fp32 row-major, d in {1, 2, 4, 8, 16,
 * 32}, blocks 16-byte aligned when d % 4 == 0.  Writes ids [n] (int64) and
 * min_dist [n] (fp32) with dist = (|b|^2 + |c|^2) - 2 b.c (:192), the sums and
 * the dot product accumulated with fused multiply-adds in element order, and
 * the first minimal codeword on ties (torch.min, :193).  Finite inputs. */
int wal_rvq_assign(const float* blocks, int64_t n, int d, const float* codebook, int64_t k_cb,
                   int64_t* ids, float* min_dist, void* stream);

/* The reductions of the k-means centroid update in _fit_kmeans
 * (src/block_vq.py:216-218): counts = bincount(ids, minlength=k_cb) and
 * sums = zeros(k_cb, d).index_add_(0, ids, blocks), each sum taken in fp32
 * from +0 in ascending block order (torch's CPU index_add_ order), so the
 * results are deterministic.  ids [n] int64 in [0, k_cb) (ids outside that
 * range are not counted: the caller checks them), blocks [n, d] fp32,
 * d in {1, 2, 4, 8, 16, 32}; writes sums [k_cb, d] fp32 and counts [k_cb]
 * int64 (zeros when n = 0). */
int wal_rvq_centroid_sums(const int64_t* ids, int64_t n, const float* blocks, int d, int64_t k_cb,
                          float* sums, int64_t* counts, void* stream);

/* ---- launch planning (diagnostics) ---------------------------------------- */

/* Kernel families of wal_rvq_linear. */
#define WAL_KERNEL_NONE 0     /* m == 0: nothing to launch */
#define WAL_KERNEL_DECODE 1   /* block-size-8 MFMA decode kernel, m <= 16 */
#define WAL_KERNEL_PREFILL 2  /* block-size-8 MFMA prefill kernel, m > 16 */
#define WAL_KERNEL_GENERIC 3  /* any other layout or semantics */

/* Where the decode kernel's activation fragments come from. */
#define WAL_XMODE_GLOBAL 0  /* global memory (L2), per item */
#define WAL_XMODE_LDS 1     /* x rows staged in LDS, per item */
#define WAL_XMODE_REG 2     /* staged in LDS, held in registers (one chunk per wave) */
#define WAL_XMODE_GREG 3    /* global memory into registers once (one chunk per wave) */
#define WAL_XMODE_GTR 4     /* row runs from global memory, transposed through LDS per item */

/* Prefill tile shapes (x rows x weight rows per workgroup). */
#define WAL_TILE_SHORT 0  /* 128 x 256 */
#define WAL_TILE_TALL 1   /* 256 x 256 */
#define WAL_TILE_WIDE 2   /* 256 x 128 */

typedef struct wal_rvq_launch_info {
  int32_t kernel;       /* WAL_KERNEL_* */
  int32_t x_mode;       /* decode: WAL_XMODE_*; else -1 */
  int32_t table_slots;  /* decode: codebook tables a workgroup keeps in LDS; else -1 */
  int32_t grid;         /* decode and prefill: workgroups (prefill: of a wal_rvq_linear_ws
                           call, the tall tile's last-round halves not counted); else -1 */
  int32_t share;        /* decode: 16-row tiles of the largest workgroup share; prefill:
                           k-steps (32 columns) of the largest workgroup; else -1 */
  int32_t lds_bytes;    /* decode: dynamic LDS per workgroup; else -1 */
  int32_t tile_shape;   /* prefill: WAL_TILE_*; else -1 */
  int32_t k_splits;     /* prefill: k slices per output tile of a wal_rvq_linear_ws call
                           with its workspace (wal_rvq_linear: 1); else -1 */
} wal_rvq_launch_info;

/* What wal_rvq_linear (prefill: wal_rvq_linear_ws with its workspace) would
 * launch for these arguments, without launching anything (no device memory is
 * read; x is only checked for alignment).  The environment overrides
 * WAL2026_DECODE_XMODE (reg, lds, greg, gtr, global), WAL2026_PREFILL_TILE
 * (short, tall, wide) and WAL2026_PREFILL_KSPLIT (1 .. 32 slices of a short
 * tile's k-steps, with a workspace) apply to every call; a forced
 * x-mode that does not apply to the layer makes both return WAL_EUNSUPPORTED.
 * No reference counterpart: the reference's forward has one code path per
 * strategy (src/runtime.py:1362-1507); this reports which of the library's
 * kernel variants serves a call, for tests and tuning. */
int wal_rvq_linear_info(const wal_rvq_layer* layer, int semantics, const void* x, int64_t m, int x_dtype,
                        wal_rvq_launch_info* info);

/* Read-bandwidth probe: reads `bytes` bytes at src (16-byte aligned, a
 * multiple of 16, below 2^31) with the decode kernel's load form -- 16-byte
 * buffer loads with the streaming hint, four in flight per lane, grid-stride
 * over grid workgroups of block threads -- and writes, per wave, the XOR of
 * the 32-bit words it read to partial[wave] (grid * block / 64 entries; their
 * XOR is that of every word in the range).  No reference counterpart: the
 * roofline calibration the bench's read-ceiling mode times against the
 * decode kernel's compressed bytes. */
int wal_read_probe(const void* src, int64_t bytes, uint32_t* partial, int grid, int block, void* stream);

/* ---- misc ---------------------------------------------------------------- */

/* Message for the last error on this thread ("" if none). */
const char* wal_last_error(void);

/* WAL_ABI_VERSION of the loaded library. */
int wal_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* WAL2026_AMD_H */
