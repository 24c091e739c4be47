// rvq_kernels.h -- declarations shared by the kernel files and the C API.
#pragma once

#include "rvq_common.h"
#include "rvq_plan.h"

namespace wal {

// Arithmetic a kernel reproduces.
enum Semantics : int {
  SEM_RECON = 0,   // reconstruct_weight, src/runtime.py:379-414
  SEM_FAST = 1,    // reconstruct_weight_fast, src/runtime.py:568-598
  SEM_TRITON = 2,  // _rvq_group_linear_kernel, src/triton_id_matmul.py:186-216
  SEM_ROUTE0 = 3,  // PackedIDRouteLinear.forward, src/runtime.py:89-97
  SEM_ROUTE1 = 4,  // _id_route_linear_kernel, src/triton_id_matmul.py:55-62
  SEM_STAGEWISE = 5  // stagewise_block_matmul, src/runtime.py:878-894
};

struct DtypeArgs {
  int32_t id_dtype;
  int32_t cb_dtype;
  int32_t sc_dtype;  // row_scale / stage_scales / block_scale
  int32_t x_dtype;
};

// Output stage.  bias_mode: 0 none; 1 y = round(acc + bias_x) (bias inside
// F.linear); 2 y = round_x(round_x(acc) + bias_x) (bias added to the rounded
// kernel output, src/runtime.py:103-104).  bias_x = bias rounded to x dtype
// (the reference's `bias.to(x.dtype)`).
struct EpilogueArgs {
  void* y;
  const void* bias;
  int64_t ldy;
  int32_t y_dtype;
  int32_t x_dtype;
  int32_t bias_dtype;
  int32_t bias_mode;
};

WAL_DEVICE float round_rt(float v, int dt) {
  if (dt == WAL_BF16) return round_dt<WAL_BF16>(v);
  if (dt == WAL_F16) return round_dt<WAL_F16>(v);
  return v;
}

WAL_DEVICE void store_output(const EpilogueArgs& E, int64_t m, int64_t n, float acc) {
  float v = acc;
  if (E.bias_mode != 0) {
    const float b = round_rt(load_f(E.bias, E.bias_dtype, n), E.x_dtype);
    if (E.bias_mode == 1) v = v + b;
    else v = round_rt(v, E.x_dtype) + b;
  }
  const int64_t i = m * E.ldy + n;
  if (E.y_dtype == WAL_F32) reinterpret_cast<float*>(E.y)[i] = v;
  else if (E.y_dtype == WAL_BF16) reinterpret_cast<uint16_t*>(E.y)[i] = (uint16_t)f32_to_bf16_rne(v);
  else reinterpret_cast<uint16_t*>(E.y)[i] = (uint16_t)f32_to_f16_rne(v);
}

// Launchers (defined in the .hip files; all return hipGetLastError()).
hipError_t launch_dequant(const LayerArgs& L, const DtypeArgs& D, int sem, void* out, int out_dtype, hipStream_t st);
hipError_t launch_generic_linear(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, int sem,
                                 const void* x, int64_t M, hipStream_t st);

// Codebook form in LDS for the block-size-8 MFMA kernels (rvq_fragment.h);
// capi.hip decides when those kernels apply (mfma_eligible).
enum LdsMode : int { LM_A16 = 0, LM_H16 = 1, LM_F32 = 2 };

// Dense weight of a block-size-8 layer the MFMA kernels accept (RECONSTRUCT or
// FAST, 16-bit output), rvq_dequant8.hip: the codebooks staged in LdsMode
// form, one workgroup per tile of L's tile kind.
hipError_t launch_dequant8(const LayerArgs& L, const DtypeArgs& D, int sem, int lmode, void* out, hipStream_t st);

// Codebook image of every group in LdsMode form (rvq_generic.hip).
hipError_t launch_image(const LayerArgs& L, const DtypeArgs& D, int sem, int lmode, void* dst, hipStream_t st);

// Let kernel `kern` use the whole 160 KB of LDS (hipFuncSetAttribute), once
// per kernel and device; thread-safe (capi.hip).
hipError_t allow_max_lds(const void* kern);

// CUs of the current device, cached per device (capi.hip).
int device_cu_count();

// One-stage decode launches fold the row scale into the staged codebook when
// every 16-row tile has a single scale value (scale runs of a power of two
// >= 16 rows).
inline __host__ __device__ bool decode_scaled_tables(int num_stages, int scale_rows) {
  return num_stages == 1 && scale_rows >= 16 && (scale_rows & (scale_rows - 1)) == 0;
}

template <int XDT, typename IdT>
hipError_t decode_entry(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, int sem, int lmode,
                        const void* x, int M, const DecodePlan& P, hipStream_t st);
// Split-K of the 128 x 256 prefill tile: ksplit slices of the k-steps, fp32
// partials in part ([ksplit][M][out_features], caller memory), summed by
// launch_splitk_reduce.  ksplit == 1 (or part == nullptr): no split.
struct PrefillSplit {
  int ksplit;
  float* part;
};

template <int XDT, typename IdT>
hipError_t prefill_entry(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, int sem, int lmode,
                         const void* x, int64_t M, int shape, const PrefillSplit& sp, hipStream_t st);

// y[m, n] = epilogue(sum over s = 0 .. ksplit-1 of part[s][m][n]), slices in
// ascending order (rvq_generic.hip).
hipError_t launch_splitk_reduce(const float* part, int ksplit, int64_t M, const EpilogueArgs& E, hipStream_t st);

// One explicit instantiation per (activation dtype, index width), each in its
// own translation unit (rvq_decode_<x>_<ids>.hip, rvq_prefill_<x>_<ids>.hip);
// these declarations keep every other unit from instantiating them again.
extern template hipError_t decode_entry<WAL_BF16, uint8_t>(const LayerArgs&, const DtypeArgs&, const EpilogueArgs&,
    int, int, const void*, int, const DecodePlan&, hipStream_t);
extern template hipError_t decode_entry<WAL_BF16, uint16_t>(const LayerArgs&, const DtypeArgs&, const EpilogueArgs&,
    int, int, const void*, int, const DecodePlan&, hipStream_t);
extern template hipError_t decode_entry<WAL_F16, uint8_t>(const LayerArgs&, const DtypeArgs&, const EpilogueArgs&,
    int, int, const void*, int, const DecodePlan&, hipStream_t);
extern template hipError_t decode_entry<WAL_F16, uint16_t>(const LayerArgs&, const DtypeArgs&, const EpilogueArgs&,
    int, int, const void*, int, const DecodePlan&, hipStream_t);
extern template hipError_t prefill_entry<WAL_BF16, uint8_t>(const LayerArgs&, const DtypeArgs&, const EpilogueArgs&,
    int, int, const void*, int64_t, int, const PrefillSplit&, hipStream_t);
extern template hipError_t prefill_entry<WAL_BF16, uint16_t>(const LayerArgs&, const DtypeArgs&, const EpilogueArgs&,
    int, int, const void*, int64_t, int, const PrefillSplit&, hipStream_t);
extern template hipError_t prefill_entry<WAL_F16, uint8_t>(const LayerArgs&, const DtypeArgs&, const EpilogueArgs&,
    int, int, const void*, int64_t, int, const PrefillSplit&, hipStream_t);
extern template hipError_t prefill_entry<WAL_F16, uint16_t>(const LayerArgs&, const DtypeArgs&, const EpilogueArgs&,
    int, int, const void*, int64_t, int, const PrefillSplit&, hipStream_t);

// Nearest codeword of n blocks of d floats (d in {1, 2, 4, 8, 16, 32}),
// rvq_assign.hip.
hipError_t launch_assign(const float* blocks, int64_t n, int d, const float* codebook, int K, int64_t* ids,
                         float* min_dist, hipStream_t st);

// k-means centroid sums and counts (block order), rvq_assign.hip.
hipError_t launch_centroid_sums(const int64_t* ids, int64_t n, const float* blocks, int d, int K, float* sums,
                                int64_t* counts, hipStream_t st);

inline hipError_t launch_decode(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, int sem,
                                int lds_mode, const void* x, int M, const DecodePlan& P, hipStream_t st) {
  if (L.n_tiles == 0) return hipSuccess;
  const bool wide = D.id_dtype != WAL_U8;
  if (D.x_dtype == WAL_BF16)
    return wide ? decode_entry<WAL_BF16, uint16_t>(L, D, E, sem, lds_mode, x, M, P, st)
                : decode_entry<WAL_BF16, uint8_t>(L, D, E, sem, lds_mode, x, M, P, st);
  return wide ? decode_entry<WAL_F16, uint16_t>(L, D, E, sem, lds_mode, x, M, P, st)
              : decode_entry<WAL_F16, uint8_t>(L, D, E, sem, lds_mode, x, M, P, st);
}

// shape: PrefillShape from plan_prefill_shape; sp: split-K of the short tile.
inline hipError_t launch_prefill(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, int sem,
                                 int lds_mode, const void* x, int64_t M, int shape, const PrefillSplit& sp,
                                 hipStream_t st) {
  if (L.n_tiles == 0 || M == 0) return hipSuccess;
  const bool wide = D.id_dtype != WAL_U8;
  if (D.x_dtype == WAL_BF16)
    return wide ? prefill_entry<WAL_BF16, uint16_t>(L, D, E, sem, lds_mode, x, M, shape, sp, st)
                : prefill_entry<WAL_BF16, uint8_t>(L, D, E, sem, lds_mode, x, M, shape, sp, st);
  return wide ? prefill_entry<WAL_F16, uint16_t>(L, D, E, sem, lds_mode, x, M, shape, sp, st)
              : prefill_entry<WAL_F16, uint8_t>(L, D, E, sem, lds_mode, x, M, shape, sp, st);
}

}  // namespace wal
