// rvq_generic.hip -- element-exact kernels for every layout the library accepts.
//
//  * rvq_dequant_kernel: the dense weight (PackedBlockRVQGroup.reconstruct_weight
//    / reconstruct_weight_fast, src/runtime.py:379-414 / :568-598), one thread
//    per (row, block) slot, writes d contiguous elements.  HBM-write bound.
//  * rvq_generic_linear_kernel: LDS-tiled fp32 VALU contraction with the weight
//    tile dequantised element by element.  Handles what the MFMA kernels do not
//    (any block size, 32-bit ids, fp32 codebooks, block_scale, unaligned rows)
//    and the Triton / route-codebook / stagewise semantics.
#include "rvq_fragment.h"

namespace wal {

// Index clamped into [0, K): ids are validated by the host when a plan is
// built; the clamp keeps a corrupt index from ever becoming a load outside the
// codebook.
WAL_DEVICE int64_t clamp_id(int64_t id, int K) { return id < 0 ? 0 : (id >= K ? K - 1 : id); }

// One weight element W[r, col] of a group (r = row inside the group) as fp32
// holding a value exact in DT.  rs is row_scale[r] as fp32 (exact).
template <int SEM, int DT>
WAL_DEVICE float weight_elem(const LayerArgs& L, const wal_rvq_group& g, const DtypeArgs& D,
                                    int64_t r, int col, float rs) {
  if constexpr (SEM == SEM_ROUTE0 || SEM == SEM_ROUTE1) {
    // ids [rows, in_features] (d = 1, one stage), codebook_sum in codebooks[0].
    const int64_t id = clamp_id(load_id(g.stage_ids[0], D.id_dtype, r * (int64_t)L.in_features + col), L.codebook_size);
    const float cs = load_f(g.codebooks[0], D.cb_dtype, id);
    if constexpr (SEM == SEM_ROUTE0) {
      // src/runtime.py:91-97: product in the buffers' dtype, then .to(x dtype)
      const float p = (D.cb_dtype == WAL_BF16) ? round_dt<WAL_BF16>(cs * rs) : round_dt<WAL_F16>(cs * rs);
      return round_dt<DT>(p);
    } else {
      // src/triton_id_matmul.py:59-60: each operand cast to x dtype, product in x dtype
      return round_dt<DT>(round_dt<DT>(cs) * round_dt<DT>(rs));
    }
  } else {
    const int d = L.block_size;
    const int b = col / d;
    const int j = col - b * d;
    const int64_t slot = r * (int64_t)L.blocks_per_row + b;
    if constexpr (SEM == SEM_RECON || SEM == SEM_TRITON) {
      float t = 0.0f;
#pragma unroll
      for (int s = 0; s < WAL_RVQ_MAX_STAGES; ++s) {
        if (s >= L.num_stages) break;
        const int64_t id = clamp_id(load_id(g.stage_ids[s], D.id_dtype, slot), L.codebook_size);
        float v = load_f(g.codebooks[s], D.cb_dtype, id * d + j);
        if (SEM == SEM_RECON && g.stage_scales) v = v * load_f(g.stage_scales, D.sc_dtype, s);
        t = t + v;
      }
      if constexpr (SEM == SEM_TRITON) {
        return round_dt<DT>(t);  // src/triton_id_matmul.py:208, scale applied after the dot
      } else {
        if (g.block_scale) t = t * load_f(g.block_scale, D.sc_dtype, slot);
        if constexpr (DT == WAL_F32) return t * rs;
        return round_dt<DT>(round_dt<DT>(t) * round_dt<DT>(rs));
      }
    } else {  // SEM_FAST
      float a = 0.0f;
      bool first = true;
#pragma unroll
      for (int s = 0; s < WAL_RVQ_MAX_STAGES; ++s) {
        if (s >= L.num_stages) break;
        if (!(L.active_mask & (1u << s))) continue;
        const int64_t id = clamp_id(load_id(g.stage_ids[s], D.id_dtype, slot), L.codebook_size);
        float c = round_dt<DT>(load_f(g.codebooks[s], D.cb_dtype, id * d + j));
        if (g.stage_scales) c = round_dt<DT>(c * round_dt<DT>(load_f(g.stage_scales, D.sc_dtype, s)));
        a = first ? c : round_dt<DT>(a + c);
        first = false;
      }
      return round_dt<DT>(a * round_dt<DT>(rs));
    }
  }
}

// Stage s's contribution to W[r, col] under stagewise_block_matmul
// (src/runtime.py:889-892): the codeword cast to x dtype, times the stage
// scale cast to x dtype (product in x dtype).  No row scale: it is applied to
// the contracted output.
template <int DT>
WAL_DEVICE float stage_elem(const LayerArgs& L, const wal_rvq_group& g, const DtypeArgs& D, int64_t r, int col,
                            int s) {
  const int d = L.block_size;
  const int b = col / d;
  const int j = col - b * d;
  const int64_t slot = r * (int64_t)L.blocks_per_row + b;
  const int64_t id = clamp_id(load_id(g.stage_ids[s], D.id_dtype, slot), L.codebook_size);
  float c = round_dt<DT>(load_f(g.codebooks[s], D.cb_dtype, id * d + j));
  if (g.stage_scales) c = round_dt<DT>(c * round_dt<DT>(load_f(g.stage_scales, D.sc_dtype, s)));
  return c;
}

template <int DT>
WAL_DEVICE void store_elem(void* out, int64_t i, float v) {
  if constexpr (DT == WAL_F32) reinterpret_cast<float*>(out)[i] = v;
  else reinterpret_cast<uint16_t*>(out)[i] = (uint16_t)to_bits16<DT>(v);
}

// ---------------------------------------------------------------------------
// Dense dequantisation.  Grid: one workgroup per 16-row tile.
// ---------------------------------------------------------------------------
template <int SEM, int DT>
__global__ __launch_bounds__(256) void rvq_dequant_kernel(LayerArgs L, DtypeArgs D, void* __restrict__ out) {
  const TileInfo ti = get_tile(L, blockIdx.x);
  const wal_rvq_group& g = ti.g;
  const int B = L.blocks_per_row;
  const int d = L.block_size;
  const int64_t slots = (int64_t)ti.rows * B;
  for (int64_t slot = threadIdx.x; slot < slots; slot += blockDim.x) {
    const int rr = (int)(slot / B);
    const int b = (int)(slot - (int64_t)rr * B);
    const int64_t r = ti.row0 + rr;
    const float rs = load_f(g.row_scale, D.sc_dtype, scale_index(L, r));
    const int64_t orow = ti.out_row0 + rr;
    for (int j = 0; j < d; ++j) {
      const int col = b * d + j;
      if (col >= L.in_features) break;
      store_elem<DT>(out, orow * L.in_features + col, weight_elem<SEM, DT>(L, g, D, r, col, rs));
    }
  }
}

// ---------------------------------------------------------------------------
// Generic tiled contraction: y[m, n] = sum_k x[m, k] W[n, k].
// Workgroup: 256 threads, tile 64 weight rows x 32 x rows, k-step 32.
// Grid: (tiles of 64 rows, ceil(M / 32)).
// ---------------------------------------------------------------------------
constexpr int GN = 64, GM = 32, GK = 32;

template <int SEM, int DT>
__global__ __launch_bounds__(256) void rvq_generic_linear_kernel(LayerArgs L, DtypeArgs D, EpilogueArgs E,
                                                                 const void* __restrict__ x, int64_t M) {
  __shared__ float ws[GN][GK + 1];
  __shared__ float xs[GM][GK + 1];
  const TileInfo ti = get_tile(L, blockIdx.x);
  const wal_rvq_group& g = ti.g;
  const int64_t m0 = (int64_t)blockIdx.y * GM;
  const int tid = threadIdx.x;
  const int tn = tid & 63;      // weight row within the tile
  const int tm = tid >> 6;      // 0..3 -> x rows tm*8 .. tm*8+7
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  constexpr int XDT = (DT == WAL_F32) ? WAL_F32 : DT;
  // SEM_STAGEWISE makes one pass per stage: out = round_x(out + round_x(x . W_s))
  // from out = +0 (src/runtime.py:886-893); every other semantics one pass.
  const int n_pass = SEM == SEM_STAGEWISE ? L.num_stages : 1;
  float out_sw[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) out_sw[i] = 0.0f;

  for (int pass = 0; pass < n_pass; ++pass) {
  if (SEM == SEM_STAGEWISE) {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  }
  for (int k0 = 0; k0 < L.in_features; k0 += GK) {
    // weight tile: 64 x 32 elements, 8 per thread
    for (int e = tid; e < GN * GK; e += 256) {
      const int rr = e / GK, kk = e - rr * GK;
      const int col = k0 + kk;
      float w = 0.0f;
      if (rr < ti.rows && col < L.in_features) {
        const int64_t r = ti.row0 + rr;
        if constexpr (SEM == SEM_STAGEWISE) {
          w = stage_elem<DT>(L, g, D, r, col, pass);
        } else {
          float rs = 1.0f;
          if (SEM != SEM_TRITON) {
            const int64_t rsi = (SEM == SEM_ROUTE0 || SEM == SEM_ROUTE1) ? r : scale_index(L, r);
            rs = load_f(g.row_scale, D.sc_dtype, rsi);
          }
          w = weight_elem<SEM, DT>(L, g, D, r, col, rs);
        }
      }
      ws[rr][kk] = w;
    }
    for (int e = tid; e < GM * GK; e += 256) {
      const int mm = e / GK, kk = e - mm * GK;
      const int64_t m = m0 + mm;
      const int col = k0 + kk;
      xs[mm][kk] = (m < M && col < L.in_features) ? load_f(x, D.x_dtype, m * L.in_features + col) : 0.0f;
    }
    __syncthreads();
#pragma unroll 4
    for (int kk = 0; kk < GK; ++kk) {
      const float w = ws[tn][kk];
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] = __builtin_fmaf(xs[tm * 8 + i][kk], w, acc[i]);
    }
    __syncthreads();
  }
  if (SEM == SEM_STAGEWISE) {
#pragma unroll
    for (int i = 0; i < 8; ++i) out_sw[i] = round_dt<DT>(out_sw[i] + round_dt<DT>(acc[i]));
  }
  }  // pass
  (void)XDT;
  if (tn >= ti.rows) return;
  const int64_t n = ti.out_row0 + tn;
  float rho = 1.0f;
  if (SEM == SEM_TRITON) rho = load_f(g.row_scale, D.sc_dtype, ti.row0 + tn);
  // stagewise: out * row_scale.to(out.dtype), product in x dtype (src/runtime.py:894)
  if (SEM == SEM_STAGEWISE) rho = round_dt<DT>(load_f(g.row_scale, D.sc_dtype, scale_index(L, ti.row0 + tn)));
  for (int i = 0; i < 8; ++i) {
    const int64_t m = m0 + tm * 8 + i;
    if (m >= M) break;
    float v = acc[i];
    if (SEM == SEM_TRITON) v = v * rho;  // src/triton_id_matmul.py:210
    if (SEM == SEM_STAGEWISE) v = round_dt<DT>(out_sw[i] * rho);
    store_output(E, m, n, v);
  }
}

// ---------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------
template <int SEM>
static hipError_t dequant_dt(const LayerArgs& L, const DtypeArgs& D, void* out, int out_dtype, int n_tiles, hipStream_t st) {
  dim3 grid(n_tiles), block(256);
  switch (out_dtype) {
    case WAL_BF16: hipLaunchKernelGGL((rvq_dequant_kernel<SEM, WAL_BF16>), grid, block, 0, st, L, D, out); break;
    case WAL_F16: hipLaunchKernelGGL((rvq_dequant_kernel<SEM, WAL_F16>), grid, block, 0, st, L, D, out); break;
    default: hipLaunchKernelGGL((rvq_dequant_kernel<SEM, WAL_F32>), grid, block, 0, st, L, D, out); break;
  }
  return hipGetLastError();
}

hipError_t launch_dequant(const LayerArgs& L, const DtypeArgs& D, int sem, void* out, int out_dtype, hipStream_t st) {
  if (L.n_tiles == 0) return hipSuccess;
  switch (sem) {
    case SEM_FAST: return dequant_dt<SEM_FAST>(L, D, out, out_dtype, L.n_tiles, st);
    case SEM_ROUTE0: return dequant_dt<SEM_ROUTE0>(L, D, out, out_dtype, L.n_tiles, st);
    case SEM_ROUTE1: return dequant_dt<SEM_ROUTE1>(L, D, out, out_dtype, L.n_tiles, st);
    default: return dequant_dt<SEM_RECON>(L, D, out, out_dtype, L.n_tiles, st);
  }
}

template <int SEM>
static hipError_t generic_dt(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, const void* x, int64_t M,
                             hipStream_t st) {
  dim3 grid(L.n_tiles, (unsigned)((M + GM - 1) / GM)), block(256);
  if (D.x_dtype == WAL_BF16)
    hipLaunchKernelGGL((rvq_generic_linear_kernel<SEM, WAL_BF16>), grid, block, 0, st, L, D, E, x, M);
  else if (D.x_dtype == WAL_F16)
    hipLaunchKernelGGL((rvq_generic_linear_kernel<SEM, WAL_F16>), grid, block, 0, st, L, D, E, x, M);
  else
    hipLaunchKernelGGL((rvq_generic_linear_kernel<SEM, WAL_F32>), grid, block, 0, st, L, D, E, x, M);
  return hipGetLastError();
}

hipError_t launch_generic_linear(const LayerArgs& L, const DtypeArgs& D, const EpilogueArgs& E, int sem,
                                 const void* x, int64_t M, hipStream_t st) {
  if (L.n_tiles == 0 || M == 0) return hipSuccess;
  switch (sem) {
    case SEM_FAST: return generic_dt<SEM_FAST>(L, D, E, x, M, st);
    case SEM_TRITON: return generic_dt<SEM_TRITON>(L, D, E, x, M, st);
    case SEM_ROUTE0: return generic_dt<SEM_ROUTE0>(L, D, E, x, M, st);
    case SEM_ROUTE1: return generic_dt<SEM_ROUTE1>(L, D, E, x, M, st);
    case SEM_STAGEWISE: return generic_dt<SEM_STAGEWISE>(L, D, E, x, M, st);
    default: return generic_dt<SEM_RECON>(L, D, E, x, M, st);
  }
}

// ---------------------------------------------------------------------------
// Split-K reduction of the 128 x 256 prefill tile: one thread per output,
// the slices' fp32 partials summed in ascending slice order from +0 (so the
// result does not depend on the order the slices ran in), then the same
// epilogue as an unsplit launch (bias, rounding to y's dtype).  The partial
// rows have the stride of y (E.ldy).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rvq_splitk_reduce_kernel(const float* __restrict__ part, int ksplit, int64_t M,
                                                                EpilogueArgs E) {
  const int64_t N = E.ldy;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * N) return;
  const int64_t slice = M * N;
  float v = 0.0f;
  for (int s = 0; s < ksplit; ++s) v += part[(int64_t)s * slice + i];
  store_output(E, i / N, i - (i / N) * N, v);
}

hipError_t launch_splitk_reduce(const float* part, int ksplit, int64_t M, const EpilogueArgs& E, hipStream_t st) {
  const int64_t n = M * E.ldy;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(rvq_splitk_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, part, ksplit, M,
                     E);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Codebook image: every entry of every stage of every group converted once
// into the form the MFMA kernels stage in LDS (store_codebook_entry, the same
// code the kernels run when they convert raw codebooks themselves).  One
// thread per entry.
// ---------------------------------------------------------------------------
template <int LMODE, int SEM, int XDT>
__global__ __launch_bounds__(256) void rvq_image_kernel(LayerArgs L, DtypeArgs D, uint8_t* __restrict__ dst) {
  const int S = L.num_stages, K = L.codebook_size;
  const int64_t per_group = (int64_t)S * K;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= per_group * L.n_groups) return;
  const int g = (int)(e / per_group);
  const int rem = (int)(e - (int64_t)g * per_group);
  const int s = rem / K;
  const int k = rem - s * K;
  const void* cbp;
  const void* ssp;
  if (L.plan == nullptr) {
    cbp = L.g0.codebooks[s];
    ssp = L.g0.stage_scales;
  } else {
    typedef const __attribute__((address_space(1))) wal_rvq_group g_group_t;
    const __attribute__((address_space(1))) char* base = (const __attribute__((address_space(1))) char*)(L.plan);
    g_group_t* G = (g_group_t*)(base + ((const __attribute__((address_space(1))) PlanHeader*)base)->groups_offset) + g;
    cbp = G->codebooks[s];
    ssp = G->stage_scales;
  }
  const char* cb = static_cast<const char*>(cbp);
  u32x4_t raw[2];
  if (D.cb_dtype == WAL_F32) {
    raw[0] = ldg128(cb + (size_t)k * 32);
    raw[1] = ldg128(cb + (size_t)k * 32 + 16);
  } else {
    raw[0] = ldg128(cb + (size_t)k * 16);
    raw[1] = u32x4_t{0, 0, 0, 0};
  }
  const bool has_ss = ssp != nullptr;
  const float ss = has_ss ? load_f(ssp, D.sc_dtype, s) : 1.0f;
  store_codebook_entry<LMODE, SEM, XDT, false>(dst + (size_t)g * per_group * lds_entry_bytes<LMODE>(), rem, s, raw,
                                               D.cb_dtype, has_ss, ss, RowScale{0.0f, 0u, 0u});
}

template <int LMODE, int SEM>
static hipError_t image_x(const LayerArgs& L, const DtypeArgs& D, void* dst, hipStream_t st) {
  const int64_t n = (int64_t)L.n_groups * L.num_stages * L.codebook_size;
  dim3 grid((unsigned)((n + 255) / 256)), block(256);
  uint8_t* d = static_cast<uint8_t*>(dst);
  if (D.x_dtype == WAL_BF16) hipLaunchKernelGGL((rvq_image_kernel<LMODE, SEM, WAL_BF16>), grid, block, 0, st, L, D, d);
  else hipLaunchKernelGGL((rvq_image_kernel<LMODE, SEM, WAL_F16>), grid, block, 0, st, L, D, d);
  return hipGetLastError();
}

hipError_t launch_image(const LayerArgs& L, const DtypeArgs& D, int sem, int lmode, void* dst, hipStream_t st) {
  if (lmode == LM_A16) return sem == SEM_FAST ? image_x<LM_A16, SEM_FAST>(L, D, dst, st) : image_x<LM_A16, SEM_RECON>(L, D, dst, st);
  if (lmode == LM_H16) return image_x<LM_H16, SEM_RECON>(L, D, dst, st);
  return image_x<LM_F32, SEM_RECON>(L, D, dst, st);
}

}  // namespace wal
