// capi.hip -- the extern "C" entry points of libwal2026_amd.so.
//
// Every argument is validated on the host before a launch, so a malformed
// call returns an error code instead of reaching a kernel.  Shapes a kernel
// relies on (tile counts, alignment, LDS budget) are derived here.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <set>
#include <utility>

#include "wal2026_amd.h"
#include "rvq_kernels.h"

using namespace wal;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(WAL_EHIP, "%s: %s", what, hipGetErrorString(e));
}

// ---- scratch of wal_rvq_linear_noalloc ---------------------------------------
// The split-K partials of the entry point that allocates nothing live in this
// file-scope device array: every GPU the library runs on holds its own copy
// until the process ends.  In host code `scratch` names a host-side stand-in,
// not a device address: the device address is taken once per device with
// hipGetSymbolAddress (that device current) and only that pointer is passed
// to kernels.  Calls that overlap on one GPU share the array and race.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

// The current device's address of `scratch` (set up on the first call on a
// device), or nullptr with the error recorded.
void* scratch_for_current_device() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    fail(WAL_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    fail(WAL_EUNSUPPORTED, "device %d: the scratch table holds %d devices", dev, kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      fail(WAL_EHIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

bool is_float_dtype(int dt) { return dt == WAL_F16 || dt == WAL_BF16 || dt == WAL_F32; }
bool is_half_dtype(int dt) { return dt == WAL_F16 || dt == WAL_BF16; }
bool is_id_dtype(int dt) { return dt == WAL_U8 || dt == WAL_I16 || dt == WAL_U16 || dt == WAL_I32; }

int64_t id_capacity(int dt) {
  switch (dt) {
    case WAL_U8: return 256;
    case WAL_I16: return 32767;
    case WAL_U16: return 65536;
    default: return 2147483647LL;
  }
}

int id_bytes(int dt) { return dt == WAL_U8 ? 1 : (dt == WAL_I32 ? 4 : 2); }
int float_bytes(int dt) { return dt == WAL_F32 ? 4 : 2; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

int validate_layer(const wal_rvq_layer* Lh) {
  if (!Lh) return fail(WAL_EINVAL, "layer is NULL");
  const wal_rvq_layer& L = *Lh;
  if (L.in_features < 1 || L.out_features < 1)
    return fail(WAL_EINVAL, "in_features/out_features must be >= 1 (got %d, %d)", L.in_features, L.out_features);
  if (L.block_size < 1 || L.blocks_per_row < 1)
    return fail(WAL_EINVAL, "block_size/blocks_per_row must be >= 1");
  if ((int64_t)L.blocks_per_row * L.block_size < L.in_features)
    return fail(WAL_EINVAL, "blocks_per_row * block_size (%lld) < in_features (%d)",
                (long long)L.blocks_per_row * L.block_size, L.in_features);
  if (L.num_stages < 1 || L.num_stages > WAL_RVQ_MAX_STAGES)
    return fail(WAL_EINVAL, "num_stages must be in [1, %d] (got %d)", WAL_RVQ_MAX_STAGES, L.num_stages);
  if (!is_id_dtype(L.id_dtype)) return fail(WAL_EINVAL, "bad id dtype %d", L.id_dtype);
  if (!is_float_dtype(L.codebook_dtype)) return fail(WAL_EINVAL, "bad codebook dtype %d", L.codebook_dtype);
  if (!is_float_dtype(L.scale_dtype)) return fail(WAL_EINVAL, "bad scale dtype %d", L.scale_dtype);
  if (L.codebook_size < 1) return fail(WAL_EINVAL, "codebook_size must be >= 1");
  if (L.codebook_size > id_capacity(L.id_dtype))
    return fail(WAL_EINVAL, "codebook_size %d does not fit id dtype %d", L.codebook_size, L.id_dtype);
  if (L.scale_rows < 1) return fail(WAL_EINVAL, "scale_rows must be >= 1");
  if (L.n_groups < 1 || !L.groups) return fail(WAL_EINVAL, "layer has no groups");
  int64_t next = 0;
  for (int g = 0; g < L.n_groups; ++g) {
    const wal_rvq_group& G = L.groups[g];
    if (G.rows < 1) return fail(WAL_EINVAL, "group %d has %d rows", g, G.rows);
    if (G.row0 != next) return fail(WAL_EINVAL, "group %d starts at row %d, expected %lld", g, G.row0, (long long)next);
    next += G.rows;
    for (int s = 0; s < L.num_stages; ++s)
      if (!G.stage_ids[s] || !G.codebooks[s]) return fail(WAL_EINVAL, "group %d stage %d has a NULL buffer", g, s);
    if (!G.row_scale) return fail(WAL_EINVAL, "group %d has no row_scale", g);
  }
  if (next != L.out_features)
    return fail(WAL_EINVAL, "groups cover %lld rows, out_features is %d", (long long)next, L.out_features);
  if (L.n_groups > 1 && !L.plan) return fail(WAL_EINVAL, "a layer with %d groups needs a plan", L.n_groups);
  return WAL_OK;
}

struct PlanLayout {
  size_t groups_offset;
  size_t tiles_offset[kNumTileKinds];
  int32_t n_tiles[kNumTileKinds];
  size_t bytes;
};

PlanLayout plan_layout(const wal_rvq_layer& L) {
  PlanLayout P;
  size_t off = (sizeof(PlanHeader) + 15) & ~size_t(15);
  P.groups_offset = off;
  off += sizeof(wal_rvq_group) * L.n_groups;
  for (int k = 0; k < kNumTileKinds; ++k) {
    int64_t n = 0;
    for (int g = 0; g < L.n_groups; ++g) n += ceil_div(L.groups[g].rows, kTileRows[k]);
    P.n_tiles[k] = (int32_t)n;
    off = (off + 15) & ~size_t(15);
    P.tiles_offset[k] = off;
    off += sizeof(PlanTile) * n;
  }
  P.bytes = off;
  return P;
}

int n_tiles_of(const wal_rvq_layer& L, int kind) {
  int64_t n = 0;
  for (int g = 0; g < L.n_groups; ++g) n += ceil_div(L.groups[g].rows, kTileRows[kind]);
  return (int)n;
}

LayerArgs make_args(const wal_rvq_layer& L, int kind, uint32_t active_mask) {
  LayerArgs A;
  memset(&A, 0, sizeof(A));
  A.in_features = L.in_features;
  A.out_features = L.out_features;
  A.block_size = L.block_size;
  A.blocks_per_row = L.blocks_per_row;
  A.codebook_size = L.codebook_size;
  A.num_stages = L.num_stages;
  A.scale_rows = L.scale_rows;
  A.scale_shift = (L.scale_rows & (L.scale_rows - 1)) == 0 ? __builtin_ctz((unsigned)L.scale_rows) : -1;
  A.tile_kind = kind;
  A.tile_rows = kTileRows[kind];
  A.n_tiles = n_tiles_of(L, kind);
  A.active_mask = active_mask;
  A.plan = L.n_groups > 1 ? reinterpret_cast<const PlanHeader*>(L.plan) : nullptr;
  A.g0 = L.groups[0];
  A.n_groups = L.n_groups;
  A.image = nullptr;
  if (A.plan != nullptr) {
    const PlanLayout P = plan_layout(L);
    A.plan_tiles = reinterpret_cast<const PlanTile*>(static_cast<const char*>(L.plan) + P.tiles_offset[kind]);
    A.plan_groups = reinterpret_cast<const wal_rvq_group*>(static_cast<const char*>(L.plan) + P.groups_offset);
  }
  return A;
}

}  // namespace

namespace wal {

// CUs of the current device (cached per device; 256 when unknown).
int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

}  // namespace wal

namespace {

// LDS form of the codebooks for the MFMA kernels.
int lds_mode_for(const wal_rvq_layer& L, int sem) {
  if (sem == SEM_FAST || L.num_stages == 1) return LM_A16;
  bool any_ss = false;
  for (int g = 0; g < L.n_groups; ++g) any_ss |= L.groups[g].stage_scales != nullptr;
  return (L.codebook_dtype == WAL_F16 && !any_ss) ? LM_H16 : LM_F32;
}

// Layout conditions of the block-size-8 MFMA kernels (decode and prefill).
bool mfma_layout_ok(const wal_rvq_layer& L, int x_dtype, const void* x) {
  if (L.block_size != 8 || (int64_t)L.blocks_per_row * 8 != L.in_features) return false;
  if (L.blocks_per_row % 16 != 0) return false;
  if (L.num_stages > 4) return false;
  if (L.id_dtype == WAL_I32) return false;
  if (!is_half_dtype(x_dtype) || !aligned16(x)) return false;
  if (!is_half_dtype(L.scale_dtype)) return false;
  for (int g = 0; g < L.n_groups; ++g) {
    const wal_rvq_group& G = L.groups[g];
    if (G.block_scale) return false;
    for (int s = 0; s < L.num_stages; ++s)
      if (!aligned16(G.stage_ids[s]) || !aligned16(G.codebooks[s])) return false;
  }
  // index and scale buffers are addressed with 32-bit buffer offsets
  for (int g = 0; g < L.n_groups; ++g)
    if ((int64_t)L.groups[g].rows * L.blocks_per_row * id_bytes(L.id_dtype) >= (int64_t)1 << 31) return false;
  return true;
}

// The prefill kernel's table fits LDS beside its double-buffered 128 x 48 and
// 256 x 48 16-bit tiles (8-bit ids with K < 256 get a 256-entry margin, see
// rvq_prefill_impl.h).
bool prefill_table_fits(const wal_rvq_layer& L, int sem) {
  const int esz = lds_mode_for(L, sem) == LM_F32 ? 32 : 16;
  const size_t cb = ((size_t)L.num_stages * L.codebook_size +
                     (L.id_dtype == WAL_U8 && L.codebook_size < 256 ? 256 - L.codebook_size : 0)) * esz;
  return cb <= (size_t)(kLdsMaxBytes - 2 * (128 + 256) * 48 * 2);
}

// Which kernel serves a wal_rvq_linear call, with its launch plan.
struct Route {
  int kernel;      // WAL_KERNEL_*
  DecodePlan dp;   // decode
  int shape;       // prefill: PrefillShape
  PrefillPlan pp;  // prefill: shape, split, grid
};

// allow_split: the call brings a workspace (wal_rvq_linear_ws), so the
// prefill planner may split the short tile's k-steps.
int route_linear(const wal_rvq_layer& L, int sem, int x_dtype, const void* x, int64_t m, bool allow_split, Route* r) {
  r->kernel = WAL_KERNEL_GENERIC;
  r->shape = -1;
  r->dp = DecodePlan{-1, -1, -1, -1, 0, 1};
  r->pp = PrefillPlan{-1, 1, -1, -1};
  if (m == 0) {
    r->kernel = WAL_KERNEL_NONE;
    return WAL_OK;
  }
  if (sem == SEM_STAGEWISE || !mfma_layout_ok(L, x_dtype, x)) return WAL_OK;
  const int lmode = lds_mode_for(L, sem);
  if (m <= 16) {
    const int force = decode_xmode_override();
    if (force == -2) return fail(WAL_EINVAL, "WAL2026_DECODE_XMODE must be reg, lds, greg, gtr or global");
    const int esz = lmode == LM_F32 ? 32 : 16;
    const bool segments = L.n_groups > 1 || decode_scaled_tables(L.num_stages, L.scale_rows);
    const int n_tiles = n_tiles_of(L, 0);
    if (plan_decode(esz, L.num_stages, L.codebook_size, (int)m, L.in_features, L.blocks_per_row, n_tiles,
                    device_cu_count(), segments, force, &r->dp)) {
      r->kernel = WAL_KERNEL_DECODE;
    } else if (force >= 0) {
      return fail(WAL_EUNSUPPORTED, "WAL2026_DECODE_XMODE forces x-mode %d, which does not apply to this layer at m = %lld",
                  force, (long long)m);
    }
    return WAL_OK;
  }
  if (!prefill_table_fits(L, sem)) return WAL_OK;
  const int force = prefill_tile_override();
  if (force == -2) return fail(WAL_EINVAL, "WAL2026_PREFILL_TILE must be short, tall or wide");
  const int force_ks = prefill_ksplit_override();
  if (force_ks < 0) return fail(WAL_EINVAL, "WAL2026_PREFILL_KSPLIT must be an integer in 1 .. %d", kMaxKSplit);
  r->kernel = WAL_KERNEL_PREFILL;
  r->pp = plan_prefill(L.num_stages, lmode, id_bytes(L.id_dtype), m, L.out_features, n_tiles_of(L, 2),
                       L.blocks_per_row, device_cu_count(), force, allow_split, force_ks);
  r->shape = r->pp.shape;
  return WAL_OK;
}

// Resolve FAST on groups that are not "plain" (src/runtime.py:416-429, :579-580).
int resolve_semantics(const wal_rvq_layer& L, int semantics, int* sem) {
  if (semantics == WAL_RVQ_RECONSTRUCT) {
    *sem = SEM_RECON;
    return WAL_OK;
  }
  if (semantics == WAL_RVQ_STAGEWISE) {
    // src/runtime.py:837-846, :879-880: block-scaled groups are refused
    for (int g = 0; g < L.n_groups; ++g)
      if (L.groups[g].block_scale) return fail(WAL_EUNSUPPORTED, "STAGEWISE on a group with block_scale");
    *sem = SEM_STAGEWISE;
    return WAL_OK;
  }
  if (semantics != WAL_RVQ_RECONSTRUCT_FAST) return fail(WAL_EINVAL, "unknown semantics %d", semantics);
  int with_bs = 0;
  for (int g = 0; g < L.n_groups; ++g) with_bs += L.groups[g].block_scale != nullptr;
  if (with_bs == 0) *sem = SEM_FAST;
  else if (with_bs == L.n_groups) *sem = SEM_RECON;
  else return fail(WAL_EUNSUPPORTED, "RECONSTRUCT_FAST on a layer where only some groups have block_scale");
  return WAL_OK;
}

uint32_t resolve_mask(const wal_rvq_layer& L, uint32_t mask) {
  const uint32_t all = (L.num_stages >= 32) ? 0xffffffffu : ((1u << L.num_stages) - 1u);
  mask &= all;
  return mask ? mask : all;
}

}  // namespace

namespace wal {

hipError_t allow_max_lds(const void* kern) {
  static std::mutex mu;
  static std::set<std::pair<int, const void*>> done;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mu);
  if (done.count({dev, kern})) return hipSuccess;
  e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMaxBytes);
  if (e == hipSuccess) done.insert({dev, kern});
  return e;
}

// Read-bandwidth probe: a streaming read of n bytes with the decode kernel's
// load form (16-byte buffer loads with the streaming hint, four in flight per
// lane), grid-stride, XOR-reduced so that nothing is optimised away; lane 0 of
// each wave stores its wave's XOR with a vector store.
__global__ __launch_bounds__(1024) void read_probe_kernel(const void* src, uint32_t n, uint32_t* partial) {
  const bufrsrc_t r = make_rsrc(src);
  const uint32_t stride = gridDim.x * blockDim.x * 16u;
  u32x4_t acc = {0u, 0u, 0u, 0u};
  for (uint32_t o = (blockIdx.x * blockDim.x + threadIdx.x) * 16u; o < n; o += 4 * stride) {
    // pieces past n (and offsets past the resource's range) read zeros
    const u32x4_t a = ldbuf128_stream(r, o);
    const u32x4_t b = ldbuf128_stream(r, o + stride < n ? o + stride : kBufOOB);
    const u32x4_t c = ldbuf128_stream(r, o + 2 * stride < n ? o + 2 * stride : kBufOOB);
    const u32x4_t d = ldbuf128_stream(r, o + 3 * stride < n ? o + 3 * stride : kBufOOB);
    acc ^= a ^ b ^ c ^ d;
  }
  uint32_t v = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v ^= __shfl_xor(v, m, 64);
  if ((threadIdx.x & 63) == 0) partial[blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)] = v;
}

}  // namespace wal

extern "C" {

const char* wal_last_error(void) { return g_err; }

int wal_abi_version(void) { return WAL_ABI_VERSION; }

int wal_rvq_plan_size(const wal_rvq_layer* layer, size_t* bytes) {
  g_err[0] = 0;
  if (!bytes) return fail(WAL_EINVAL, "bytes is NULL");
  if (!layer || layer->n_groups < 1 || !layer->groups) return fail(WAL_EINVAL, "layer has no groups");
  *bytes = plan_layout(*layer).bytes;
  return WAL_OK;
}

int wal_rvq_plan_build(const wal_rvq_layer* layer, void* dst, size_t bytes) {
  g_err[0] = 0;
  if (!layer || layer->n_groups < 1 || !layer->groups) return fail(WAL_EINVAL, "layer has no groups");
  if (!dst) return fail(WAL_EINVAL, "dst is NULL");
  const PlanLayout P = plan_layout(*layer);
  if (bytes < P.bytes) return fail(WAL_ESIZE, "plan needs %zu bytes, got %zu", P.bytes, bytes);
  memset(dst, 0, P.bytes);
  char* base = static_cast<char*>(dst);
  PlanHeader* H = reinterpret_cast<PlanHeader*>(base);
  H->magic = kPlanMagic;
  H->n_groups = layer->n_groups;
  H->groups_offset = (int32_t)P.groups_offset;
  memcpy(base + P.groups_offset, layer->groups, sizeof(wal_rvq_group) * layer->n_groups);
  for (int k = 0; k < kNumTileKinds; ++k) {
    H->tiles_offset[k] = (int32_t)P.tiles_offset[k];
    H->n_tiles[k] = P.n_tiles[k];
    PlanTile* T = reinterpret_cast<PlanTile*>(base + P.tiles_offset[k]);
    int i = 0;
    for (int g = 0; g < layer->n_groups; ++g) {
      const wal_rvq_group& G = layer->groups[g];
      for (int r = 0; r < G.rows; r += kTileRows[k]) {
        T[i].group = g;
        T[i].row0 = r;
        T[i].rows = (G.rows - r) < kTileRows[k] ? (G.rows - r) : kTileRows[k];
        T[i].out_row0 = G.row0 + r;
        ++i;
      }
    }
  }
  return WAL_OK;
}

// Image bytes: per group, S x K entries of the LdsMode entry size.
size_t image_bytes(const wal_rvq_layer& L, int sem) {
  const int esz = lds_mode_for(L, sem) == LM_F32 ? 32 : 16;
  return (size_t)L.n_groups * L.num_stages * L.codebook_size * esz;
}

int image_args(const wal_rvq_layer* layer, int semantics, int x_dtype, int* sem) {
  int rc = validate_layer(layer);
  if (rc) return rc;
  if (layer->block_size != 8) return fail(WAL_EUNSUPPORTED, "codebook images are for block_size 8 (got %d)", layer->block_size);
  if (layer->num_stages > 4) return fail(WAL_EUNSUPPORTED, "codebook images are for at most 4 stages");
  if (!is_half_dtype(x_dtype)) return fail(WAL_EINVAL, "x dtype must be F16 or BF16 (got %d)", x_dtype);
  if (semantics == WAL_RVQ_STAGEWISE) return fail(WAL_EUNSUPPORTED, "STAGEWISE calls use no codebook image");
  return resolve_semantics(*layer, semantics, sem);
}

int wal_rvq_image_size(const wal_rvq_layer* layer, int semantics, int x_dtype, size_t* bytes) {
  g_err[0] = 0;
  if (!bytes) return fail(WAL_EINVAL, "bytes is NULL");
  int sem = 0;
  int rc = image_args(layer, semantics, x_dtype, &sem);
  if (rc) return rc;
  *bytes = image_bytes(*layer, sem);
  return WAL_OK;
}

int wal_rvq_image_build(const wal_rvq_layer* layer, int semantics, int x_dtype, void* dst, size_t bytes,
                        void* stream) {
  g_err[0] = 0;
  int sem = 0;
  int rc = image_args(layer, semantics, x_dtype, &sem);
  if (rc) return rc;
  if (!dst || !aligned16(dst)) return fail(WAL_EINVAL, "dst must be a 16-byte aligned device pointer");
  const size_t need = image_bytes(*layer, sem);
  if (bytes < need) return fail(WAL_ESIZE, "image needs %zu bytes, got %zu", need, bytes);
  for (int g = 0; g < layer->n_groups; ++g)
    for (int s = 0; s < layer->num_stages; ++s)
      if (!aligned16(layer->groups[g].codebooks[s])) return fail(WAL_EINVAL, "codebooks must be 16-byte aligned");
  LayerArgs A = make_args(*layer, 0, resolve_mask(*layer, 0));
  DtypeArgs D{layer->id_dtype, layer->codebook_dtype, layer->scale_dtype, x_dtype};
  hipError_t e = launch_image(A, D, sem, lds_mode_for(*layer, sem), dst, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? WAL_OK : hip_fail(e, "wal_rvq_image_build launch");
}

int wal_rvq_reconstruct(const wal_rvq_layer* layer, int semantics, uint32_t active_stage_mask, void* w_out,
                        int out_dtype, void* stream) {
  g_err[0] = 0;
  int rc = validate_layer(layer);
  if (rc) return rc;
  if (!w_out) return fail(WAL_EINVAL, "w_out is NULL");
  if (!is_float_dtype(out_dtype)) return fail(WAL_EINVAL, "bad out dtype %d", out_dtype);
  int sem = 0;
  if (semantics == WAL_RVQ_STAGEWISE) return fail(WAL_EINVAL, "STAGEWISE has no dense weight (it rounds per stage output)");
  if ((rc = resolve_semantics(*layer, semantics, &sem))) return rc;
  const uint32_t mask = resolve_mask(*layer, active_stage_mask);
  DtypeArgs D{layer->id_dtype, layer->codebook_dtype, layer->scale_dtype, out_dtype};
  hipError_t e;
  const int lmode = lds_mode_for(*layer, sem);
  const size_t table = (size_t)layer->num_stages * layer->codebook_size * (lmode == LM_F32 ? 32 : 16);
  if ((sem == SEM_RECON || sem == SEM_FAST) && mfma_layout_ok(*layer, out_dtype, w_out) && table <= kLdsMaxBytes) {
    // the block-size-8 kernel: 16-row tiles, 64-row tiles when the staged
    // table is large enough that staging it per 16 rows would cost as much
    // as the rows' weights
    LayerArgs A = make_args(*layer, table >= 32 * 1024 ? 1 : 0, mask);
    e = launch_dequant8(A, D, sem, lmode, w_out, static_cast<hipStream_t>(stream));
  } else {
    LayerArgs A = make_args(*layer, 0, mask);
    e = launch_dequant(A, D, sem, w_out, out_dtype, static_cast<hipStream_t>(stream));
  }
  return e == hipSuccess ? WAL_OK : hip_fail(e, "wal_rvq_reconstruct launch");
}

// Bytes of the split-K partials a prefill call with this plan writes.
static size_t splitk_bytes(const wal_rvq_layer& L, int64_t m, const Route& r) {
  return r.kernel == WAL_KERNEL_PREFILL && r.pp.ksplit > 1 ? (size_t)r.pp.ksplit * (size_t)m * L.out_features * 4 : 0;
}

static int linear_impl(const wal_rvq_layer* layer, int semantics, uint32_t active_stage_mask, const void* x, int64_t m,
                int x_dtype, const void* bias, int bias_dtype, void* y, int y_dtype, void* workspace,
                size_t workspace_bytes, void* stream) {
  g_err[0] = 0;
  int rc = validate_layer(layer);
  if (rc) return rc;
  if (m < 0) return fail(WAL_EINVAL, "m must be >= 0");
  if (m == 0) return WAL_OK;
  if (!x || !y) return fail(WAL_EINVAL, "x and y must not be NULL");
  if (!is_float_dtype(x_dtype)) return fail(WAL_EINVAL, "bad x dtype %d", x_dtype);
  if (!is_float_dtype(y_dtype)) return fail(WAL_EINVAL, "bad y dtype %d", y_dtype);
  if (bias && !is_float_dtype(bias_dtype)) return fail(WAL_EINVAL, "bad bias dtype %d", bias_dtype);
  int sem = 0;
  if ((rc = resolve_semantics(*layer, semantics, &sem))) return rc;
  const uint32_t mask = resolve_mask(*layer, active_stage_mask);
  hipStream_t st = static_cast<hipStream_t>(stream);
  DtypeArgs D{layer->id_dtype, layer->codebook_dtype, layer->scale_dtype, x_dtype};
  // bias inside F.linear (mode 1), or added to the rounded stagewise output (mode 2, src/runtime.py:1470-1473)
  EpilogueArgs E{y, bias, (int64_t)layer->out_features, y_dtype, x_dtype, bias_dtype,
                 bias ? (sem == SEM_STAGEWISE ? 2 : 1) : 0};
  if (layer->image != nullptr && layer->image_tag != WAL_RVQ_IMAGE_TAG(semantics, x_dtype))
    return fail(WAL_EINVAL, "the layer's codebook image was built for tag 0x%x, this call needs 0x%x",
                layer->image_tag, WAL_RVQ_IMAGE_TAG(semantics, x_dtype));
  if (workspace != nullptr && !aligned16(workspace)) return fail(WAL_EINVAL, "workspace must be 16-byte aligned");
  Route r;
  if ((rc = route_linear(*layer, sem, x_dtype, x, m, workspace != nullptr, &r))) return rc;
  const size_t need = splitk_bytes(*layer, m, r);
  if (need > 0 && workspace_bytes < need)
    return fail(WAL_ESIZE, "workspace of %zu bytes, this call needs %zu (wal_rvq_linear_workspace_size)",
                workspace_bytes, need);
  hipError_t e;
  if (r.kernel == WAL_KERNEL_DECODE) {
    LayerArgs A = make_args(*layer, 0, mask);
    A.image = static_cast<const uint8_t*>(layer->image);
    e = launch_decode(A, D, E, sem, lds_mode_for(*layer, sem), x, (int)m, r.dp, st);
  } else if (r.kernel == WAL_KERNEL_PREFILL) {
    LayerArgs A = make_args(*layer, 2, mask);
    const PrefillSplit sp{need > 0 ? r.pp.ksplit : 1, need > 0 ? static_cast<float*>(workspace) : nullptr};
    e = launch_prefill(A, D, E, sem, lds_mode_for(*layer, sem), x, m, r.shape, sp, st);
  } else {
    // the generic kernel (STAGEWISE runs every stage: its mask is all stages)
    LayerArgs A = make_args(*layer, 1, sem == SEM_STAGEWISE ? resolve_mask(*layer, 0) : mask);
    e = launch_generic_linear(A, D, E, sem, x, m, st);
  }
  return e == hipSuccess ? WAL_OK : hip_fail(e, "wal_rvq_linear launch");
}

int wal_rvq_linear(const wal_rvq_layer* layer, int semantics, uint32_t active_stage_mask, const void* x, int64_t m,
                   int x_dtype, const void* bias, int bias_dtype, void* y, int y_dtype, void* stream) {
  return linear_impl(layer, semantics, active_stage_mask, x, m, x_dtype, bias, bias_dtype, y, y_dtype, nullptr, 0,
                     stream);
}

int wal_rvq_linear_ws(const wal_rvq_layer* layer, int semantics, uint32_t active_stage_mask, const void* x,
                      int64_t m, int x_dtype, const void* bias, int bias_dtype, void* y, int y_dtype,
                      void* workspace, size_t workspace_bytes, void* stream) {
  return linear_impl(layer, semantics, active_stage_mask, x, m, x_dtype, bias, bias_dtype, y, y_dtype, workspace,
                     workspace_bytes, stream);
}

int wal_rvq_linear_noalloc(const wal_rvq_layer* layer, int semantics, uint32_t active_stage_mask, const void* x,
                           int64_t m, int x_dtype, const void* bias, int bias_dtype, void* y, int y_dtype,
                           void* stream) {
  g_err[0] = 0;
  size_t need = 0;
  int rc = wal_rvq_linear_workspace_size(layer, semantics, x, m, x_dtype, &need);
  if (rc) return rc;
  if (need > kNoAllocScratchBytes)
    return fail(WAL_ESIZE, "this call needs %zu bytes of split-K scratch, the maximum is %zu (use wal_rvq_linear_ws)",
                need, kNoAllocScratchBytes);
  void* ptr = nullptr;
  if (need > 0 && (ptr = scratch_for_current_device()) == nullptr) return WAL_EHIP;
  // every partial the kernels read is written first in the same call: nothing
  // in the scratch has to start at zero
  return linear_impl(layer, semantics, active_stage_mask, x, m, x_dtype, bias, bias_dtype, y, y_dtype, ptr,
                     need > 0 ? kNoAllocScratchBytes : 0, stream);
}

int wal_rvq_linear_workspace_size(const wal_rvq_layer* layer, int semantics, const void* x, int64_t m, int x_dtype,
                                  size_t* bytes) {
  g_err[0] = 0;
  if (!bytes) return fail(WAL_EINVAL, "bytes is NULL");
  *bytes = 0;
  int rc = validate_layer(layer);
  if (rc) return rc;
  if (m < 0) return fail(WAL_EINVAL, "m must be >= 0");
  if (!is_float_dtype(x_dtype)) return fail(WAL_EINVAL, "bad x dtype %d", x_dtype);
  int sem = 0;
  if ((rc = resolve_semantics(*layer, semantics, &sem))) return rc;
  Route r;
  if ((rc = route_linear(*layer, sem, x_dtype, x, m, true, &r))) return rc;
  *bytes = splitk_bytes(*layer, m, r);
  return WAL_OK;
}

int wal_rvq_linear_info(const wal_rvq_layer* layer, int semantics, const void* x, int64_t m, int x_dtype,
                        wal_rvq_launch_info* info) {
  g_err[0] = 0;
  if (!info) return fail(WAL_EINVAL, "info is NULL");
  int rc = validate_layer(layer);
  if (rc) return rc;
  if (m < 0) return fail(WAL_EINVAL, "m must be >= 0");
  if (!is_float_dtype(x_dtype)) return fail(WAL_EINVAL, "bad x dtype %d", x_dtype);
  int sem = 0;
  if ((rc = resolve_semantics(*layer, semantics, &sem))) return rc;
  Route r;
  if ((rc = route_linear(*layer, sem, x_dtype, x, m, true, &r))) return rc;
  info->kernel = r.kernel;
  const bool dec = r.kernel == WAL_KERNEL_DECODE, pre = r.kernel == WAL_KERNEL_PREFILL;
  info->x_mode = dec ? r.dp.xmode : -1;
  info->table_slots = dec ? r.dp.nslots : -1;
  info->grid = dec ? r.dp.grid : (pre ? r.pp.grid : -1);
  info->share = dec ? r.dp.share : (pre ? r.pp.ksteps : -1);
  info->lds_bytes = dec ? (int32_t)r.dp.lds : -1;
  info->tile_shape = pre ? r.shape : -1;
  info->k_splits = pre ? r.pp.ksplit : -1;
  return WAL_OK;
}

int wal_rvq_group_linear_matmul(const void* x, int64_t m, int64_t k_in, int x_dtype, const void* stage_ids,
                                int id_dtype, int32_t num_stages, int64_t n, int64_t blocks_per_row,
                                const void* codebooks, int cb_dtype, int64_t codebook_size, int32_t block_size,
                                const void* row_scale, int rs_dtype, void* out, int out_dtype, void* stream) {
  g_err[0] = 0;
  if (!x || !stage_ids || !codebooks || !row_scale || !out) return fail(WAL_EINVAL, "NULL buffer");
  if (m < 0 || n < 1 || k_in < 1 || blocks_per_row < 1 || block_size < 1 || codebook_size < 1)
    return fail(WAL_EINVAL, "bad shape");
  if (num_stages < 1 || num_stages > WAL_RVQ_MAX_STAGES) return fail(WAL_EINVAL, "bad stage count %d", num_stages);
  // src/triton_id_matmul.py:246-248: the padded width must equal x's width
  if (blocks_per_row * block_size != k_in)
    return fail(WAL_EINVAL, "Feature mismatch: expected %lld, got %lld", (long long)(blocks_per_row * block_size),
                (long long)k_in);
  if (!is_float_dtype(x_dtype)) return fail(WAL_EINVAL, "bad x dtype");
  if (!is_id_dtype(id_dtype) || !is_half_dtype(cb_dtype) || !is_float_dtype(rs_dtype) || !is_float_dtype(out_dtype))
    return fail(WAL_EINVAL, "bad dtype");
  if (codebook_size > id_capacity(id_dtype)) return fail(WAL_EINVAL, "codebook_size does not fit id dtype");
  if (n > 0x7fffffff || k_in > 0x7fffffff) return fail(WAL_EINVAL, "shape too large");
  if (m == 0) return WAL_OK;
  wal_rvq_group G;
  memset(&G, 0, sizeof(G));
  for (int s = 0; s < num_stages; ++s) {
    G.stage_ids[s] = static_cast<const char*>(stage_ids) + (size_t)s * n * blocks_per_row * id_bytes(id_dtype);
    G.codebooks[s] = static_cast<const char*>(codebooks) + (size_t)s * codebook_size * block_size * float_bytes(cb_dtype);
  }
  G.row_scale = row_scale;
  G.row0 = 0;
  G.rows = (int32_t)n;
  wal_rvq_layer L;
  memset(&L, 0, sizeof(L));
  L.in_features = (int32_t)k_in;
  L.out_features = (int32_t)n;
  L.block_size = block_size;
  L.blocks_per_row = (int32_t)blocks_per_row;
  L.codebook_size = (int32_t)codebook_size;
  L.num_stages = num_stages;
  L.id_dtype = id_dtype;
  L.codebook_dtype = cb_dtype;
  L.scale_dtype = rs_dtype;
  L.scale_rows = 1;
  L.n_groups = 1;
  L.groups = &G;
  LayerArgs A = make_args(L, 1, 0);
  DtypeArgs D{id_dtype, cb_dtype, rs_dtype, x_dtype};
  EpilogueArgs E{out, nullptr, n, out_dtype, x_dtype, WAL_F32, 0};
  hipError_t e = launch_generic_linear(A, D, E, SEM_TRITON, x, m, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? WAL_OK : hip_fail(e, "wal_rvq_group_linear_matmul launch");
}

int wal_id_route_linear(const void* x, int64_t m, int64_t k, int x_dtype, const void* ids, int id_dtype, int64_t n,
                        const void* codebook_sum, int64_t routes, int cs_dtype, const void* row_scale,
                        const void* bias, int bias_dtype, int mode, void* y, int y_dtype, void* stream) {
  g_err[0] = 0;
  if (!x || !ids || !codebook_sum || !row_scale || !y) return fail(WAL_EINVAL, "NULL buffer");
  if (m < 0 || k < 1 || n < 1 || routes < 1) return fail(WAL_EINVAL, "bad shape");
  if (n > 0x7fffffff || k > 0x7fffffff || routes > 0x7fffffff) return fail(WAL_EINVAL, "shape too large");
  if (mode != 0 && mode != 1) return fail(WAL_EINVAL, "mode must be 0 or 1");
  if (!is_float_dtype(x_dtype)) return fail(WAL_EINVAL, "bad x dtype");
  if (!(id_dtype == WAL_I16 || id_dtype == WAL_U16 || id_dtype == WAL_I32)) return fail(WAL_EINVAL, "bad id dtype");
  if (!is_half_dtype(cs_dtype) || !is_float_dtype(y_dtype)) return fail(WAL_EINVAL, "bad dtype");
  if (bias && !is_float_dtype(bias_dtype)) return fail(WAL_EINVAL, "bad bias dtype");
  if (m == 0) return WAL_OK;
  wal_rvq_group G;
  memset(&G, 0, sizeof(G));
  G.stage_ids[0] = ids;
  G.codebooks[0] = codebook_sum;
  G.row_scale = row_scale;
  G.rows = (int32_t)n;
  wal_rvq_layer L;
  memset(&L, 0, sizeof(L));
  L.in_features = (int32_t)k;
  L.out_features = (int32_t)n;
  L.block_size = 1;
  L.blocks_per_row = (int32_t)k;
  L.codebook_size = (int32_t)routes;
  L.num_stages = 1;
  L.id_dtype = id_dtype;
  L.codebook_dtype = cs_dtype;
  L.scale_dtype = cs_dtype;
  L.scale_rows = 1;
  L.n_groups = 1;
  L.groups = &G;
  LayerArgs A = make_args(L, 1, 0);
  DtypeArgs D{id_dtype, cs_dtype, cs_dtype, x_dtype};
  EpilogueArgs E{y, bias, n, y_dtype, x_dtype, bias_dtype, bias ? (mode == 0 ? 1 : 2) : 0};
  hipError_t e = launch_generic_linear(A, D, E, mode == 0 ? SEM_ROUTE0 : SEM_ROUTE1, x, m,
                                       static_cast<hipStream_t>(stream));
  return e == hipSuccess ? WAL_OK : hip_fail(e, "wal_id_route_linear launch");
}

int wal_id_route_reconstruct(const void* ids, int id_dtype, int64_t n, int64_t k, const void* codebook_sum,
                             int64_t routes, int cs_dtype, const void* row_scale, int mode, int out_dtype, void* w_out,
                             void* stream) {
  g_err[0] = 0;
  if (!ids || !codebook_sum || !row_scale || !w_out) return fail(WAL_EINVAL, "NULL buffer");
  if (k < 1 || n < 1 || routes < 1) return fail(WAL_EINVAL, "bad shape");
  if (n > 0x7fffffff || k > 0x7fffffff || routes > 0x7fffffff) return fail(WAL_EINVAL, "shape too large");
  if (mode != 0 && mode != 1) return fail(WAL_EINVAL, "mode must be 0 or 1");
  if (!(id_dtype == WAL_I16 || id_dtype == WAL_U16 || id_dtype == WAL_I32)) return fail(WAL_EINVAL, "bad id dtype");
  if (!is_half_dtype(cs_dtype) || !is_float_dtype(out_dtype)) return fail(WAL_EINVAL, "bad dtype");
  wal_rvq_group G;
  memset(&G, 0, sizeof(G));
  G.stage_ids[0] = ids;
  G.codebooks[0] = codebook_sum;
  G.row_scale = row_scale;
  G.rows = (int32_t)n;
  wal_rvq_layer L;
  memset(&L, 0, sizeof(L));
  L.in_features = (int32_t)k;
  L.out_features = (int32_t)n;
  L.block_size = 1;
  L.blocks_per_row = (int32_t)k;
  L.codebook_size = (int32_t)routes;
  L.num_stages = 1;
  L.id_dtype = id_dtype;
  L.codebook_dtype = cs_dtype;
  L.scale_dtype = cs_dtype;
  L.scale_rows = 1;
  L.n_groups = 1;
  L.groups = &G;
  LayerArgs A = make_args(L, 0, 0);
  DtypeArgs D{id_dtype, cs_dtype, cs_dtype, out_dtype};
  hipError_t e = launch_dequant(A, D, mode == 0 ? SEM_ROUTE0 : SEM_ROUTE1, w_out, out_dtype,
                                static_cast<hipStream_t>(stream));
  return e == hipSuccess ? WAL_OK : hip_fail(e, "wal_id_route_reconstruct launch");
}

int wal_rvq_assign(const float* blocks, int64_t n, int d, const float* codebook, int64_t k_cb, int64_t* ids,
                   float* min_dist, void* stream) {
  g_err[0] = 0;
  if (n < 0) return fail(WAL_EINVAL, "n must be >= 0 (got %lld)", (long long)n);
  if (n == 0) return WAL_OK;
  if (!blocks || !codebook || !ids || !min_dist) return fail(WAL_EINVAL, "NULL buffer");
  if (!(d == 1 || d == 2 || d == 4 || d == 8 || d == 16 || d == 32))
    return fail(WAL_EUNSUPPORTED, "block size %d not supported (1, 2, 4, 8, 16 or 32)", d);
  if (k_cb < 1 || k_cb > 0x7fffffff) return fail(WAL_EINVAL, "codebook size must be in [1, 2^31) (got %lld)", (long long)k_cb);
  if (d % 4 == 0 && (reinterpret_cast<uintptr_t>(blocks) & 15u) != 0)
    return fail(WAL_EINVAL, "blocks must be 16-byte aligned");
  hipError_t e = launch_assign(blocks, n, d, codebook, (int)k_cb, ids, min_dist, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? WAL_OK : hip_fail(e, "wal_rvq_assign launch");
}

int wal_rvq_centroid_sums(const int64_t* ids, int64_t n, const float* blocks, int d, int64_t k_cb, float* sums,
                          int64_t* counts, void* stream) {
  g_err[0] = 0;
  if (n < 0) return fail(WAL_EINVAL, "n must be >= 0 (got %lld)", (long long)n);
  if ((n > 0 && (!ids || !blocks)) || !sums || !counts) return fail(WAL_EINVAL, "NULL buffer");
  if (!(d == 1 || d == 2 || d == 4 || d == 8 || d == 16 || d == 32))
    return fail(WAL_EUNSUPPORTED, "block size %d not supported (1, 2, 4, 8, 16 or 32)", d);
  if (k_cb < 1 || k_cb > 0x7fffffff) return fail(WAL_EINVAL, "codebook size must be in [1, 2^31) (got %lld)", (long long)k_cb);
  hipError_t e = launch_centroid_sums(ids, n, blocks, d, (int)k_cb, sums, counts, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? WAL_OK : hip_fail(e, "wal_rvq_centroid_sums launch");
}

int wal_read_probe(const void* src, int64_t bytes, uint32_t* partial, int grid, int block, void* stream) {
  if (!src || !partial) return fail(WAL_EINVAL, "src and partial must be non-NULL");
  if (!aligned16(src)) return fail(WAL_EINVAL, "src must be 16-byte aligned");
  if (bytes < 0 || bytes % 16 != 0 || bytes > ((int64_t)1 << 31) - 16)
    return fail(WAL_EINVAL, "bytes must be a multiple of 16 in [0, 2^31 - 16] (got %lld)", (long long)bytes);
  if (grid < 1 || block < 64 || block > 1024 || block % 64 != 0)
    return fail(WAL_EINVAL, "grid must be >= 1 and block a multiple of 64 in [64, 1024] (got %d, %d)", grid, block);
  if ((int64_t)grid * block * 64 > ((int64_t)1 << 31))
    return fail(WAL_EINVAL, "grid * block must be at most 2^25 (32-bit offsets, four strides per trip)");
  hipLaunchKernelGGL(read_probe_kernel, dim3((unsigned)grid), dim3((unsigned)block), 0,
                     reinterpret_cast<hipStream_t>(stream), src, (uint32_t)bytes, partial);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? WAL_OK : hip_fail(e, "read_probe_kernel");
}

}  // extern "C"
