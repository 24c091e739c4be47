// torch_ops.cpp -- the PyTorch-ROCm operator over the C ABI (libwal2026_amd_torch.so).
//
// One op per hot call, registered as torch.ops.wal2026_amd.*: the module
// forward of the reference's PackedGroupedBlockRVQLinear
// (src/runtime.py:1362-1507) reaches the kernels through it instead of
// ctypes.  The op checks its tensors with TORCH_CHECK (a failed check, or an
// error status of the library, raises RuntimeError -- the exception the
// reference's fused-kernel callers catch, src/runtime.py:1655-1661),
// allocates the output with torch's caching allocator and launches on the
// current HIP stream, so it is safe under HIP graph capture.  The layer
// descriptor (struct wal_rvq_layer with its plan and codebook image) is built
// once by the Python layer and passed as its address; it must outlive the
// call.
#include <cstdlib>

#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>
#include <torch/library.h>

#include "wal2026_amd.h"

namespace {

// Cost model of the two prefill forms (microseconds), from measurements on
// MI355X at the c4 shapes (M = 64 .. 2048, HIP events):
//  * fused kernel: rounds of workgroups x k-steps (32 columns each) of the
//    largest workgroup x the time of one k-step of the tile shape the
//    library picks: 0.84 (128 x 256 short), 1.22 (256 x 256 tall), 0.76
//    (256 x 128 wide); with the short tile's k-steps split over several
//    workgroups (wal_rvq_linear_ws), plus the pass that adds the fp32
//    partials (read at 3 TB/s).  Without the split, few weight-row tiles
//    leave most CUs idle (a 4096-row layer is 16 short tiles per 128 x
//    rows): down_proj at M = 64 took 249 us fused, 64 us in two passes.
//  * two passes: the dense weight written at 4.5 TB/s, then torch's GEMM,
//    which took the weight's read at 4.0 TB/s plus its flops at 1.6 PFLOP/s
//    times the share of CUs its 128 x 128 output tiles fill (fitted over
//    M = 64 .. 2048 at the c4 shapes, within 20 %), plus 5 us of launches.
//    At small M the GEMM streams the weight: fused gate_up (29 MB of indices
//    instead of 235 MB of weight) wins up to M = 512.
double fused_prefill_us(const wal_rvq_layer* L, int64_t m, const wal_rvq_launch_info& info, int n_cu) {
  const double step_us = info.tile_shape == WAL_TILE_TALL ? 1.22 : (info.tile_shape == WAL_TILE_WIDE ? 0.76 : 0.84);
  const int64_t rounds = ((int64_t)info.grid + n_cu - 1) / n_cu;
  double us = (double)rounds * (double)info.share * step_us;
  if (info.k_splits > 1)
    us += ((double)info.k_splits * m * L->out_features * 4.0 + (double)m * L->out_features * 2.0) / 3.0e6 + 2.0;
  return us;
}

double two_pass_us(const wal_rvq_layer* L, int64_t m, int n_cu) {
  const double wbytes = 2.0 * (double)L->out_features * (double)L->in_features;
  const double flops = 2.0 * (double)m * (double)L->out_features * (double)L->in_features;
  const double tiles = (double)((m + 127) / 128) * (double)((L->out_features + 127) / 128);
  const double fill = tiles < n_cu ? tiles / n_cu : 1.0;
  return wbytes / 4.5e6 + wbytes / 4.0e6 + flops / (1.6e9 * fill) + 5.0;
}

int device_cu_count() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      n < 1)
    n = 256;
  return n;
}

int dtype_tag(at::ScalarType t) {
  switch (t) {
    case at::kHalf: return WAL_F16;
    case at::kBFloat16: return WAL_BF16;
    case at::kFloat: return WAL_F32;
    default: return -1;
  }
}

// Whether a prefill call (the library routes it to the fused MFMA kernel)
// runs as two passes instead: the dense weight, bit for bit the reference's
// reconstruct_weight / reconstruct_weight_fast (wal_rvq_reconstruct, written
// at HBM speed), then the library's bf16/fp16 GEMM with the bias in its
// epilogue -- the reference's own per_group order of work
// (src/runtime.py:1501-1507), on the GPU, whenever the cost model above
// says it is the faster form (c4, M = 2048: 0.7-0.8 of the fused kernel's
// time, since torch's GEMM on the natural weight layout runs at about half
// the bf16 peak and writing and re-reading the weight costs less than the
// fused kernel loses to its dequantisation).  WAL2026_PREFILL_TWO_PASS=0
// keeps the fused kernel, and so does a forced tile shape
// (WAL2026_PREFILL_TILE); WAL2026_PREFILL_TWO_PASS=1 takes the two passes
// for every eligible call.
bool prefill_two_pass(const wal_rvq_layer* L, int64_t semantics, const void* x, int64_t m, int xt, int yt) {
  if (semantics != WAL_RVQ_RECONSTRUCT && semantics != WAL_RVQ_RECONSTRUCT_FAST) return false;
  if (yt != xt || (xt != WAL_BF16 && xt != WAL_F16)) return false;
  const char* f = getenv("WAL2026_PREFILL_TWO_PASS");
  if (f != nullptr && f[0] == '0') return false;
  const char* t = getenv("WAL2026_PREFILL_TILE");
  if (t != nullptr && t[0] != 0) return false;
  wal_rvq_launch_info info;
  if (wal_rvq_linear_info(L, (int)semantics, x, m, xt, &info) != WAL_OK || info.kernel != WAL_KERNEL_PREFILL)
    return false;
  if (f != nullptr && f[0] == '1') return true;
  const int n_cu = device_cu_count();
  return two_pass_us(L, m, n_cu) < fused_prefill_us(L, m, info, n_cu);
}

const wal_rvq_layer* checked_layer(const at::Tensor& x, int64_t layer) {
  const wal_rvq_layer* L = reinterpret_cast<const wal_rvq_layer*>(layer);
  TORCH_CHECK(L != nullptr, "wal2026_amd: null layer descriptor");
  TORCH_CHECK(x.is_cuda(), "wal2026_amd: x must be on a ROCm device (got ", x.device(), ")");
  TORCH_CHECK(x.dim() >= 1 && x.size(-1) == L->in_features, "wal2026_amd: x has ", x.size(-1),
              " features, the layer ", L->in_features);
  TORCH_CHECK(dtype_tag(x.scalar_type()) >= 0, "wal2026_amd: unsupported activation dtype ", x.scalar_type());
  return L;
}

// y[..., out_features] = x[..., in_features] W^T (+ bias) into y (contiguous,
// on x's device): wal_rvq_linear_ws on the current stream, or the dense weight
// and torch's GEMM where that form is faster (prefill_two_pass).
void linear_into(const wal_rvq_layer* L, const at::Tensor& x, int64_t semantics, int64_t stage_mask,
                 const c10::optional<at::Tensor>& bias, at::Tensor& y) {
  const int xt = dtype_tag(x.scalar_type());
  const at::ScalarType yt = y.scalar_type();
  at::Tensor xc = x.contiguous();
  if (reinterpret_cast<uintptr_t>(xc.data_ptr()) % 16 != 0) xc = xc.clone();  // the fused kernels load 16 B
  const int64_t m = x.numel() / L->in_features;
  if (m == 0) return;
  const void* b = nullptr;
  int bt = WAL_F32;
  at::Tensor bc;
  if (bias.has_value() && bias->defined()) {
    bc = bias->contiguous();
    TORCH_CHECK(bc.is_cuda() && bc.device() == x.device(), "wal2026_amd: bias must be on the device of x");
    TORCH_CHECK(bc.numel() == L->out_features, "wal2026_amd: bias has ", bc.numel(), " entries for ",
                L->out_features, " outputs");
    bt = dtype_tag(bc.scalar_type());
    TORCH_CHECK(bt >= 0, "wal2026_amd: unsupported bias dtype ", bc.scalar_type());
    b = bc.data_ptr();
  }
  hipStream_t st = c10::hip::getCurrentHIPStream(x.device().index()).stream();
  if (prefill_two_pass(L, semantics, xc.data_ptr(), m, xt, dtype_tag(yt))) {
    at::Tensor w = at::empty({L->out_features, L->in_features}, x.options());
    const int rc = wal_rvq_reconstruct(L, (int)semantics, (uint32_t)stage_mask, w.data_ptr(), xt, st);
    TORCH_CHECK(rc == WAL_OK, "wal2026_amd error ", rc, ": ", wal_last_error());
    // the bias rounded to the x dtype, added to the fp32 accumulator before
    // the final rounding (F.linear's order, as the fused kernels do)
    c10::optional<at::Tensor> bx;
    if (bc.defined()) bx = bc.to(x.scalar_type());
    at::Tensor yv = y.view({m, L->out_features});
    at::linear_out(yv, xc.view({m, L->in_features}), w, bx);
    return;
  }
  // a prefill call may split its k-steps over more workgroups: its fp32
  // partials go to a workspace from torch's caching allocator
  size_t ws_bytes = 0;
  int rc = wal_rvq_linear_workspace_size(L, (int)semantics, xc.data_ptr(), m, xt, &ws_bytes);
  TORCH_CHECK(rc == WAL_OK, "wal2026_amd error ", rc, ": ", wal_last_error());
  at::Tensor ws;
  if (ws_bytes > 0) ws = at::empty({(int64_t)ws_bytes}, x.options().dtype(at::kByte));
  rc = wal_rvq_linear_ws(L, (int)semantics, (uint32_t)stage_mask, xc.data_ptr(), m, xt, b, bt, y.data_ptr(),
                         dtype_tag(yt), ws_bytes > 0 ? ws.data_ptr() : nullptr, ws_bytes, st);
  TORCH_CHECK(rc == WAL_OK, "wal2026_amd error ", rc, ": ", wal_last_error());
}

// The module forward's op: y allocated with torch's caching allocator, in
// out_dtype (default x's dtype).
at::Tensor rvq_linear(const at::Tensor& x, int64_t layer, int64_t semantics, int64_t stage_mask,
                      const c10::optional<at::Tensor>& bias, c10::optional<at::ScalarType> out_dtype) {
  const wal_rvq_layer* L = checked_layer(x, layer);
  const at::ScalarType yt = out_dtype.has_value() ? *out_dtype : x.scalar_type();
  TORCH_CHECK(dtype_tag(yt) >= 0, "wal2026_amd: unsupported output dtype ", yt);
  std::vector<int64_t> shape(x.sizes().begin(), x.sizes().end());
  shape.back() = L->out_features;
  at::Tensor y = at::empty(shape, x.options().dtype(yt));
  linear_into(L, x, semantics, stage_mask, bias, y);
  return y;
}

// The same into a caller's output (its dtype is the output dtype): for code
// that keeps its buffers across calls, such as a captured HIP graph.
at::Tensor& rvq_linear_out(const at::Tensor& x, int64_t layer, int64_t semantics, int64_t stage_mask,
                           const c10::optional<at::Tensor>& bias, at::Tensor& out) {
  const wal_rvq_layer* L = checked_layer(x, layer);
  TORCH_CHECK(out.is_cuda() && out.device() == x.device(), "wal2026_amd: out must be on the device of x");
  TORCH_CHECK(out.is_contiguous(), "wal2026_amd: out must be contiguous");
  TORCH_CHECK(dtype_tag(out.scalar_type()) >= 0, "wal2026_amd: unsupported output dtype ", out.scalar_type());
  std::vector<int64_t> shape(x.sizes().begin(), x.sizes().end());
  shape.back() = L->out_features;
  TORCH_CHECK(out.sizes().vec() == shape, "wal2026_amd: out has shape ", out.sizes(), ", the call needs ",
              at::IntArrayRef(shape));
  linear_into(L, x, semantics, stage_mask, bias, out);
  return out;
}

// Whether rvq_linear takes the two-pass form for m activation rows of dtype
// `dtype` (bf16 or fp16 output): the same decision, for reports and tests.
bool rvq_prefill_two_pass(int64_t layer, int64_t semantics, int64_t m, at::ScalarType dtype) {
  const wal_rvq_layer* L = reinterpret_cast<const wal_rvq_layer*>(layer);
  TORCH_CHECK(L != nullptr, "wal2026_amd: null layer descriptor");
  const int xt = dtype_tag(dtype);
  // (the launch query reads only the alignment of x: any 16-byte aligned address)
  return xt >= 0 && prefill_two_pass(L, semantics, reinterpret_cast<const void*>(uintptr_t{4096}), m, xt, xt);
}

// Tensors on the CPU are refused loudly: the library is the only compute path.
at::Tensor rvq_linear_cpu(const at::Tensor& x, int64_t, int64_t, int64_t, const c10::optional<at::Tensor>&,
                          c10::optional<at::ScalarType>) {
  TORCH_CHECK(false, "wal2026_amd: x must be on a ROCm device (got ", x.device(),
              "); the HIP library is the only compute path");
}
at::Tensor& rvq_linear_out_cpu(const at::Tensor& x, int64_t, int64_t, int64_t, const c10::optional<at::Tensor>&,
                               at::Tensor& out) {
  TORCH_CHECK(false, "wal2026_amd: x must be on a ROCm device (got ", x.device(),
              "); the HIP library is the only compute path");
  return out;
}

}  // namespace

TORCH_LIBRARY(wal2026_amd, m) {
  m.def("rvq_linear(Tensor x, int layer, int semantics, int stage_mask, Tensor? bias, ScalarType? out_dtype) -> Tensor");
  m.def("rvq_linear_out(Tensor x, int layer, int semantics, int stage_mask, Tensor? bias, Tensor(a!) out) -> Tensor(a!)");
  m.def("rvq_prefill_two_pass(int layer, int semantics, int m, ScalarType dtype) -> bool", &rvq_prefill_two_pass);
}

TORCH_LIBRARY_IMPL(wal2026_amd, CUDA, m) {
  m.impl("rvq_linear", rvq_linear);
  m.impl("rvq_linear_out", rvq_linear_out);
}
TORCH_LIBRARY_IMPL(wal2026_amd, CPU, m) {
  m.impl("rvq_linear", rvq_linear_cpu);
  m.impl("rvq_linear_out", rvq_linear_out_cpu);
}
