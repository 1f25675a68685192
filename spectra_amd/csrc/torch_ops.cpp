// The quantized linear as a registered PyTorch operator (the thin PyTorch-ROCm extension
// over the C ABI): torch.ops.spectra_hip.w4a16_linear.
//
// Replaces SpectraFusedLinear.forward's kernel calls (engine.py:90-124, kernels.py:132-184
// for one row, :333-389 for more) with one dispatcher call.  It builds the library's weight
// descriptor from the module's buffers (no copy, no validation pass of its own beyond the
// shapes the output needs: spectra_w4a16_linear validates the descriptor), allocates the
// output (and, for more than one row, the GEMM workspace the library asks for) from the
// caching allocator, and launches on the current HIP stream -- no host synchronisation, so
// the call can be captured in a HIP graph.  With a schema registered, torch.compile traces
// through it (the Meta kernel gives the output's shape) instead of breaking the graph, which
// the reference's @torch.compiler.disable forces (engine.py:90).
#include <ATen/ATen.h>
#include <ATen/hip/EmptyTensor.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <algorithm>
#include <string>
#include <vector>

#include "spectra_hip.h"

namespace {

int32_t act_code(const at::Tensor& t, const char* what) {
  if (t.scalar_type() == at::kHalf) return SPECTRA_F16;
  if (t.scalar_type() == at::kBFloat16) return SPECTRA_BF16;
  if (t.scalar_type() == at::kFloat) return SPECTRA_F32;
  TORCH_CHECK(false, what, " must be float16, bfloat16 or float32, got ", t.scalar_type());
}

int64_t row_stride(const at::Tensor& t, const char* what) {
  TORCH_CHECK(t.dim() == 2 && t.stride(1) == 1, what, " must be 2-D with unit inner stride");
  return t.size(0) > 1 ? t.stride(0) : t.size(1);
}

// The storage layout of one quantized weight in one integer (one argument instead of four:
// every argument costs the Python caller of a registered operator about 0.15 us):
//   bit 0        codebook: 0 = Format A (asymmetric group-32 INT4 with zero points), 1 = NF4
//   bit 1        nibble order: 1 = Marlin interleave, 0 = even/odd
//   bits 2..13   group (Format A) or block (NF4) size
//   bits 14..25  Hadamard block applied to x (0 = none)
// spectra_amd.kernels.layout_word builds it.
struct Layout {
  int32_t format, group_size, hadamard_block, marlin;
};

Layout decode_layout(int64_t layout) {
  TORCH_CHECK(layout >= 0 && (layout >> 26) == 0, "layout word ", layout, " has bits above 25 set");
  return Layout{(layout & 1) ? SPECTRA_FMT_NF4 : SPECTRA_FMT_ASYM_G32, (int32_t)((layout >> 2) & 0xFFF),
                (int32_t)((layout >> 14) & 0xFFF), (int32_t)((layout >> 1) & 1)};
}

// the descriptor of one quantized weight.  CSR outliers when outlier_rowptr is given
// (outlier_idx / outlier_w are then col int32 / val fp16), dense outlier columns otherwise.
spectra_qweight_t describe(const at::Tensor& packed, const at::Tensor& scales, const c10::optional<at::Tensor>& zeros,
                           const c10::optional<at::Tensor>& outlier_idx, const c10::optional<at::Tensor>& outlier_w,
                           const c10::optional<at::Tensor>& outlier_rowptr, const c10::optional<at::Tensor>& bias,
                           int64_t layout) {
  spectra_qweight_t w{};
  TORCH_CHECK(packed.is_cuda() && packed.scalar_type() == at::kByte, "packed_w must be a uint8 GPU tensor");
  const Layout l = decode_layout(layout);
  w.n = packed.size(0);
  w.k = packed.size(1) * 2;
  w.format = l.format;
  w.group_size = l.group_size;
  w.hadamard_block = l.hadamard_block;
  w.marlin_layout = l.marlin;
  w.packed = static_cast<const uint8_t*>(packed.data_ptr());
  w.packed_stride = row_stride(packed, "packed_w");
  TORCH_CHECK(scales.scalar_type() == at::kHalf, "scales must be float16");
  w.scales = static_cast<const uint16_t*>(scales.data_ptr());
  w.scales_stride = row_stride(scales, "scales");
  if (zeros.has_value()) {
    w.zeros = static_cast<const uint8_t*>(zeros->data_ptr());
    w.zeros_stride = row_stride(*zeros, "zeros");
  }
  w.outlier_kind = SPECTRA_OUTLIERS_NONE;
  if (outlier_rowptr.has_value()) {
    TORCH_CHECK(outlier_idx.has_value() && outlier_w.has_value(), "CSR outliers need col and val");
    TORCH_CHECK(outlier_rowptr->scalar_type() == at::kInt && outlier_idx->scalar_type() == at::kInt &&
                    outlier_w->scalar_type() == at::kHalf,
                "CSR outliers: rowptr and col int32, val float16");
    w.outlier_kind = SPECTRA_OUTLIERS_CSR;
    w.csr_rowptr = outlier_rowptr->data_ptr<int32_t>();
    w.csr_col = outlier_idx->data_ptr<int32_t>();
    w.csr_val = static_cast<const uint16_t*>(outlier_w->data_ptr());
    w.csr_nnz = outlier_idx->numel();
  } else if (outlier_idx.has_value() && outlier_w.has_value()) {
    TORCH_CHECK(outlier_idx->scalar_type() == at::kLong, "outlier_idx must be int64");
    w.outlier_kind = SPECTRA_OUTLIERS_COLUMNS;
    w.num_outliers = (int32_t)outlier_idx->numel();
    w.outlier_idx = outlier_idx->data_ptr<int64_t>();
    w.outlier_w = outlier_w->data_ptr();
    w.outlier_w_stride = row_stride(*outlier_w, "outlier_w");
    w.outlier_w_dtype = act_code(*outlier_w, "outlier_w");
  }
  if (bias.has_value()) {
    w.bias = bias->data_ptr();
    w.bias_dtype = act_code(*bias, "bias");
  }
  return w;
}

void check_status(int st) {
  if (st == SPECTRA_OK) return;
  const char* msg = spectra_last_error();
  TORCH_CHECK(st != SPECTRA_ERR_INVALID && st != SPECTRA_ERR_WORKSPACE && st != SPECTRA_ERR_UNSUPPORTED,
              "spectra_w4a16_linear: ", msg ? msg : "invalid arguments");
  TORCH_CHECK(false, "spectra_w4a16_linear: HIP error: ", msg ? msg : "");
}

at::Tensor w4a16_linear(const at::Tensor& x, const at::Tensor& packed, const at::Tensor& scales,
                        const c10::optional<at::Tensor>& zeros, const c10::optional<at::Tensor>& outlier_idx,
                        const c10::optional<at::Tensor>& outlier_w, const c10::optional<at::Tensor>& outlier_rowptr,
                        const c10::optional<at::Tensor>& bias, int64_t layout) {
  const spectra_qweight_t w = describe(packed, scales, zeros, outlier_idx, outlier_w, outlier_rowptr, bias, layout);
  TORCH_CHECK(x.dim() >= 1 && x.size(-1) == w.k, "x has ", x.size(-1), " values per row, the weight K = ", w.k);
  TORCH_CHECK(x.device() == packed.device(), "x and the weights are on different devices");
  const c10::DeviceGuard guard(x.device());  // launches and allocations on x's GPU
  const int32_t in_dt = act_code(x, "x");
  // float32 activations are computed in float16, the reference's compute dtype
  // (kernels.py:347-348), and the result is returned in float32
  at::Tensor x2 = in_dt == SPECTRA_F32 ? x.to(at::kHalf) : x;
  if (x2.dim() != 2) x2 = x2.reshape({-1, w.k});  // a view whenever the rows allow one
  const int32_t dt = in_dt == SPECTRA_F32 ? SPECTRA_F16 : in_dt;
  // the kernels read rows with 16-byte loads: unit inner stride, 16-byte aligned base and rows
  if (x2.stride(1) != 1 || (x2.size(0) > 1 && x2.stride(0) < w.k) ||
      reinterpret_cast<uintptr_t>(x2.data_ptr()) % 16 != 0 || (row_stride(x2, "x") * 2) % 16 != 0)
    x2 = x2.clone(at::MemoryFormat::Contiguous);  // a fresh block from the caching allocator
  const int64_t m = x2.size(0);
  // [m, n] straight from the caching allocator (no dispatcher round trip on the per-call path)
  at::Tensor out = at::detail::empty_cuda({m, w.n}, x2.scalar_type(), x2.device(), c10::nullopt);
  if (m > 0) {
    const hipStream_t stream = c10::hip::getCurrentHIPStream(x.device().index()).stream();
    const int64_t ldx = row_stride(x2, "x");
    // one row runs without a workspace (the GEMV family) unless the library asks for one
    // (operand combinations the GEMV family does not serve run on the GEMM family)
    int st = SPECTRA_ERR_WORKSPACE;
    if (m == 1) st = spectra_w4a16_linear(&w, x2.data_ptr(), ldx, m, dt, out.data_ptr(), w.n, nullptr, 0, stream);
    if (st == SPECTRA_ERR_WORKSPACE) {
      const size_t need = spectra_w4a16_gemm_workspace(&w, m, dt);
      const at::Tensor ws = at::detail::empty_cuda({(int64_t)std::max<size_t>(need, 1)}, at::kByte, x2.device(),
                                                   c10::nullopt);
      st = spectra_w4a16_linear(&w, x2.data_ptr(), ldx, m, dt, out.data_ptr(), w.n, ws.data_ptr(), need, stream);
    }
    check_status(st);
  }
  if (x.dim() != 2) {
    std::vector<int64_t> shape(x.sizes().begin(), x.sizes().end());
    shape.back() = w.n;
    out = out.view(shape);
  }
  return in_dt == SPECTRA_F32 ? out.to(at::kFloat) : out;
}

at::Tensor w4a16_linear_meta(const at::Tensor& x, const at::Tensor& packed, const at::Tensor& scales,
                             const c10::optional<at::Tensor>&, const c10::optional<at::Tensor>&,
                             const c10::optional<at::Tensor>&, const c10::optional<at::Tensor>&,
                             const c10::optional<at::Tensor>&, int64_t layout) {
  (void)decode_layout(layout);
  std::vector<int64_t> shape(x.sizes().begin(), x.sizes().end());
  shape.back() = packed.size(0);
  return at::empty(shape, x.options());
}

}  // namespace

TORCH_LIBRARY(spectra_hip, m) {
  m.def(
      "w4a16_linear(Tensor x, Tensor packed_w, Tensor scales, Tensor? zeros, Tensor? outlier_idx, Tensor? outlier_w, "
      "Tensor? outlier_rowptr, Tensor? bias, int layout) -> Tensor");
}

TORCH_LIBRARY_IMPL(spectra_hip, CUDA, m) { m.impl("w4a16_linear", &w4a16_linear); }

TORCH_LIBRARY_IMPL(spectra_hip, Meta, m) { m.impl("w4a16_linear", &w4a16_linear_meta); }
