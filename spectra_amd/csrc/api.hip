// C-ABI glue: error state, weight-descriptor validation, module dispatch.
#include <cstdio>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "common.h"

namespace spectra {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int status, const std::string& msg) {
  g_last_error = msg;
  return status;
}

int validate_qweight(const spectra_qweight_t* w) {
  SPECTRA_REQUIRE(w != nullptr, "weight descriptor is NULL");
  SPECTRA_REQUIRE(w->n > 0 && w->k > 0, "N and K must be positive");
  SPECTRA_REQUIRE(w->n < (1LL << 31) && w->k < (1LL << 30), "N or K too large");
  SPECTRA_REQUIRE(w->packed != nullptr && w->scales != nullptr, "packed/scales pointer is NULL");
  SPECTRA_REQUIRE(w->format == SPECTRA_FMT_ASYM_G32 || w->format == SPECTRA_FMT_NF4, "unknown format");
  if (w->format == SPECTRA_FMT_ASYM_G32) {
    SPECTRA_REQUIRE(w->group_size == 32, "Format A (asymmetric INT4) requires group_size 32");
    SPECTRA_REQUIRE(w->zeros != nullptr, "Format A needs unpacked zero points");
    SPECTRA_REQUIRE(w->zeros_stride >= w->k / 32, "zeros row stride too small");
  } else {
    SPECTRA_REQUIRE(w->group_size >= 16 && is_pow2(w->group_size), "NF4 block size must be a power of two >= 16");
  }
  SPECTRA_REQUIRE(w->k % 32 == 0, "K must be a multiple of 32");
  SPECTRA_REQUIRE(w->k % w->group_size == 0, "K must be a multiple of the group/block size");
  SPECTRA_REQUIRE(w->hadamard_block == 0 || (is_pow2(w->hadamard_block) && w->hadamard_block >= 2 &&
                                             w->hadamard_block <= 1024 && w->k % w->hadamard_block == 0),
                  "hadamard_block must be 0 or a power of two in [2, 1024] dividing K");
  SPECTRA_REQUIRE(w->packed_stride >= w->k / 2, "packed row stride too small");
  SPECTRA_REQUIRE(w->scales_stride >= w->k / w->group_size, "scales row stride too small");
  SPECTRA_REQUIRE(w->outlier_kind >= SPECTRA_OUTLIERS_NONE && w->outlier_kind <= SPECTRA_OUTLIERS_CSR,
                  "unknown outlier kind");
  if (w->outlier_kind == SPECTRA_OUTLIERS_COLUMNS) {
    SPECTRA_REQUIRE(w->num_outliers > 0 && w->outlier_idx && w->outlier_w, "outlier columns need idx and w");
    SPECTRA_REQUIRE(w->outlier_w_dtype == SPECTRA_F16 || w->outlier_w_dtype == SPECTRA_BF16,
                    "outlier weights must be fp16 or bf16");
    SPECTRA_REQUIRE(w->outlier_w_stride >= w->num_outliers, "outlier_w row stride too small");
  }
  if (w->outlier_kind == SPECTRA_OUTLIERS_CSR) {
    SPECTRA_REQUIRE(w->csr_rowptr != nullptr, "CSR outliers need rowptr");
    SPECTRA_REQUIRE(w->csr_nnz >= 0 && w->csr_nnz < (1LL << 31), "bad CSR nnz");
    SPECTRA_REQUIRE(w->csr_nnz == 0 || (w->csr_col && w->csr_val), "CSR outliers need col/val");
  }
  if (w->bias)
    SPECTRA_REQUIRE(w->bias_dtype == SPECTRA_F16 || w->bias_dtype == SPECTRA_BF16 || w->bias_dtype == SPECTRA_F32,
                    "bias dtype must be fp16, bf16 or fp32");
  return SPECTRA_OK;
}

int ensure_lds_limit(const void* kernel, bool dyn_at_zero) {
  static std::mutex mu;
  static std::vector<std::pair<const void*, int>> done;
  int dev = 0;
  SPECTRA_HIP_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(mu);
  for (const auto& d : done)
    if (d.first == kernel && d.second == dev) return SPECTRA_OK;
  int max_lds = 0;
  SPECTRA_HIP_CHECK(hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
  hipFuncAttributes fa;
  SPECTRA_HIP_CHECK(hipFuncGetAttributes(&fa, kernel));
  if (dyn_at_zero && fa.sharedSizeBytes != 0)  // the kernel addresses its dynamic LDS from 0
    return fail(SPECTRA_ERR_UNSUPPORTED, "kernel was built with static LDS; its LDS layout needs none");
  const int dyn = max_lds - (int)fa.sharedSizeBytes;  // static LDS counts against the same limit
  SPECTRA_HIP_CHECK(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, dyn));
  done.emplace_back(kernel, dev);
  return SPECTRA_OK;
}

int device_cu_count() {
  static std::mutex mu;
  static std::vector<std::pair<int, int>> known;  // (device, CUs)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 256;
  }
  std::lock_guard<std::mutex> lk(mu);
  for (const auto& d : known)
    if (d.first == dev) return d.second;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
    (void)hipGetLastError();
    cus = 256;
  }
  known.emplace_back(dev, cus);
  return cus;
}

}  // namespace spectra

// gemv.hip / gemm.hip
namespace spectra {
int gemv_launch(const spectra_qweight_t* w, const void* x, int64_t ldx, int m, int act_dtype, void* out,
                int64_t ldo, hipStream_t stream, const spectra_gemv_fusion_t* fusion);
int gemv_plan_grid(const spectra_qweight_t* w, int m);
int skinny_supported(const spectra_qweight_t* w, const void* x, int64_t ldx, int64_t m);
size_t gemm_workspace_min(const spectra_qweight_t* w, int64_t m);
}

extern "C" const char* spectra_version(void) { return "spectra_hip 0.1.0 gfx950"; }

extern "C" const char* spectra_last_error(void) { return spectra::g_last_error.c_str(); }

// ---------------------------------------------------------------------------
// no-allocation variant of spectra_w4a16_linear: its workspace is this file-scope array
// ---------------------------------------------------------------------------
namespace spectra {

// Scratch of the no-allocation entry point: one copy per GPU the library runs on, held until
// the process ends.  In host code the name is only a handle: its device address on each GPU
// comes from hipGetSymbolAddress (scratch_ptr), and only that address is passed to kernels.
static __device__ __align__(256) uint8_t scratch[SPECTRA_NOALLOC_SCRATCH_BYTES];

// Device address of `scratch` on the current device, looked up once per device (with that
// device current) and kept; nullptr (and a message) when the lookup fails.
static void* scratch_ptr() {
  static std::mutex mu;
  static std::vector<std::pair<int, void*>> known;  // (device, address)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    set_error("hipGetDevice failed");
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(mu);
  for (const auto& d : known)
    if (d.first == dev) return d.second;
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || ptr == nullptr) {
    (void)hipGetLastError();
    set_error(std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
    return nullptr;
  }
  known.emplace_back(dev, ptr);
  return ptr;
}

}  // namespace spectra

extern "C" int spectra_w4a16_linear_noalloc(const spectra_qweight_t* w, const void* x, int64_t ldx, int64_t m,
                                            int32_t act_dtype, void* out, int64_t ldo, spectra_stream_t stream) {
  int st = spectra::validate_qweight(w);
  if (st != SPECTRA_OK) return st;
  SPECTRA_REQUIRE(m >= 1, "m must be >= 1");
  // the MFMA families' buffers (at m >= 512 the library path, whose workspace holds the
  // whole dequantized weight, is not taken from the scratch)
  const size_t need = m >= 2 ? spectra::gemm_workspace_min(w, m) : 0;
  if (need > (size_t)SPECTRA_NOALLOC_SCRATCH_BYTES)
    return spectra::fail(SPECTRA_ERR_WORKSPACE,
                         "this call needs " + std::to_string(need) + " bytes of workspace, more than the " +
                             std::to_string((size_t)SPECTRA_NOALLOC_SCRATCH_BYTES) +
                             "-byte scratch of spectra_w4a16_linear_noalloc; use spectra_w4a16_linear with a workspace");
  void* ws = spectra::scratch_ptr();
  if (ws == nullptr) return SPECTRA_ERR_HIP;
  return spectra_w4a16_linear(w, x, ldx, m, act_dtype, out, ldo, ws, (size_t)SPECTRA_NOALLOC_SCRATCH_BYTES, stream);
}

extern "C" int spectra_w4a16_linear(const spectra_qweight_t* w, const void* x, int64_t ldx, int64_t m,
                                    int32_t act_dtype, void* out, int64_t ldo, void* workspace,
                                    size_t workspace_bytes, spectra_stream_t stream) {
  // engine.py:94-124: single-token rows go to the GEMV family, everything else (and any
  // operand combination the GEMV family does not serve) to the GEMM family.
  // 2..4 rows: the row-owning GEMV (one workgroup per CU; K = 3072, 4096, 8192) where it
  // plans the shape.  A shape only the older multi-row GEMV kernels serve, whose plan needs
  // more than one workgroup per CU (they hold more than 128 VGPRs, so a second round of
  // workgroups runs behind the first), goes to the small-batch MFMA family, which streams
  // the weights in one round, when it serves the operands and the workspace holds its
  // buffers.
  if (m >= 2 && m <= 4 && spectra::validate_qweight(w) == SPECTRA_OK &&
      spectra::gemv_plan_grid(w, (int)m) > spectra::device_cu_count() &&
      x != nullptr && spectra::skinny_supported(w, x, ldx, m) == SPECTRA_OK && workspace != nullptr &&
      workspace_bytes >= spectra_w4a16_gemm_workspace(w, m, act_dtype))
    return spectra_w4a16_gemm(w, x, ldx, m, act_dtype, out, ldo, workspace, workspace_bytes, stream);
  if (m >= 1 && m <= 4) {
    const int st = spectra_w4a16_gemv(w, x, ldx, (int32_t)m, act_dtype, out, ldo, stream);
    if (st != SPECTRA_ERR_UNSUPPORTED) return st;
  }
  return spectra_w4a16_gemm(w, x, ldx, m, act_dtype, out, ldo, workspace, workspace_bytes, stream);
}
