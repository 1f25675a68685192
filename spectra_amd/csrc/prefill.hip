// Prefill GEMM on the matrix-core library (M >= kPrefillMinM activation rows):
//   out = FWHT_b(a) / sqrt(b) . W_eff^T + bias
// the reference's batched GEMM (kernels.py:191-389, dispatched at engine.py:111-124) at
// prompt sizes, where the layer is compute-bound and the decode of the 4-bit weights is
// amortized over thousands of rows.  The reference's arithmetic, in its own compute dtype
// (fp16 or bf16, the activations' dtype: kernels.py:238-242, 347-348):
//  * W_eff dequantized once per call into the compute dtype (the bit-exact dequant of
//    spectra_w4_dequant, outliers included);
//  * the Hadamard rotation on the weights: with H_b symmetric, FWHT_b(a) / sqrt(b) . W_eff^T =
//    a . (W_eff H_b / sqrt(b))^T, so the dequant writes the rotated rows (blocks up to 512,
//    K a multiple of 512) and the GEMM reads the activations where they are (16-byte aligned,
//    row stride a multiple of 8); otherwise the activations are rotated in fp32 and rounded
//    to the compute dtype into the workspace (without a rotation they are read as given);
//  * one plain GEMM of hipBLASLt over the two (fp32 accumulation, host alpha 1 and beta 0),
//    D in the compute dtype written straight to `out`, the bias added in its epilogue.
// Per shape the heuristic's candidate algorithms are timed once (on an eager call; under
// graph capture the first candidate runs untimed) and the fastest is kept.  Calls the path
// does not serve (strided or misaligned output, a bias dtype the library's epilogue does not
// take, a workspace too small for it) return SPECTRA_ERR_UNSUPPORTED with nothing launched
// and run on the MFMA GEMM family.
#include <hipblaslt/hipblaslt.h>

#include <cmath>
#include <map>
#include <mutex>
#include <tuple>

#include "common.h"

namespace spectra {

// gemm.hip: the rotation into the compute dtype (natural order, unscaled)
int gemm_prep_rotate(const void* a, int64_t lda, int64_t m, int dt, int k, int had, uint16_t* a16, int32_t* fexp,
                     hipStream_t s);
// dequant.hip: the row dequant's operand check and its rotated rows (W_eff H_b / sqrt(b))
bool dequant_rows_ok(const spectra_qweight_t* w, const void* out, int64_t ldo, int out_dtype, int rot_had);
int w4_dequant_rotated(const spectra_qweight_t* w, void* out, int out_dtype, int had, hipStream_t s);

constexpr int64_t kPrefillMinM = 512;
constexpr size_t kPrefillLtWorkspace = size_t(32) << 20;
constexpr int kPrefillCandidates = 32;

namespace {

struct LtPlan {
  hipblasLtMatmulDesc_t md = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, ld = nullptr;
  hipblasLtMatmulHeuristicResult_t cand[kPrefillCandidates];
  int ncand = 0, best = 0;
  bool timed = false;
};

// (device, m, n, k, ldo, compute dtype, bias dtype or -1, activation row stride)
typedef std::tuple<int, int64_t, int64_t, int64_t, int64_t, int, int, int64_t> PlanKey;

std::mutex g_mu;
std::map<int, hipblasLtHandle_t> g_handles;
std::map<PlanKey, LtPlan> g_plans;

hipblasLtHandle_t handle_for(int dev) {
  auto it = g_handles.find(dev);
  if (it != g_handles.end()) return it->second;
  hipblasLtHandle_t h = nullptr;
  if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) return nullptr;
  g_handles[dev] = h;
  return h;
}

hipDataType lt_type(int dt) { return dt == SPECTRA_BF16 ? HIP_R_16BF : dt == SPECTRA_F32 ? HIP_R_32F : HIP_R_16F; }

// D (N x M column-major = out [m][ldo] row-major) = op(W) op(A) (+ bias per row of D, i.e.
// per output column), W: K x N column-major (the [N][K] rows of W_eff), op T; A: K x M
// column-major (the [M][K] rotated rows, row stride lda), op N.  Only candidates the
// heuristic marks valid and that fit the workspace are kept.
LtPlan* plan_for(hipblasLtHandle_t h, const PlanKey& key) {
  auto it = g_plans.find(key);
  if (it != g_plans.end()) return it->second.ncand > 0 ? &it->second : nullptr;
  LtPlan& pl = g_plans[key];
  const int64_t m = std::get<1>(key), n = std::get<2>(key), k = std::get<3>(key), ldo = std::get<4>(key);
  const hipDataType dt = lt_type(std::get<5>(key));
  const int bias_dt = std::get<6>(key);
  const int64_t lda = std::get<7>(key);
  bool ok = hipblasLtMatmulDescCreate(&pl.md, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  ok = ok && hipblasLtMatmulDescSetAttribute(pl.md, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatmulDescSetAttribute(pl.md, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) == HIPBLAS_STATUS_SUCCESS;
  if (ok && bias_dt >= 0) {
    const hipblasLtEpilogue_t ep = HIPBLASLT_EPILOGUE_BIAS;
    const int32_t bdt = lt_type(bias_dt);
    ok = hipblasLtMatmulDescSetAttribute(pl.md, HIPBLASLT_MATMUL_DESC_EPILOGUE, &ep, sizeof(ep)) == HIPBLAS_STATUS_SUCCESS &&
         hipblasLtMatmulDescSetAttribute(pl.md, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bdt, sizeof(bdt)) ==
             HIPBLAS_STATUS_SUCCESS;
  }
  ok = ok && hipblasLtMatrixLayoutCreate(&pl.la, dt, (uint64_t)k, (uint64_t)n, k) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&pl.lb, dt, (uint64_t)k, (uint64_t)m, lda) == HIPBLAS_STATUS_SUCCESS;
  ok = ok && hipblasLtMatrixLayoutCreate(&pl.ld, dt, (uint64_t)n, (uint64_t)m, ldo) == HIPBLAS_STATUS_SUCCESS;
  hipblasLtMatmulPreference_t pref = nullptr;
  ok = ok && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
  uint64_t wsz = kPrefillLtWorkspace;
  ok = ok && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsz, sizeof(wsz)) ==
                 HIPBLAS_STATUS_SUCCESS;
  hipblasLtMatmulHeuristicResult_t res[kPrefillCandidates];
  int got = 0;
  if (ok && hipblasLtMatmulAlgoGetHeuristic(h, pl.md, pl.la, pl.lb, pl.ld, pl.ld, pref, kPrefillCandidates, res, &got) ==
                HIPBLAS_STATUS_SUCCESS) {
    for (int i = 0; i < got && i < kPrefillCandidates; ++i)
      if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize <= kPrefillLtWorkspace) pl.cand[pl.ncand++] = res[i];
  }
  if (!ok) pl.ncand = 0;
  if (pref != nullptr) hipblasLtMatmulPreferenceDestroy(pref);
  return pl.ncand > 0 ? &pl : nullptr;
}

struct PrefillLayout {
  size_t weff, a16, fexp, ltws, total;
};

PrefillLayout prefill_layout(const spectra_qweight_t* w, int64_t m) {
  auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
  PrefillLayout L;
  size_t off = 0;
  L.weff = off; off += al((size_t)w->n * w->k * 2);
  L.a16 = off; off += al((size_t)m * w->k * 2);
  L.fexp = off; off += al((size_t)m * 4);
  L.ltws = off; off += kPrefillLtWorkspace;
  L.total = off;
  return L;
}

bool prefill_eligible(const spectra_qweight_t* w, int64_t m, int act_dtype) {
  if (m < kPrefillMinM || m >= (int64_t(1) << 31)) return false;
  if (act_dtype != SPECTRA_F16 && act_dtype != SPECTRA_BF16) return false;
  if (w->k % 8 != 0 || w->k > 32768 || w->n % 8 != 0 || w->n >= (int64_t(1) << 31)) return false;
  if (w->hadamard_block > 1024) return false;
  return true;
}

}  // namespace

// workspace of the library path (0 when it does not serve the shape)
size_t prefill_workspace(const spectra_qweight_t* w, int64_t m, int act_dtype) {
  return prefill_eligible(w, m, act_dtype) ? prefill_layout(w, m).total : 0;
}

// SPECTRA_ERR_UNSUPPORTED (nothing launched) when the library path does not serve the call
int prefill_launch(const spectra_qweight_t* w, const void* a, int64_t lda, int64_t m, int act_dtype, void* out,
                   int64_t ldo, void* workspace, size_t workspace_bytes, hipStream_t s) {
  if (!prefill_eligible(w, m, act_dtype)) return fail(SPECTRA_ERR_UNSUPPORTED, "prefill library path: shape");
  if (ldo % 8 != 0 || (reinterpret_cast<uintptr_t>(out) % 16) != 0)
    return fail(SPECTRA_ERR_UNSUPPORTED, "prefill library path: output stride / alignment");
  const PrefillLayout L = prefill_layout(w, m);
  if (workspace == nullptr || workspace_bytes < L.total)
    return fail(SPECTRA_ERR_UNSUPPORTED, "prefill library path: workspace");
  int dev = 0;
  SPECTRA_HIP_CHECK(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_mu);
  hipblasLtHandle_t h = handle_for(dev);
  if (h == nullptr) return fail(SPECTRA_ERR_UNSUPPORTED, "prefill library path: no hipBLASLt handle");
  const int bias_dt = w->bias == nullptr ? -1 : w->bias_dtype;
  // the activations are the GEMM's operand as given when there is no rotation, or when the
  // rotation goes onto the weights (the row dequant's rotated rows); otherwise the prep rotates
  // them into the workspace.  The weights take it when the activations are the larger side
  // (4 M >= N): the prep moves 4 M K bytes, the rotated rows add their transform's work to the
  // N K weights (measured at cfg4: K = 14336, N = 4096 saves 17 us; K = 4096, N = 14336 runs
  // 4-7 us slower than the prep)
  const bool x_ok = lda % 8 == 0 && (reinterpret_cast<uintptr_t>(a) % 16) == 0;
  const int had = w->hadamard_block;
  const bool rot_w = x_ok && had > 1 && 4 * m >= w->n &&
                     dequant_rows_ok(w, (const uint8_t*)workspace + L.weff, w->k, act_dtype, had);
  const bool direct_a = x_ok && (had <= 1 || rot_w);
  const PlanKey key(dev, m, w->n, w->k, ldo, act_dtype, bias_dt, direct_a ? lda : (int64_t)w->k);
  LtPlan* pl = plan_for(h, key);
  if (pl == nullptr) return fail(SPECTRA_ERR_UNSUPPORTED, "prefill library path: no algorithm for the shape");
  uint8_t* ws = (uint8_t*)workspace;
  uint16_t* weff = (uint16_t*)(ws + L.weff);
  const uint16_t* a16 = direct_a ? (const uint16_t*)a : (const uint16_t*)(ws + L.a16);
  // (1) W_eff [N][K] in the compute dtype (outliers included; rotated when rot_w), (2) the
  // rotated activations
  int st = rot_w ? w4_dequant_rotated(w, weff, act_dtype, had, s) : spectra_w4_dequant(w, weff, w->k, act_dtype, s);
  if (st != SPECTRA_OK) return st;
  if (!direct_a) {
    st = gemm_prep_rotate(a, lda, m, act_dtype, (int)w->k, w->hadamard_block, (uint16_t*)(ws + L.a16),
                          (int32_t*)(ws + L.fexp), s);
    if (st != SPECTRA_OK) return st;
  }
  // (3) the GEMM
  if (bias_dt >= 0) {
    const void* bp = w->bias;
    if (hipblasLtMatmulDescSetAttribute(pl->md, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bp, sizeof(bp)) !=
        HIPBLAS_STATUS_SUCCESS)
      return fail(SPECTRA_ERR_HIP, "hipBLASLt: bias pointer");
  }
  void* ltws = ws + L.ltws;
  const float alpha = 1.0f, beta = 0.0f;
  auto run = [&](int i) {
    return hipblasLtMatmul(h, pl->md, &alpha, weff, pl->la, a16, pl->lb, &beta, out, pl->ld, out, pl->ld,
                           &pl->cand[i].algo, ltws, kPrefillLtWorkspace, s);
  };
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  SPECTRA_HIP_CHECK(hipStreamIsCapturing(s, &cap));
  if (!pl->timed && cap == hipStreamCaptureStatusNone && pl->ncand > 1) {
    // time each candidate on this call's operands (the final run below rewrites the output)
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float best = 1e30f;
    bool ok = hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess;
    for (int i = 0; ok && i < pl->ncand; ++i) {
      if (run(i) != HIPBLAS_STATUS_SUCCESS) continue;  // (warm-up)
      ok = hipEventRecord(e0, s) == hipSuccess;
      const bool ran = ok && run(i) == HIPBLAS_STATUS_SUCCESS && run(i) == HIPBLAS_STATUS_SUCCESS;
      ok = ok && hipEventRecord(e1, s) == hipSuccess && hipEventSynchronize(e1) == hipSuccess;
      float ms = 0.0f;
      ok = ok && hipEventElapsedTime(&ms, e0, e1) == hipSuccess;
      if (ok && ran && ms < best) {
        best = ms;
        pl->best = i;
      }
    }
    if (e0 != nullptr) (void)hipEventDestroy(e0);
    if (e1 != nullptr) (void)hipEventDestroy(e1);
    if (!ok) {
      (void)hipGetLastError();
      return fail(SPECTRA_ERR_HIP, "prefill library path: timing the candidates failed");
    }
    pl->timed = true;
  }
  if (run(pl->best) != HIPBLAS_STATUS_SUCCESS) return fail(SPECTRA_ERR_HIP, "hipBLASLt matmul failed");
  return SPECTRA_OK;
}

}  // namespace spectra
