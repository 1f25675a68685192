// W_eff materialisation, bit-exact against the reference's torch dequant:
//   Format A: round_out((q - z) * s) in fp32 (tests/test_kernels.py:31-36,
//             engine.py:185-206), then outlier columns := round_out(outlier_w)
//             (tests/test_kernels.py:38-39, engine.py:209-210)
//   Format B: round_out(fp32(NF4[q]) * fp32(absmax)), then CSR positions := round_out(val)
#include "common.h"

namespace spectra {

constexpr int kDqThreads = 256;

__global__ void __launch_bounds__(kDqThreads) dequant_kernel(spectra_qweight_t w, void* __restrict__ out,
                                                              int64_t ldo, int out_dt) {
  const int64_t kb = w.k / 2;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= w.n * kb) return;
  const int64_t row = t / kb, j = t % kb;
  const uint8_t byte = w.packed[row * w.packed_stride + j];
  for (int half = 0; half < 2; ++half) {
    const int q = half ? (byte >> 4) : (byte & 15);
    const int64_t kk = nibble_k(j, half, w.marlin_layout);
    float v;
    if (w.format == SPECTRA_FMT_ASYM_G32) {
      const int64_t g = kk / 32;
      const float s = h2f(w.scales[row * w.scales_stride + g]);
      const float z = (float)w.zeros[row * w.zeros_stride + g];
      v = ((float)q - z) * s;
    } else {
      const int64_t blk = kk / w.group_size;
      v = nf4_code_f32(q) * h2f(w.scales[row * w.scales_stride + blk]);
    }
    store_elem(out, row * ldo + kk, out_dt, v);
  }
}

__global__ void __launch_bounds__(kDqThreads) scatter_columns_kernel(spectra_qweight_t w, void* __restrict__ out,
                                                                      int64_t ldo, int out_dt) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= w.n * w.num_outliers) return;
  const int64_t row = t / w.num_outliers, j = t % w.num_outliers;
  const float v = load_elem(w.outlier_w, row * w.outlier_w_stride + j, w.outlier_w_dtype);
  store_elem(out, row * ldo + w.outlier_idx[j], out_dt, v);
}

__global__ void __launch_bounds__(kDqThreads) scatter_csr_kernel(spectra_qweight_t w, void* __restrict__ out,
                                                                  int64_t ldo, int out_dt) {
  const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= w.n) return;
  for (int e = w.csr_rowptr[row]; e < w.csr_rowptr[row + 1]; ++e)
    store_elem(out, row * ldo + w.csr_col[e], out_dt, h2f(w.csr_val[e]));
}

// Embedding gather (engine.py:127-212, SpectraFusedEmbedding.forward): row ids[b] of
// W_eff, bit-identical to the same row of spectra_w4_dequant.  One workgroup per id: the
// dense values first, then (after the barrier) the row's outlier columns / CSR entries.
// Ids outside [0, N) produce a row of zeros.
__global__ void __launch_bounds__(kDqThreads) embed_kernel(spectra_qweight_t w, const int64_t* __restrict__ ids,
                                                            void* __restrict__ out, int64_t ldo, int out_dt) {
  const int64_t b = blockIdx.x;
  const int64_t id = ids[b];
  const bool ok = id >= 0 && id < w.n;
  const int64_t row = ok ? id : 0;
  const int64_t kb = w.k / 2;
  for (int64_t j = threadIdx.x; j < kb; j += blockDim.x) {
    const uint8_t byte = w.packed[row * w.packed_stride + j];
    for (int half = 0; half < 2; ++half) {
      const int q = half ? (byte >> 4) : (byte & 15);
      const int64_t kk = nibble_k(j, half, w.marlin_layout);
      float v;
      if (w.format == SPECTRA_FMT_ASYM_G32) {
        const int64_t g = kk / 32;
        v = ((float)q - (float)w.zeros[row * w.zeros_stride + g]) * h2f(w.scales[row * w.scales_stride + g]);
      } else {
        v = nf4_code_f32(q) * h2f(w.scales[row * w.scales_stride + kk / w.group_size]);
      }
      store_elem(out, b * ldo + kk, out_dt, ok ? v : 0.0f);
    }
  }
  __syncthreads();
  if (!ok) return;
  if (w.outlier_kind == SPECTRA_OUTLIERS_COLUMNS) {
    for (int j = threadIdx.x; j < w.num_outliers; j += blockDim.x)
      store_elem(out, b * ldo + w.outlier_idx[j], out_dt,
                 load_elem(w.outlier_w, row * w.outlier_w_stride + j, w.outlier_w_dtype));
  } else if (w.outlier_kind == SPECTRA_OUTLIERS_CSR) {
    for (int e = w.csr_rowptr[row] + threadIdx.x; e < w.csr_rowptr[row + 1]; e += blockDim.x)
      store_elem(out, b * ldo + w.csr_col[e], out_dt, h2f(w.csr_val[e]));
  }
}

}  // namespace spectra

using namespace spectra;

extern "C" int spectra_w4_embedding(const spectra_qweight_t* w, const int64_t* ids, int64_t n_ids, void* out,
                                    int64_t ldo, int32_t out_dtype, spectra_stream_t stream) {
  int st = validate_qweight(w);
  if (st != SPECTRA_OK) return st;
  SPECTRA_REQUIRE(ids != nullptr && out != nullptr, "ids/out is NULL");
  SPECTRA_REQUIRE(n_ids >= 0 && n_ids < (1LL << 31), "n_ids out of range");
  SPECTRA_REQUIRE(ldo >= w->k, "out row stride smaller than K");
  SPECTRA_REQUIRE(out_dtype >= SPECTRA_F16 && out_dtype <= SPECTRA_F32, "bad out dtype");
  if (n_ids == 0) return SPECTRA_OK;
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)n_ids), dim3(kDqThreads), 0, (hipStream_t)stream, *w, ids, out, ldo,
                     (int)out_dtype);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

extern "C" int spectra_w4_dequant(const spectra_qweight_t* w, void* out, int64_t ldo, int32_t out_dtype,
                                  spectra_stream_t stream) {
  int st = validate_qweight(w);
  if (st != SPECTRA_OK) return st;
  SPECTRA_REQUIRE(out != nullptr, "out is NULL");
  SPECTRA_REQUIRE(ldo >= w->k, "out row stride smaller than K");
  SPECTRA_REQUIRE(out_dtype >= SPECTRA_F16 && out_dtype <= SPECTRA_F32, "bad out dtype");
  const hipStream_t s = (hipStream_t)stream;
  const int64_t work = w->n * (w->k / 2);
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((work + kDqThreads - 1) / kDqThreads)), dim3(kDqThreads), 0, s,
                     *w, out, ldo, (int)out_dtype);
  SPECTRA_HIP_CHECK(hipGetLastError());
  if (w->outlier_kind == SPECTRA_OUTLIERS_COLUMNS) {
    const int64_t cw = w->n * w->num_outliers;
    hipLaunchKernelGGL(scatter_columns_kernel, dim3((unsigned)((cw + kDqThreads - 1) / kDqThreads)),
                       dim3(kDqThreads), 0, s, *w, out, ldo, (int)out_dtype);
    SPECTRA_HIP_CHECK(hipGetLastError());
  } else if (w->outlier_kind == SPECTRA_OUTLIERS_CSR) {
    hipLaunchKernelGGL(scatter_csr_kernel, dim3((unsigned)((w->n + kDqThreads - 1) / kDqThreads)),
                       dim3(kDqThreads), 0, s, *w, out, ldo, (int)out_dtype);
    SPECTRA_HIP_CHECK(hipGetLastError());
  }
  return SPECTRA_OK;
}
