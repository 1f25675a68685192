// Outlier-column selection of the compressor (replaces compressor.py:158-215,
// _isolate_hdsq_outliers) on the GPU, in two kernels:
//
// 1. colsumsq_kernel: per column, the fp32 sum of squares over the rows in 4096-row chunks
//    (each chunk summed, chunks added in order, as the reference accumulates, :173-178);
//    within a chunk four row-interleaved partial sums meet in a fixed order, so the result
//    is deterministic.
// 2. select_kernel (one workgroup): saliency = sqrt(sumsq) (times |gamma| when a norm vector
//    is given, :183-187), fp32 mean / variance + 1e-8 / fourth moment, kurtosis clamped
//    to >= 1, the kurtosis-adaptive ratio (1 + 0.15 log1p(excess)) * base rounded to fp32
//    and clamped to [0.005, 0.03] in fp32, n_out = max(1, round-half-even(K * ratio))
//    (:189-201); then the n_out largest saliencies by a 4-pass 8-bit radix select on the
//    fp32 bit patterns (non-negative, so they order like unsigned integers), ties at the
//    threshold taken lowest column first, written in ascending column order by a
//    compaction (the reference sorts topk's indices, :202-203).
#include <cmath>

#include "common.h"

namespace spectra {

constexpr int kColThreads = 256;   // 64 columns x 4 row phases
constexpr int kSelThreads = 1024;
constexpr int kSelMaxK = 32768;

__global__ void __launch_bounds__(kColThreads) colsumsq_kernel(const void* __restrict__ w, int64_t ldw, int dt,
                                                                int64_t n, int64_t k, float* __restrict__ sumsq) {
  __shared__ float part[4][64];
  const int c = threadIdx.x & 63, ph = threadIdx.x >> 6;
  const int64_t col = (int64_t)blockIdx.x * 64 + c;
  const bool ok = col < k;
  float total = 0.0f;
  for (int64_t r0 = 0; r0 < n; r0 += 4096) {  // compressor.py:173-178: 4096-row chunks
    const int64_t r1 = r0 + 4096 < n ? r0 + 4096 : n;
    float acc = 0.0f;
    if (ok)
      for (int64_t r = r0 + ph; r < r1; r += 4) {
        const float v = load_elem(w, r * ldw + col, dt);
        acc = __builtin_fmaf(v, v, acc);
      }
    part[ph][c] = acc;
    __syncthreads();
    if (ph == 0) total += (part[0][c] + part[1][c]) + (part[2][c] + part[3][c]);
    __syncthreads();
  }
  if (ph == 0 && ok) sumsq[col] = total;
}

__device__ __forceinline__ float block_sum(float v, float* red) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  const int wv = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[wv] = v;
  __syncthreads();
  float t = 0.0f;
  for (int i = 0; i < kSelThreads / 64; ++i) t += red[i];  // fixed order
  return t;
}

__global__ void __launch_bounds__(kSelThreads) select_kernel(const float* __restrict__ sumsq,
                                                              const float* __restrict__ norm, int k,
                                                              double base_ratio, int adaptive,
                                                              int32_t* __restrict__ idx, int32_t* __restrict__ n_out,
                                                              float* __restrict__ stats) {
  extern __shared__ float sal[];  // [k]
  __shared__ float red[kSelThreads / 64];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t sh_prefix, sh_remaining;
  __shared__ uint32_t scan_gt[kSelThreads], scan_eq[kSelThreads];
  const int tid = threadIdx.x;
  float s = 0.0f;
  for (int i = tid; i < k; i += kSelThreads) {
    float v = sqrtf(sumsq[i]);
    if (norm != nullptr) v = norm[i] * v;  // compressor.py:183-184
    sal[i] = v;
    s += v;
  }
  const float mu = block_sum(s, red) / (float)k;
  float s2 = 0.0f, s4 = 0.0f;
  for (int i = tid; i < k; i += kSelThreads) {
    const float d = sal[i] - mu;
    const float d2 = d * d;
    s2 += d2;
    s4 += d2 * d2;
  }
  const float sigma2 = block_sum(s2, red) / (float)k + 1e-8f;  // compressor.py:189-191
  const float m4 = block_sum(s4, red) / (float)k;
  double kurt = (double)(m4 / (sigma2 * sigma2));
  kurt = kurt > 1.0 ? kurt : 1.0;
  double ratio = base_ratio;
  if (adaptive) {  // compressor.py:193-197
    const double excess = kurt - 3.0 > 0.0 ? kurt - 3.0 : 0.0;
    const double kmult = 1.0 + 0.15 * log1p(excess);
    float r32 = (float)(base_ratio * kmult);
    r32 = r32 < 0.005f ? 0.005f : (r32 > 0.03f ? 0.03f : r32);
    ratio = (double)r32;
  }
  int want = (int)rint((double)k * ratio);  // round half to even, as Python's round()
  want = want < 1 ? 1 : (want > k ? k : want);

  // radix select: the key of the want-th largest saliency
  uint32_t prefix = 0, mask = 0, remaining = (uint32_t)want;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int b = tid; b < 256; b += kSelThreads) hist[b] = 0;
    __syncthreads();
    for (int i = tid; i < k; i += kSelThreads) {
      const uint32_t key = __builtin_bit_cast(uint32_t, sal[i]);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t cum = 0;
      int b = 255;
      for (; b > 0; --b) {
        if (cum + hist[b] >= remaining) break;
        cum += hist[b];
      }
      sh_prefix = prefix | ((uint32_t)b << shift);
      sh_remaining = remaining - cum;
    }
    __syncthreads();
    prefix = sh_prefix;
    remaining = sh_remaining;
    mask |= 255u << shift;
  }
  // compaction in column order: every key above the threshold, and the first `remaining`
  // columns whose key equals it
  const int per = (k + kSelThreads - 1) / kSelThreads;
  const int lo = tid * per, hi = min(lo + per, k);
  uint32_t ngt = 0, neq = 0;
  for (int i = lo; i < hi; ++i) {
    const uint32_t key = __builtin_bit_cast(uint32_t, sal[i]);
    ngt += key > prefix;
    neq += key == prefix;
  }
  scan_gt[tid] = ngt;
  scan_eq[tid] = neq;
  __syncthreads();
  for (int off = 1; off < kSelThreads; off <<= 1) {  // inclusive scans
    const uint32_t a = tid >= off ? scan_gt[tid - off] : 0u, b = tid >= off ? scan_eq[tid - off] : 0u;
    __syncthreads();
    scan_gt[tid] += a;
    scan_eq[tid] += b;
    __syncthreads();
  }
  uint32_t gt_before = scan_gt[tid] - ngt, eq_before = scan_eq[tid] - neq;
  for (int i = lo; i < hi; ++i) {
    const uint32_t key = __builtin_bit_cast(uint32_t, sal[i]);
    const bool take_eq = key == prefix && eq_before < remaining;
    if (key > prefix || take_eq) {
      const uint32_t eq_taken = eq_before < remaining ? eq_before : remaining;
      idx[gt_before + eq_taken] = i;
    }
    gt_before += key > prefix;
    eq_before += key == prefix;
  }
  if (tid == 0) {
    *n_out = want;
    stats[0] = (float)ratio;
    stats[1] = (float)kurt;
  }
}

}  // namespace spectra

using namespace spectra;

extern "C" size_t spectra_outlier_columns_workspace(int64_t k) { return (size_t)(k > 0 ? k : 0) * sizeof(float); }

extern "C" int spectra_outlier_columns(const void* w, int64_t ldw, int32_t w_dtype, int64_t n, int64_t k,
                                       const float* norm_vector, double base_ratio, int32_t adaptive, int32_t* idx,
                                       int32_t* n_out, float* stats, void* workspace, size_t workspace_bytes,
                                       spectra_stream_t stream) {
  SPECTRA_REQUIRE(w && idx && n_out && stats, "NULL pointer");
  SPECTRA_REQUIRE(n > 0 && k > 0, "n and k must be positive");
  if (k > kSelMaxK) return fail(SPECTRA_ERR_UNSUPPORTED, "outlier selection serves K <= 32768");
  SPECTRA_REQUIRE(ldw >= k, "row stride smaller than k");
  SPECTRA_REQUIRE(w_dtype >= SPECTRA_F16 && w_dtype <= SPECTRA_F32, "bad dtype");
  SPECTRA_REQUIRE(base_ratio > 0.0 && base_ratio < 1.0, "base ratio must lie in (0, 1)");
  if (workspace == nullptr || workspace_bytes < spectra_outlier_columns_workspace(k))
    return fail(SPECTRA_ERR_WORKSPACE, "workspace missing or smaller than spectra_outlier_columns_workspace()");
  const hipStream_t s = (hipStream_t)stream;
  float* sumsq = (float*)workspace;
  hipLaunchKernelGGL(colsumsq_kernel, dim3((unsigned)((k + 63) / 64)), dim3(kColThreads), 0, s, w, ldw,
                     (int)w_dtype, n, k, sumsq);
  SPECTRA_HIP_CHECK(hipGetLastError());
  const int st = ensure_lds_limit((const void*)select_kernel);
  if (st != SPECTRA_OK) return st;
  hipLaunchKernelGGL(select_kernel, dim3(1), dim3(kSelThreads), (size_t)k * sizeof(float), s, sumsq, norm_vector,
                     (int)k, base_ratio, (int)adaptive, idx, n_out, stats);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}
