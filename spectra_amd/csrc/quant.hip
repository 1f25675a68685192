// Compressor-side kernels: blockwise FWHT, Format A (asymmetric INT4 group-32)
// quantizer and Format B (NF4 + Hadamard + CSR) quantizer.  All are bit-exact
// restatements of float32 reference arithmetic: compiled with -ffp-contract=off
// and the default correctly-rounded fp32 division, so each +,-,*,/ rounds once,
// exactly as torch's CPU float32 kernels do.
#include <cmath>

#include "common.h"

namespace spectra {

constexpr int kQThreads = 256;

// In-LDS normalised FWHT of `nblk` consecutive blocks of `b` floats starting at s.
// Stage order h = 1, 2, 4, ... and the (u+v, u-v) butterfly follow
// compressor.py:34-39; normalisation is a division by fp32(sqrt(b)) (:40-41).
__device__ void fwht_lds(float* s, int nblk, int b, float div) {
  const int npairs = nblk * (b >> 1);
  for (int h = 1; h < b; h <<= 1) {
    __syncthreads();
    for (int p = threadIdx.x; p < npairs; p += blockDim.x) {
      const int blk = p / (b >> 1), w = p % (b >> 1);
      const int i = blk * b + (w / h) * 2 * h + (w % h);
      const float u = s[i], v = s[i + h];
      s[i] = u + v;
      s[i + h] = u - v;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nblk * b; i += blockDim.x) s[i] = s[i] / div;
  __syncthreads();
}

// ---------------------------------------------------------------------------
// spectra_fwht_rows: one workgroup transforms `seg` consecutive elements of one row
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kQThreads) fwht_rows_kernel(const void* __restrict__ x, int64_t ldx, int in_dt,
                                                                void* __restrict__ out, int64_t ldo, int out_dt,
                                                                int64_t k, int b, int seg, float div) {
  extern __shared__ float fs[];
  const int64_t segs_per_row = k / seg;
  const int64_t row = blockIdx.x / segs_per_row;
  const int64_t k0 = (blockIdx.x % segs_per_row) * seg;
  for (int i = threadIdx.x; i < seg; i += blockDim.x) fs[i] = load_elem(x, row * ldx + k0 + i, in_dt);
  fwht_lds(fs, seg / b, b, div);
  for (int i = threadIdx.x; i < seg; i += blockDim.x) store_elem(out, row * ldo + k0 + i, out_dt, fs[i]);
}

// ---------------------------------------------------------------------------
// Format A quantizer (compressor.py:71-112); one thread per pair of 32-groups
// ---------------------------------------------------------------------------
struct G32Result {
  uint8_t q[32];
  float scale;
  uint8_t zero;
};

__device__ void quant_group32(const float* w, G32Result& r) {
  float wmin = w[0], wmax = w[0];
  for (int i = 1; i < 32; ++i) {
    wmin = fminf(wmin, w[i]);
    wmax = fmaxf(wmax, w[i]);
  }
  const float diff = wmax - wmin;                       // :80
  const bool is_const = diff < 1e-8f;                   // :81 (scalar rounded to fp32)
  float s = is_const ? (wmin == 0.0f ? 1.0f : fabsf(wmin)) : diff / 15.0f;  // :83
  s = fmaxf(s, 1e-8f);                                  // :84
  uint8_t z;
  if (is_const) {
    z = wmin < 0.0f ? 1 : 0;                            // :88
  } else {
    const float zr = fminf(fmaxf(rintf(-wmin / s), 0.0f), 15.0f);  // :89
    z = (uint8_t)zr;
  }
  const float neg_zs = (-(float)z) * s;                 // -zeros.float() * scales   :95
  for (int i = 0; i < 32; ++i) {
    uint8_t q;
    if (is_const) {
      q = wmin > 0.0f ? 1 : 0;                          // :94
    } else {
      q = (uint8_t)fminf(fmaxf(rintf((w[i] - neg_zs) / s), 0.0f), 15.0f);  // :95
    }
    r.q[i] = q;
  }
  r.scale = s;
  r.zero = z;
}

__global__ void __launch_bounds__(kQThreads) quant_g32_kernel(const void* __restrict__ w, int64_t ldw, int w_dt,
                                                                int64_t n, int64_t k,
                                                                const int64_t* __restrict__ oidx, int n_out,
                                                                uint8_t* __restrict__ packed,
                                                                uint16_t* __restrict__ scales,
                                                                uint8_t* __restrict__ pzeros) {
  const int64_t G = k / 32, GP = (G + 1) / 2;  // groups, group pairs (= packed zero bytes per row)
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n * GP) return;
  const int64_t row = t / GP, gp = t % GP;
  uint8_t zb = 0;
  for (int h = 0; h < 2; ++h) {
    const int64_t g = 2 * gp + h;
    if (g >= G) break;  // odd group count: high nibble stays 0 (compressor.py:106-107)
    float wv[32];
    for (int i = 0; i < 32; ++i) wv[i] = load_elem(w, row * ldw + g * 32 + i, w_dt);
    // outlier columns are zeroed before quantization (compressor.py:134-135)
    if (oidx != nullptr) {
      int lo = 0, hi = n_out;  // first idx >= g*32 (idx ascending)
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (oidx[mid] < g * 32) lo = mid + 1; else hi = mid;
      }
      for (int j = lo; j < n_out && oidx[j] < g * 32 + 32; ++j) wv[oidx[j] - g * 32] = 0.0f;
    }
    G32Result r;
    quant_group32(wv, r);
    uint8_t* prow = packed + row * (k / 2) + g * 16;
    for (int j = 0; j < 16; ++j) prow[j] = (uint8_t)(r.q[j] | (r.q[j + 16] << 4));  // :99-102
    scales[row * G + g] = f2h(r.scale);                                              // :112
    zb |= (uint8_t)(r.zero << (4 * h));                                              // :108-110
  }
  pzeros[row * GP + gp] = zb;
}

// ---------------------------------------------------------------------------
// Format B quantizer: one workgroup per row segment of `seg` elements
// ---------------------------------------------------------------------------
__device__ __forceinline__ int nf4_nearest(float r) {
  // argmin_i |C_i - r| in fp32, lowest index on ties
  int best = 0;
  float bd = fabsf(-1.0f - r);
#pragma unroll
  for (int i = 1; i < 16; ++i) {
    const float d = fabsf(nf4_code_f32(i) - r);
    if (d < bd) {
      bd = d;
      best = i;
    }
  }
  return best;
}

__global__ void __launch_bounds__(kQThreads) quant_nf4_kernel(const void* __restrict__ w, int64_t ldw, int w_dt,
                                                                int64_t k, int seg, int bs, int had, float div,
                                                                int marlin, const int32_t* __restrict__ rowptr,
                                                                const int32_t* __restrict__ ccol,
                                                                uint16_t* __restrict__ cval,
                                                                uint8_t* __restrict__ packed,
                                                                uint16_t* __restrict__ absmax) {
  extern __shared__ float fs[];
  const int64_t segs_per_row = k / seg;
  const int64_t row = blockIdx.x / segs_per_row;
  const int64_t k0 = (blockIdx.x % segs_per_row) * seg;
  for (int i = threadIdx.x; i < seg; i += blockDim.x) fs[i] = load_elem(w, row * ldw + k0 + i, w_dt);
  __syncthreads();
  if (had) fwht_lds(fs, seg / had, had, div);
  // CSR outliers inside this segment: record fp16 value, then zero the position
  if (rowptr != nullptr) {
    const int e0 = rowptr[row], e1 = rowptr[row + 1];
    for (int e = e0 + threadIdx.x; e < e1; e += blockDim.x) {
      const int64_t c = ccol[e];
      if (c >= k0 && c < k0 + seg) cval[e] = f2h(fs[c - k0]);
    }
    __syncthreads();
    for (int e = e0 + threadIdx.x; e < e1; e += blockDim.x) {
      const int64_t c = ccol[e];
      if (c >= k0 && c < k0 + seg) fs[c - k0] = 0.0f;
    }
  }
  __syncthreads();
  // one thread per block: fp16 absmax, nearest codes, packed nibbles
  const int nblk = seg / bs;
  for (int b = threadIdx.x; b < nblk; b += blockDim.x) {
    const float* v = fs + b * bs;
    float m = 0.0f;
    for (int i = 0; i < bs; ++i) m = fmaxf(m, fabsf(v[i]));
    const uint16_t a16 = f2h(m);
    const float a = h2f(a16);
    absmax[row * (k / bs) + (k0 / bs) + b] = a16;
    // a block (>= 32, a multiple of 32) owns the contiguous bytes [kb/2, kb/2 + bs/2)
    // in both nibble layouts, and both nibbles of each of those bytes
    const int64_t kb = k0 + (int64_t)b * bs;
    uint8_t* pb = packed + row * (k / 2) + kb / 2;
    for (int jj = 0; jj < bs / 2; ++jj) {
      const int64_t j = kb / 2 + jj;
      const int elo = (int)(nibble_k(j, 0, marlin) - kb), ehi = (int)(nibble_k(j, 1, marlin) - kb);
      const int qlo = nf4_nearest(a > 0.0f ? v[elo] / a : 0.0f);
      const int qhi = nf4_nearest(a > 0.0f ? v[ehi] / a : 0.0f);
      pb[jj] = (uint8_t)(qlo | (qhi << 4));
    }
  }
}

}  // namespace spectra

using namespace spectra;

static int fwht_seg(int64_t k, int b) {
  // largest segment <= 4096 elements made of whole blocks and dividing k
  int64_t seg = b;
  while (seg * 2 <= 4096 && k % (seg * 2) == 0) seg *= 2;
  return (int)seg;
}

extern "C" int spectra_fwht_rows(const void* x, int64_t ldx, int32_t in_dtype, int64_t rows, int64_t k,
                                 int32_t block, void* out, int64_t ldo, int32_t out_dtype,
                                 spectra_stream_t stream) {
  SPECTRA_REQUIRE(x && out, "NULL pointer");
  SPECTRA_REQUIRE(rows > 0 && k > 0, "rows and k must be positive");
  SPECTRA_REQUIRE(is_pow2(block) && block >= 2 && block <= 1024 && k % block == 0,
                  "block must be a power of two in [2, 1024] dividing k");
  SPECTRA_REQUIRE(in_dtype >= SPECTRA_F16 && in_dtype <= SPECTRA_F32 && out_dtype >= SPECTRA_F16 &&
                      out_dtype <= SPECTRA_F32, "bad dtype");
  SPECTRA_REQUIRE(ldx >= k && ldo >= k, "row stride smaller than k");
  const int seg = fwht_seg(k, block);
  const int64_t grid = rows * (k / seg);
  SPECTRA_REQUIRE(grid < (1LL << 31), "too many rows");
  const float div = (float)std::sqrt((double)block);
  hipLaunchKernelGGL(fwht_rows_kernel, dim3((unsigned)grid), dim3(kQThreads), seg * sizeof(float),
                     (hipStream_t)stream, x, ldx, (int)in_dtype, out, ldo, (int)out_dtype, k, (int)block, seg,
                     div);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

extern "C" int spectra_quantize_group32(const void* w, int64_t ldw, int32_t w_dtype, int64_t n, int64_t k,
                                        int32_t group_size, const int64_t* outlier_idx, int32_t n_out,
                                        uint8_t* packed, uint16_t* scales, uint8_t* packed_zeros,
                                        spectra_stream_t stream) {
  if (group_size != 32)  // compressor.py:53-54
    return fail(SPECTRA_ERR_INVALID, "SPECTRA currently requires group_size=32 (Group-32 microscales)");
  SPECTRA_REQUIRE(w && packed && scales && packed_zeros, "NULL pointer");
  SPECTRA_REQUIRE(n > 0 && k > 0 && k % 32 == 0, "k must be a positive multiple of 32");
  SPECTRA_REQUIRE(ldw >= k, "row stride smaller than k");
  SPECTRA_REQUIRE(w_dtype >= SPECTRA_F16 && w_dtype <= SPECTRA_F32, "bad dtype");
  SPECTRA_REQUIRE(outlier_idx == nullptr || n_out > 0, "n_out must be positive with outlier_idx");
  const int64_t work = n * ((k / 32 + 1) / 2);
  const int64_t grid = (work + kQThreads - 1) / kQThreads;
  SPECTRA_REQUIRE(grid < (1LL << 31), "matrix too large");
  hipLaunchKernelGGL(quant_g32_kernel, dim3((unsigned)grid), dim3(kQThreads), 0, (hipStream_t)stream, w, ldw,
                     (int)w_dtype, n, k, outlier_idx, outlier_idx ? n_out : 0, packed, scales, packed_zeros);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

extern "C" int spectra_quantize_nf4(const void* w, int64_t ldw, int32_t w_dtype, int64_t n, int64_t k,
                                    int32_t blocksize, int32_t hadamard_block, int32_t marlin_layout,
                                    const int32_t* csr_rowptr, const int32_t* csr_col, uint16_t* csr_val,
                                    uint8_t* packed, uint16_t* absmax, spectra_stream_t stream) {
  SPECTRA_REQUIRE(w && packed && absmax, "NULL pointer");
  SPECTRA_REQUIRE(n > 0 && k > 0, "n and k must be positive");
  SPECTRA_REQUIRE(is_pow2(blocksize) && blocksize >= 32 && k % blocksize == 0,
                  "blocksize must be a power of two >= 32 dividing k");
  SPECTRA_REQUIRE(hadamard_block == 0 || (is_pow2(hadamard_block) && hadamard_block >= 2 &&
                                          hadamard_block <= 1024 && k % hadamard_block == 0),
                  "hadamard_block must be 0 or a power of two in [2, 1024] dividing k");
  SPECTRA_REQUIRE(ldw >= k, "row stride smaller than k");
  SPECTRA_REQUIRE(w_dtype >= SPECTRA_F16 && w_dtype <= SPECTRA_F32, "bad dtype");
  SPECTRA_REQUIRE((csr_rowptr == nullptr) == (csr_col == nullptr) && (csr_rowptr == nullptr) == (csr_val == nullptr),
                  "CSR rowptr/col/val must be given together");
  // segment: whole rows up to 8192 elements, otherwise the largest power-of-two
  // multiple of max(blocksize, hadamard_block) dividing k
  int64_t unit = blocksize > hadamard_block ? blocksize : hadamard_block;
  int64_t seg = unit;
  while (seg * 2 <= 8192 && k % (seg * 2) == 0) seg *= 2;
  if (k <= 8192) seg = k;
  SPECTRA_REQUIRE(k % seg == 0 && seg % unit == 0, "unsupported k for the NF4 quantizer");
  const int64_t grid = n * (k / seg);
  SPECTRA_REQUIRE(grid < (1LL << 31), "matrix too large");
  const float div = hadamard_block ? (float)std::sqrt((double)hadamard_block) : 1.0f;
  hipLaunchKernelGGL(quant_nf4_kernel, dim3((unsigned)grid), dim3(kQThreads), seg * sizeof(float),
                     (hipStream_t)stream, w, ldw, (int)w_dtype, k, (int)seg, (int)blocksize, (int)hadamard_block,
                     div, (int)marlin_layout, csr_rowptr, csr_col, csr_val, packed, absmax);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}
