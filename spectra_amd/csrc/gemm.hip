// Batched / prefill GEMM family for gfx950 (replaces kernels.py:187-389):
//   out = FWHT(a) . W_eff^T + bias
//
// 1. act_prep_kernel: one workgroup per activation row rotates it (blockwise FWHT,
//    fp32, reference butterfly order), scales it by a power of two so max|a| lands in
//    [2^14, 2^15) and stores fp16 -- exact scaling, so fp16 keeps 11 significant bits
//    for fp16 and bf16 inputs alike.
// 2. gemm_kernel: 128x128 output tile per workgroup, 4 waves of 64x64, K step 64.
//    Each step the workgroup loads the fp16 activation tile into LDS and dequantizes
//    the packed weight tile into LDS: packed byte -> (code_lo, code_hi) fp16 pair via a
//    32-column LUT (lane l reads column l & 31, conflict-free), times the block scale
//    with packed fp16 math (Format A: (q - z) * s, exact for fp16 output), then the
//    outliers of the tile (CSR entries or dense outlier columns) overwrite their
//    positions.  MFMA v_mfma_f32_32x32x16_f16 accumulates in fp32; the epilogue
//    undoes the row scale, adds the bias in fp32 and rounds once.
#include <cmath>

#include "common.h"

namespace spectra {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f16v_t __attribute__((ext_vector_type(16)));
typedef _Float16 f16x2g_t __attribute__((ext_vector_type(2)));

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kPad = 8;                  // fp16 elements of row padding in LDS tiles
constexpr int kLdsRow = kBK + kPad;      // 72 fp16 = 144 bytes
constexpr int kTileBytes = kBM * kLdsRow * 2;
constexpr int kGemmThreads = 256;
constexpr int kPrepThreads = 256;
constexpr int kWin = 4;                  // outlier entries prefetched per weight row

// ---------------------------------------------------------------------------
// activation pre-pass
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(kPrepThreads) act_prep_kernel(const void* __restrict__ a, int64_t lda, int dt,
                                                                 int64_t k, int had, float div,
                                                                 uint16_t* __restrict__ a16, int32_t* __restrict__ fexp) {
  extern __shared__ float fs[];
  __shared__ float wmax[kPrepThreads / 64];
  const int64_t row = blockIdx.x;
  for (int64_t i = threadIdx.x; i < k; i += blockDim.x) fs[i] = load_elem(a, row * lda + i, dt);
  __syncthreads();
  if (had) {
    const int npairs = (int)(k >> 1);
    for (int h = 1; h < had; h <<= 1) {
      for (int p = threadIdx.x; p < npairs; p += blockDim.x) {
        const int blk = p / (had >> 1), w = p % (had >> 1);
        const int i = blk * had + (w / h) * 2 * h + (w % h);
        const float u = fs[i], v = fs[i + h];
        fs[i] = u + v;
        fs[i + h] = u - v;
      }
      __syncthreads();
    }
    for (int64_t i = threadIdx.x; i < k; i += blockDim.x) fs[i] = fs[i] / div;
    __syncthreads();
  }
  float m = 0.0f;
  for (int64_t i = threadIdx.x; i < k; i += blockDim.x) m = fmaxf(m, fabsf(fs[i]));
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
  __syncthreads();
  float mx = 0.0f;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) mx = fmaxf(mx, wmax[w]);
  const uint32_t bits = __builtin_bit_cast(uint32_t, mx);
  const int eb = (int)(bits >> 23);
  const int E = eb == 0 ? -126 : eb - 127;
  int F = bits == 0 ? 0 : 14 - E;
  F = F < -126 ? -126 : (F > 126 ? 126 : F);
  const float f = __builtin_bit_cast(float, (uint32_t)(F + 127) << 23);
  for (int64_t i = threadIdx.x; i < k; i += blockDim.x) a16[row * k + i] = f2h(fs[i] * f);
  if (threadIdx.x == 0) fexp[row] = F;
}

// ---------------------------------------------------------------------------
// MFMA GEMM
// ---------------------------------------------------------------------------
struct GemmParams {
  const uint16_t* a16;  // [M, K] fp16, row stride K
  const int32_t* fexp;  // [M]
  const uint8_t* packed;
  int64_t ldp;
  const uint16_t* scales;
  int64_t lds;
  const uint8_t* zeros;
  int64_t ldz;
  const int64_t* oidx;
  const void* ow;
  int64_t ldow;
  const int32_t* rowptr;
  const int32_t* ccol;
  const uint16_t* cval;
  const void* bias;
  void* out;
  int64_t ldo;
  int m, n, k;
  int gshift, marlin, okind, n_out, ow_dt, bias_dt, act_dt;
};

template <int FMT>
__device__ __forceinline__ uint32_t gemm_lut_entry(int v) {
  const int lo = v & 15, hi = v >> 4;
  if (FMT == SPECTRA_FMT_NF4) {
    const uint16_t a = f2h(nf4_code_f32(lo)), b = f2h(nf4_code_f32(hi));
    return (uint32_t)a | ((uint32_t)b << 16);
  }
  return (uint32_t)f2h((float)lo) | ((uint32_t)f2h((float)hi) << 16);
}

template <int FMT>
__global__ void __launch_bounds__(kGemmThreads, 2) gemm_kernel(const GemmParams p) {
  extern __shared__ __align__(16) uint8_t smem[];
  uint16_t* As = (uint16_t*)smem;                       // [kBM][kLdsRow]
  uint16_t* Ws = (uint16_t*)(smem + kTileBytes);        // [kBN][kLdsRow]
  uint8_t* lut = smem + 2 * kTileBytes;                 // 256 x 32 columns x 4 bytes
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.x * kBM, n0 = blockIdx.y * kBN;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;  // wave tile origin
  const int K = p.k;

  for (int w = tid; w < 256 * 8; w += kGemmThreads) {  // 2048 x 16-byte stores
    const int v = w >> 3, cq = w & 7;
    const uint32_t e = gemm_lut_entry<FMT>(v);
    *(uint4*)(lut + v * 128 + cq * 16) = make_uint4(e, e, e, e);
  }

  // per-thread global load assignment
  const int a_row = tid >> 1, a_half = tid & 1;        // A: 64 bytes of one row
  const int am = min(m0 + a_row, p.m - 1);
  const int w_row = tid >> 1, w_half = tid & 1;        // W: 16 packed bytes (32 k) of one row
  const int wn_g = min(n0 + w_row, p.n - 1);
  const bool w_row_ok = n0 + w_row < p.n;
  const uint32_t lanebits = (uint32_t)(lane & 31) << 2;

  // Outliers: a window of the next kWin entries (column, value) of this thread's row,
  // refilled after it is consumed so the loads fly during the MFMAs.  CSR: cursor over
  // the row's entries; dense columns: one cursor over idx shared by all rows.
  int cur = 0, cend = 0;
  if (p.okind == SPECTRA_OUTLIERS_CSR) {
    cur = p.rowptr[wn_g];
    cend = p.rowptr[wn_g + 1];
  } else if (p.okind == SPECTRA_OUTLIERS_COLUMNS) {
    cend = p.n_out;
  }
  int wc[kWin];
  uint16_t wv[kWin];
  auto fill_window = [&]() {
#pragma unroll
    for (int q = 0; q < kWin; ++q) {
      const int e = cur + q;
      const bool ok = e < cend;
      const int ei = ok ? e : 0;
      if (p.okind == SPECTRA_OUTLIERS_CSR) {
        wc[q] = ok ? p.ccol[ei] : 0x7fffffff;
        wv[q] = p.cval[ei];
      } else {
        wc[q] = ok ? (int)p.oidx[ei] : 0x7fffffff;
        wv[q] = f2h(load_elem(p.ow, (int64_t)wn_g * p.ldow + ei, p.ow_dt));
      }
    }
  };
  if (p.okind != SPECTRA_OUTLIERS_NONE) fill_window();

  uint4 ar0, ar1, ar2, ar3, wr;
  uint16_t sr;
  uint8_t zr = 0;
#define SPECTRA_GLOAD(K0)                                                                   \
  do {                                                                                      \
    const uint4* asrc_ = (const uint4*)(p.a16 + (int64_t)am * K + (K0) + a_half * 32);      \
    ar0 = asrc_[0];                                                                         \
    ar1 = asrc_[1];                                                                         \
    ar2 = asrc_[2];                                                                         \
    ar3 = asrc_[3];                                                                         \
    const int kk_ = (K0) + w_half * 32;                                                     \
    wr = *(const uint4*)(p.packed + (int64_t)wn_g * p.ldp + (kk_ >> 1));                    \
    sr = p.scales[(int64_t)wn_g * p.lds + (kk_ >> p.gshift)];                               \
    if (FMT == SPECTRA_FMT_ASYM_G32) zr = p.zeros[(int64_t)wn_g * p.ldz + (kk_ >> 5)];      \
  } while (0)

  f16v_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int nk = K / kBK;
  SPECTRA_GLOAD(0);
  for (int kt = 0; kt < nk; ++kt) {
    const int k0 = kt * kBK;
    __syncthreads();  // previous tile fully consumed (and LUT written on the first pass)
    // ---- activation tile -> LDS
    {
      uint4* dst = (uint4*)(As + a_row * kLdsRow + a_half * 32);
      dst[0] = ar0;
      dst[1] = ar1;
      dst[2] = ar2;
      dst[3] = ar3;
    }
    // ---- weight tile: LUT decode, block scale, k order -> LDS
    {
      const uint32_t bytes4[4] = {wr.x, wr.y, wr.z, wr.w};
      uint32_t e[16];
      const _Float16 sh = __builtin_bit_cast(_Float16, sr);
      f16x2g_t s2 = {sh, sh};
      f16x2g_t z2 = {(_Float16)(-(float)zr), (_Float16)(-(float)zr)};
#pragma unroll
      for (int b = 0; b < 16; ++b) {
        const uint32_t byte = (bytes4[b >> 2] >> (8 * (b & 3))) & 0xffu;
        const uint32_t code2 = *(const uint32_t*)(lut + ((byte << 7) | lanebits));
        f16x2g_t c = __builtin_bit_cast(f16x2g_t, code2);
        if (FMT == SPECTRA_FMT_ASYM_G32) c = c + z2;  // q - z, exact
        c = c * s2;                                   // one fp16 rounding
        e[b] = __builtin_bit_cast(uint32_t, c);
      }
      uint32_t d[16];
      if (p.marlin) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          d[q] = __builtin_amdgcn_perm(e[2 * q + 1], e[2 * q], 0x05040100u);      // k = 2q, 2q+1
          d[8 + q] = __builtin_amdgcn_perm(e[2 * q + 1], e[2 * q], 0x07060302u);  // k = 16 + 2q, +1
        }
      } else {
#pragma unroll
        for (int q = 0; q < 16; ++q) d[q] = e[q];
      }
      uint4* dst = (uint4*)(Ws + w_row * kLdsRow + w_half * 32);
      dst[0] = make_uint4(d[0], d[1], d[2], d[3]);
      dst[1] = make_uint4(d[4], d[5], d[6], d[7]);
      dst[2] = make_uint4(d[8], d[9], d[10], d[11]);
      dst[3] = make_uint4(d[12], d[13], d[14], d[15]);
      // outliers of this row inside this thread's 32 k (the dequant there is exactly 0):
      // entries are ascending, so the ones below k0 + kBK are a prefix of the window
      if (p.okind != SPECTRA_OUTLIERS_NONE) {
        const int klo = k0 + w_half * 32, khi = klo + 32, kend = k0 + kBK;
        int used = 0;
#pragma unroll
        for (int q = 0; q < kWin; ++q) {
          if (wc[q] < kend) {
            if (wc[q] >= klo && wc[q] < khi && w_row_ok) Ws[w_row * kLdsRow + (wc[q] - k0)] = wv[q];
            ++used;
          }
        }
        cur += used;
        if (used == kWin) {  // more than kWin entries in one tile: read the rest directly
          while (cur < cend) {
            int c;
            uint16_t v;
            if (p.okind == SPECTRA_OUTLIERS_CSR) {
              c = p.ccol[cur];
              v = p.cval[cur];
            } else {
              c = (int)p.oidx[cur];
              v = f2h(load_elem(p.ow, (int64_t)wn_g * p.ldow + cur, p.ow_dt));
            }
            if (c >= kend) break;
            if (c >= klo && c < khi && w_row_ok) Ws[w_row * kLdsRow + (c - k0)] = v;
            ++cur;
          }
        }
        if (used > 0) fill_window();
      }
    }
    __syncthreads();
    if (kt + 1 < nk) SPECTRA_GLOAD(k0 + kBK);  // next tile's global loads fly during the MFMAs
    // ---- MFMA: 4 k-steps of 16, 2x2 tiles of 32x32 per wave
#pragma unroll
    for (int ks = 0; ks < kBK; ks += 16) {
      h8_t af[2], bf[2];
      const int kof = ks + 8 * (lane >> 5);
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *(const h8_t*)(As + (wm + i * 32 + (lane & 31)) * kLdsRow + kof);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bf[j] = *(const h8_t*)(Ws + (wn + j * 32 + (lane & 31)) * kLdsRow + kof);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  }

#undef SPECTRA_GLOAD
  // ---- epilogue: C[row][col], row = 8*(r/4) + 4*(lane/32) + r%4, col = lane%32
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn + j * 32 + (lane & 31);
      if (col >= p.n) continue;
      const float bv = p.bias ? load_elem(p.bias, col, p.bias_dt) : 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (row < p.m) {
          const int F = p.fexp[row];
          const float y = acc[i][j][r] * __builtin_bit_cast(float, (uint32_t)(127 - F) << 23) + bv;
          ((uint16_t*)p.out)[(int64_t)row * p.ldo + col] = from_f32_16(y, p.act_dt);
        }
      }
    }
  }
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// skinny.hip: the small-batch MFMA family (2 <= m <= 16)
size_t skinny_workspace(const spectra_qweight_t* w, int64_t m);
int skinny_launch(const spectra_qweight_t* w, const void* x, int64_t ldx, int64_t m, int act_dtype, void* out,
                  int64_t ldo, void* workspace, size_t workspace_bytes, hipStream_t stream);

}  // namespace spectra

using namespace spectra;

extern "C" size_t spectra_w4a16_gemm_workspace(const spectra_qweight_t* w, int64_t m, int32_t act_dtype) {
  (void)act_dtype;
  if (w == nullptr || m <= 0) return 0;
  const size_t gemm = align256((size_t)m * (size_t)w->k * 2) + align256((size_t)m * 4);
  const size_t small = skinny_workspace(w, m);
  return gemm > small ? gemm : small;
}

extern "C" int spectra_w4a16_gemm(const spectra_qweight_t* w, const void* a, int64_t lda, int64_t m,
                                  int32_t act_dtype, void* out, int64_t ldo, void* workspace,
                                  size_t workspace_bytes, spectra_stream_t stream) {
  int st = validate_qweight(w);
  if (st != SPECTRA_OK) return st;
  SPECTRA_REQUIRE(a != nullptr && out != nullptr, "a/out is NULL");
  SPECTRA_REQUIRE(m >= 1 && m < (1LL << 31) / kBM, "m out of range");
  SPECTRA_REQUIRE(act_dtype == SPECTRA_F16 || act_dtype == SPECTRA_BF16, "activations must be fp16 or bf16");
  SPECTRA_REQUIRE(lda >= w->k && ldo >= w->n, "row stride too small");
  if (w->k % kBK != 0) return fail(SPECTRA_ERR_UNSUPPORTED, "the GEMM family needs K % 64 == 0");
  if (w->k > 40000) return fail(SPECTRA_ERR_UNSUPPORTED, "the GEMM family serves K <= 40000");
  if (w->format == SPECTRA_FMT_NF4 && w->group_size < 32)
    return fail(SPECTRA_ERR_UNSUPPORTED, "the GEMM family needs an NF4 block of at least 32");
  SPECTRA_REQUIRE((reinterpret_cast<uintptr_t>(w->packed) % 16) == 0 && w->packed_stride % 16 == 0,
                  "packed weights must be 16-byte aligned with a row stride multiple of 16");
  const size_t need = spectra_w4a16_gemm_workspace(w, m, act_dtype);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(SPECTRA_ERR_WORKSPACE, "workspace missing or smaller than spectra_w4a16_gemm_workspace()");
  SPECTRA_REQUIRE((reinterpret_cast<uintptr_t>(workspace) % 256) == 0, "workspace must be 256-byte aligned");
  const hipStream_t s = (hipStream_t)stream;
  if (m >= 2 && m <= 16) {  // HBM-bound small batches: the MFMA stream family when it serves the operands
    const int sst = skinny_launch(w, a, lda, m, act_dtype, out, ldo, workspace, workspace_bytes, s);
    if (sst != SPECTRA_ERR_UNSUPPORTED) return sst;
  }
  uint16_t* a16 = (uint16_t*)workspace;
  int32_t* fexp = (int32_t*)((uint8_t*)workspace + align256((size_t)m * w->k * 2));
  const int had = w->hadamard_block;
  const float div = had ? (float)std::sqrt((double)had) : 1.0f;
  const size_t prep_lds = (size_t)w->k * 4;
  int st2 = ensure_lds_limit((const void*)act_prep_kernel);
  if (st2 != SPECTRA_OK) return st2;
  hipLaunchKernelGGL(act_prep_kernel, dim3((unsigned)m), dim3(kPrepThreads), prep_lds, s, a, lda, (int)act_dtype,
                     w->k, had, div, a16, fexp);
  SPECTRA_HIP_CHECK(hipGetLastError());

  GemmParams p;
  p.a16 = a16; p.fexp = fexp;
  p.packed = w->packed; p.ldp = w->packed_stride;
  p.scales = w->scales; p.lds = w->scales_stride;
  p.zeros = w->zeros; p.ldz = w->zeros_stride;
  p.oidx = w->outlier_idx; p.ow = w->outlier_w; p.ldow = w->outlier_w_stride;
  p.rowptr = w->csr_rowptr; p.ccol = w->csr_col; p.cval = w->csr_val;
  p.bias = w->bias; p.out = out; p.ldo = ldo;
  p.m = (int)m; p.n = (int)w->n; p.k = (int)w->k;
  int gs = 0;
  while ((1 << gs) < w->group_size) ++gs;
  p.gshift = gs;
  p.marlin = w->marlin_layout ? 1 : 0;
  const bool csr = w->outlier_kind == SPECTRA_OUTLIERS_CSR && w->csr_nnz > 0;
  p.okind = csr ? SPECTRA_OUTLIERS_CSR
                : (w->outlier_kind == SPECTRA_OUTLIERS_COLUMNS ? SPECTRA_OUTLIERS_COLUMNS : SPECTRA_OUTLIERS_NONE);
  p.n_out = w->num_outliers; p.ow_dt = w->outlier_w_dtype; p.bias_dt = w->bias_dtype; p.act_dt = act_dtype;
  const size_t lds = 2 * kTileBytes + 256 * 128;
  dim3 grid((unsigned)((m + kBM - 1) / kBM), (unsigned)((w->n + kBN - 1) / kBN));
  const void* kern = w->format == SPECTRA_FMT_NF4 ? (const void*)gemm_kernel<SPECTRA_FMT_NF4>
                                                  : (const void*)gemm_kernel<SPECTRA_FMT_ASYM_G32>;
  st2 = ensure_lds_limit(kern);
  if (st2 != SPECTRA_OK) return st2;
  if (w->format == SPECTRA_FMT_NF4)
    hipLaunchKernelGGL(gemm_kernel<SPECTRA_FMT_NF4>, grid, dim3(kGemmThreads), lds, s, p);
  else
    hipLaunchKernelGGL(gemm_kernel<SPECTRA_FMT_ASYM_G32>, grid, dim3(kGemmThreads), lds, s, p);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}
