// W_eff materialisation, bit-exact against the reference's torch dequant:
//   Format A: round_out((q - z) * s) in fp32 (tests/test_kernels.py:31-36,
//             engine.py:185-206), then outlier columns := round_out(outlier_w)
//             (tests/test_kernels.py:38-39, engine.py:209-210)
//   Format B: round_out(fp32(NF4[q]) * fp32(absmax)), then CSR positions := round_out(val)
#include <algorithm>
#include <cmath>

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

// f2bf without a branch (same bits: round to nearest even, NaN quieted)
__device__ __forceinline__ uint32_t f2bf_sel(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  return (u & 0x7fffffffu) > 0x7f800000u ? ((u >> 16) | 0x40u) : r;
}

// Row dequant at HBM rate (the prefill path materialises whole weights with it).  One wave per
// (row, segment of segc 32-element runs, segc <= kDqSegChunks a whole number of passes chosen by
// the host so that the grid holds about kDqWaves waves); in a pass over a block of 64 kE elements
// lane l owns the kE consecutive outputs kE l .. kE l + kE - 1 (kE = 8 for 16-bit, 4 for
// fp32 outputs), so every store instruction of the wave writes 1 KB contiguously.  In both
// nibble orders the 16 bytes of run c hold elements 32 c .. 32 c + 31 under one scale (group
// size a multiple of 32): with the marlin pairs (k, k + 16) a lane reads kE bytes and takes
// their low (first half of the run) or high nibbles, in the natural order kE / 2 bytes and
// both nibbles.  All of a segment's loads are issued before the first decode.  The NF4 codes
// come from a 16-entry LDS table.  Same values and roundings as dequant_kernel.  After the
// segment's dense stores have completed (the wave waits on its store counter; the fence keeps
// the compiler from moving stores across), the same wave stores the row's outliers that fall
// in its segment over them, so they land last.
constexpr int kDqSegChunks = 224;  // at most 7168 elements per segment
constexpr int64_t kDqWaves = 12288;  // 48 waves per CU on 256 CUs
constexpr int kDqPre = 2;            // outlier entries preloaded per lane

template <int kOut, bool kMarlin>
struct DqShape {
  static constexpr int kE = kOut == SPECTRA_F32 ? 4 : 8;   // outputs per lane per pass
  static constexpr int kPasses = kDqSegChunks * 32 / (64 * kE);
  static constexpr int kBytes = kMarlin ? kE : kE / 2;      // packed bytes per lane per pass
};

template <int kBytes>
__device__ __forceinline__ uint64_t load_bytes(const uint8_t* p) {
  if (kBytes == 8) return *(const uint64_t*)p;
  if (kBytes == 4) return *(const uint32_t*)p;
  return *(const uint16_t*)p;
}

// kOut: SPECTRA_F16, SPECTRA_BF16 or SPECTRA_F32.
// kRot (16-bit outputs, K a multiple of 512, Hadamard blocks of 2 .. 512): the rows come out
// rotated, W_eff H_b / sqrt(b) blockwise (the prefill library path's weights: with H_b
// symmetric, x_rot . W_eff^T = x . (W_eff H_b / sqrt(b))^T).  Each pass of 512 elements then
// goes through the wave's LDS slot: the dense values, the outliers that fall in the pass over
// them, back into registers, then the transform (stages 1, 2, 4 in registers, 8 .. 256 across
// the lanes of a block, as gemm_prep_kernel), the sign and 1 / sqrt(b) in one product, one
// rounding to the output dtype.  There is no outlier tail.
template <bool kAsym, int kOut, bool kMarlin, bool kRot>
__global__ void __launch_bounds__(kDqThreads) dequant_rows_kernel(spectra_qweight_t w, void* __restrict__ out,
                                                                   int64_t ldo, int out_dt, int nseg, int segc,
                                                                   int log_had, float rot_scale) {
  typedef DqShape<kOut, kMarlin> S;
  static_assert(!kRot || S::kE == 8, "the rotated rows are 16-bit outputs");
  __shared__ float code[16];
  __shared__ __align__(16) float stage[kRot ? kDqThreads / 64 : 1][kRot ? 512 : 4];
  if (threadIdx.x < 16) code[threadIdx.x] = nf4_code_f32((int)threadIdx.x);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int64_t wid = (int64_t)blockIdx.x * (kDqThreads / 64) + (threadIdx.x >> 6);
  const int64_t row = wid / nseg;
  if (row >= w.n) return;
  const int nch = (int)(w.k >> 5);
  const int c0 = (int)(wid - row * nseg) * segc;
  const int e_end = 32 * (min(nch, c0 + segc) - c0);  // elements of this segment
  const int gch = kAsym ? 1 : w.group_size >> 5;              // runs per scale group
  const uint8_t* prow = w.packed + row * w.packed_stride + 16 * (int64_t)c0;
  uint64_t qb[S::kPasses];
#pragma unroll
  for (int b = 0; b < S::kPasses; ++b) {
    const int o = 64 * S::kE * b + S::kE * lane;  // first element of the lane's outputs
    const int e0 = o & 31;
    if (o < e_end)
      qb[b] = load_bytes<S::kBytes>(prow + 16 * (o >> 5) + (kMarlin ? (e0 & 15) : (e0 >> 1)));
  }
  // the first kDqPre * 64 outlier entries of the row (column, value), loaded with the weights so
  // that the tail below only filters and stores them
  int64_t ocol[kDqPre];
  float oval[kDqPre];
  int64_t e_beg = 0, e_lim = 0;  // entries of the row (CSR: [rowptr[row], rowptr[row + 1]))
  if (w.outlier_kind == SPECTRA_OUTLIERS_CSR) {
    e_beg = w.csr_rowptr[row];
    e_lim = w.csr_rowptr[row + 1];
  } else if (w.outlier_kind == SPECTRA_OUTLIERS_COLUMNS) {
    e_lim = w.num_outliers;
  }
#pragma unroll
  for (int t = 0; t < kDqPre; ++t) {
    const int64_t e = e_beg + lane + 64 * t;
    ocol[t] = -1;
    oval[t] = 0.0f;
    if (e < e_lim) {
      if (w.outlier_kind == SPECTRA_OUTLIERS_CSR) {
        ocol[t] = w.csr_col[e];
        oval[t] = h2f(w.csr_val[e]);
      } else {
        ocol[t] = w.outlier_idx[e];
        oval[t] = load_elem(w.outlier_w, row * w.outlier_w_stride + e, w.outlier_w_dtype);
      }
    }
  }
#pragma unroll
  for (int b = 0; b < S::kPasses; ++b) {
    const int o = 64 * S::kE * b + S::kE * lane;
    if (o >= e_end) break;
    const int c = c0 + (o >> 5), e0 = o & 31;
    const float s = h2f(w.scales[row * w.scales_stride + c / gch]);
    const float z = kAsym ? (float)w.zeros[row * w.zeros_stride + c] : 0.0f;
    float v[S::kE];
#pragma unroll
    for (int i = 0; i < S::kE; ++i) {
      // nibble of output e0 + i: marlin -> byte (e0 & 15) + i, high half when e0 >= 16;
      // natural -> byte e0 / 2 + i / 2, high nibble for odd i
      const int bit = kMarlin ? 8 * i : 8 * (i >> 1);
      const uint32_t byte = (uint32_t)(qb[b] >> bit) & 0xffu;
      const uint32_t q = kMarlin ? (e0 >= 16 ? byte >> 4 : byte & 15u) : ((i & 1) ? byte >> 4 : byte & 15u);
      v[i] = kAsym ? ((float)q - z) * s : code[q] * s;
      if (kOut == SPECTRA_F16 && !kRot) {
        // the product is rounded to fp32 first, then to fp16 (the compiler would otherwise fold
        // the product and the conversion into one v_fma_mixlo_f16)
        asm volatile("" : "+v"(v[i]));
      }
    }
    if constexpr (kRot) {
      // the pass's dense values and its outliers through the wave's LDS slot (one wave:
      // in-order LDS, the wait and the memory clobber keep every read after every write)
      float* st = stage[threadIdx.x >> 6];
      const int64_t pk0 = 32 * (int64_t)c0 + 64 * S::kE * b;  // first column of the pass
      *(float4*)&st[8 * lane] = make_float4(v[0], v[1], v[2], v[3]);
      *(float4*)&st[8 * lane + 4] = make_float4(v[4], v[5], v[6], v[7]);
#pragma unroll
      for (int t = 0; t < kDqPre; ++t)
        if (ocol[t] >= pk0 && ocol[t] < pk0 + 512) st[ocol[t] - pk0] = oval[t];
      for (int64_t e = e_beg + 64 * kDqPre + lane; e < e_lim; e += 64) {  // rows with more entries
        const int64_t col = w.outlier_kind == SPECTRA_OUTLIERS_CSR ? (int64_t)w.csr_col[e] : w.outlier_idx[e];
        if (col >= pk0 && col < pk0 + 512)
          st[col - pk0] = w.outlier_kind == SPECTRA_OUTLIERS_CSR
                              ? h2f(w.csr_val[e])
                              : load_elem(w.outlier_w, row * w.outlier_w_stride + e, w.outlier_w_dtype);
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      float r[1][8];
      const float4 ra = *(const float4*)&st[8 * lane], rb = *(const float4*)&st[8 * lane + 4];
      r[0][0] = ra.x; r[0][1] = ra.y; r[0][2] = ra.z; r[0][3] = ra.w;
      r[0][4] = rb.x; r[0][5] = rb.y; r[0][6] = rb.z; r[0][7] = rb.w;
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot is rewritten by the next pass
#pragma unroll
      for (int lh = 0; lh < 3; ++lh) {
        if (lh < log_had) {
          const int h = 1 << lh;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if ((e & h) == 0) {
              const float x0 = r[0][e], x1 = r[0][e | h];
              r[0][e] = x0 + x1;
              r[0][e | h] = x0 - x1;
            }
        }
      }
      float sgn = 1.0f;
      auto side = [&](int lb) { const bool hi = (lane & lb) != 0; if (hi) sgn = -sgn; return hi ? -1.0f : 1.0f; };
      if (log_had > 3) prep_fly<1>(r, side(1), lane);
      if (log_had > 4) prep_fly<2>(r, side(2), lane);
      if (log_had > 5) prep_fly<4>(r, side(4), lane);
      if (log_had > 6) prep_fly<8>(r, side(8), lane);
      if (log_had > 7) prep_fly<16>(r, side(16), lane);
      if (log_had > 8) prep_fly<32>(r, side(32), lane);
      const float f = sgn * rot_scale;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        v[i] = r[0][i] * f;
        if (kOut == SPECTRA_F16) asm volatile("" : "+v"(v[i]));  // fp32, then fp16
      }
    }
    if (kOut == SPECTRA_F32) {
      *(float4*)((float*)out + row * ldo + 32 * (int64_t)c0 + o) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      uint32_t p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        p[i] = kOut == SPECTRA_BF16 ? f2bf_sel(v[2 * i]) | (f2bf_sel(v[2 * i + 1]) << 16)
                                    : (uint32_t)f2h(v[2 * i]) | ((uint32_t)f2h(v[2 * i + 1]) << 16);
      *(uint4*)((uint16_t*)out + row * ldo + 32 * (int64_t)c0 + o) = make_uint4(p[0], p[1], p[2], p[3]);
    }
  }
  const int64_t k0 = 32 * (int64_t)c0, k1 = k0 + e_end;
  if (!kRot && e_lim > e_beg) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int t = 0; t < kDqPre; ++t)
      if (ocol[t] >= k0 && ocol[t] < k1) store_elem(out, row * ldo + ocol[t], out_dt, oval[t]);
    for (int64_t e = e_beg + 64 * kDqPre + lane; e < e_lim; e += 64) {  // rows with more entries
      const int64_t col = w.outlier_kind == SPECTRA_OUTLIERS_CSR ? (int64_t)w.csr_col[e] : w.outlier_idx[e];
      if (col >= k0 && col < k1)
        store_elem(out, row * ldo + col, out_dt,
                   w.outlier_kind == SPECTRA_OUTLIERS_CSR
                       ? h2f(w.csr_val[e])
                       : load_elem(w.outlier_w, row * w.outlier_w_stride + e, w.outlier_w_dtype));
    }
  }
}

// Embedding gather (engine.py:127-212, SpectraFusedEmbedding.forward): row ids[b] of
// W_eff, bit-identical to the same row of spectra_w4_dequant.  One workgroup per id.  The
// row's loads are requested before its first store (a wait for a load also waits for every
// store issued before it, so a load behind a store costs a round trip of its own): the
// packed bytes (8 per thread), their scales and zero points, the CSR extent and each
// thread's first CSR entry; then the dense values; then, after the barrier, the outlier
// columns / CSR entries over them.  Ids outside [0, N) produce a row of zeros.
__global__ void __launch_bounds__(kDqThreads) embed_kernel(spectra_qweight_t w, const int64_t* __restrict__ ids,
                                                            void* __restrict__ out, int64_t ldo, int out_dt) {
  const int64_t b = blockIdx.x;
  const int64_t id = ids[b];
  const bool ok = id >= 0 && id < w.n;
  const int64_t row = ok ? id : 0;
  const int64_t kb = w.k / 2;
  const int tid = threadIdx.x;
  const bool asym = w.format == SPECTRA_FMT_ASYM_G32;
  const bool csr = ok && w.outlier_kind == SPECTRA_OUTLIERS_CSR;
  int eb = 0, ee = 0;
  if (csr) {
    eb = w.csr_rowptr[row];
    ee = w.csr_rowptr[row + 1];
  }
  const bool has_e = csr && eb + tid < ee;
  int ecol = 0;
  uint16_t eval = 0;
  if (has_e) {
    ecol = w.csr_col[eb + tid];
    eval = w.csr_val[eb + tid];
  }
  const uint8_t* prow = w.packed + row * w.packed_stride;
  const uint16_t* srow = w.scales + row * w.scales_stride;
  const uint8_t* zrow = asym ? w.zeros + row * w.zeros_stride : nullptr;
  const int gsh = __builtin_ctz((unsigned)w.group_size);  // the group size is a power of two (validated)
  const int k32 = (int)w.k;
  const bool vec = (reinterpret_cast<uintptr_t>(prow) & 7) == 0;
  for (int64_t j0 = (int64_t)tid * 8; j0 < kb; j0 += (int64_t)blockDim.x * 8) {
    uint32_t d[2];
    if (vec && j0 + 8 <= kb) {
      const uint2 v = *(const uint2*)(prow + j0);
      d[0] = v.x;
      d[1] = v.y;
    } else {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        d[u] = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (j0 + 4 * u + i < kb) d[u] |= (uint32_t)prow[j0 + 4 * u + i] << (8 * i);
      }
    }
    float sc[16], zp[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int kk = (int)nibble_k(j0 + (e >> 1), e & 1, w.marlin_layout);
      const int g = (kk < k32 ? kk : 0) >> gsh;
      sc[e] = h2f(srow[g]);
      zp[e] = asym ? (float)zrow[g] : 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      if (j0 + (e >> 1) < kb) {
        const int q = (int)((d[e >> 3] >> (4 * (e & 7))) & 15u);  // byte e / 2, nibble e & 1
        const int64_t kk = nibble_k(j0 + (e >> 1), e & 1, w.marlin_layout);
        const float v = asym ? ((float)q - zp[e]) * sc[e] : nf4_code_f32(q) * sc[e];
        store_elem(out, b * ldo + kk, out_dt, ok ? v : 0.0f);
      }
    }
  }
  __syncthreads();
  if (!ok) return;
  if (w.outlier_kind == SPECTRA_OUTLIERS_COLUMNS) {
    for (int j = tid; j < w.num_outliers; j += blockDim.x)
      store_elem(out, b * ldo + w.outlier_idx[j], out_dt,
                 load_elem(w.outlier_w, row * w.outlier_w_stride + j, w.outlier_w_dtype));
  } else if (csr) {
    if (has_e) store_elem(out, b * ldo + ecol, out_dt, h2f(eval));
    for (int e = eb + tid + (int)blockDim.x; e < ee; e += blockDim.x)
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

namespace spectra {

// whether the row kernel serves the operands: 16-byte aligned rows of whole 32-element runs
// under one scale each (rot_had > 0: the rotated rows, see kRot)
bool dequant_rows_ok(const spectra_qweight_t* w, const void* out, int64_t ldo, int out_dtype, int rot_had) {
  const int esz = out_dtype == SPECTRA_F32 ? 4 : 2;
  const bool asym = w->format == SPECTRA_FMT_ASYM_G32;
  if (!(w->k % 32 == 0 && (asym || w->group_size % 32 == 0) && (reinterpret_cast<uintptr_t>(w->packed) % 16) == 0 &&
        w->packed_stride % 16 == 0 && (reinterpret_cast<uintptr_t>(out) % 16) == 0 && (ldo * esz) % 16 == 0))
    return false;
  return rot_had == 0 || (esz == 2 && w->k % 512 == 0 && rot_had >= 2 && rot_had <= 512 && is_pow2(rot_had));
}

// the row kernel's launch; SPECTRA_ERR_UNSUPPORTED (nothing launched) where dequant_rows_ok fails
static int launch_dequant_rows(const spectra_qweight_t* w, void* out, int64_t ldo, int out_dtype, int rot_had,
                               hipStream_t s) {
  if (!dequant_rows_ok(w, out, ldo, out_dtype, rot_had)) return SPECTRA_ERR_UNSUPPORTED;
  const int esz = out_dtype == SPECTRA_F32 ? 4 : 2;
  const bool asym = w->format == SPECTRA_FMT_ASYM_G32;
  typedef const void* K;
  // [rotated][asym][out dtype][marlin]
  static const K kerns[2][2][3][2] = {
      {{{(K)dequant_rows_kernel<false, SPECTRA_F16, false, false>, (K)dequant_rows_kernel<false, SPECTRA_F16, true, false>},
        {(K)dequant_rows_kernel<false, SPECTRA_BF16, false, false>, (K)dequant_rows_kernel<false, SPECTRA_BF16, true, false>},
        {(K)dequant_rows_kernel<false, SPECTRA_F32, false, false>, (K)dequant_rows_kernel<false, SPECTRA_F32, true, false>}},
       {{(K)dequant_rows_kernel<true, SPECTRA_F16, false, false>, (K)dequant_rows_kernel<true, SPECTRA_F16, true, false>},
        {(K)dequant_rows_kernel<true, SPECTRA_BF16, false, false>, (K)dequant_rows_kernel<true, SPECTRA_BF16, true, false>},
        {(K)dequant_rows_kernel<true, SPECTRA_F32, false, false>, (K)dequant_rows_kernel<true, SPECTRA_F32, true, false>}}},
      {{{(K)dequant_rows_kernel<false, SPECTRA_F16, false, true>, (K)dequant_rows_kernel<false, SPECTRA_F16, true, true>},
        {(K)dequant_rows_kernel<false, SPECTRA_BF16, false, true>, (K)dequant_rows_kernel<false, SPECTRA_BF16, true, true>},
        {nullptr, nullptr}},
       {{(K)dequant_rows_kernel<true, SPECTRA_F16, false, true>, (K)dequant_rows_kernel<true, SPECTRA_F16, true, true>},
        {(K)dequant_rows_kernel<true, SPECTRA_BF16, false, true>, (K)dequant_rows_kernel<true, SPECTRA_BF16, true, true>},
        {nullptr, nullptr}}}};
  const int oi = out_dtype == SPECTRA_F16 ? 0 : out_dtype == SPECTRA_BF16 ? 1 : 2;
  const void* kern = kerns[rot_had > 0 ? 1 : 0][asym ? 1 : 0][oi][w->marlin_layout ? 1 : 0];
  if (kern == nullptr) return SPECTRA_ERR_UNSUPPORTED;
  spectra_qweight_t wc = *w;
  int odt = out_dtype;
  // segments of whole passes (16 runs for 16-bit outputs, 8 for fp32): enough of them for
  // about kDqWaves waves, none longer than kDqSegChunks runs
  const int64_t nch = w->k / 32, unit = esz == 4 ? 8 : 16;
  int64_t ns = std::min((nch + unit - 1) / unit, std::max<int64_t>(1, (kDqWaves + w->n - 1) / w->n));
  int64_t sc = ((nch + ns - 1) / ns + unit - 1) / unit * unit;
  sc = std::min<int64_t>(sc, kDqSegChunks);
  int nseg = (int)((nch + sc - 1) / sc), segc = (int)sc;
  int log_had = 0;
  while (rot_had > 1 && (1 << log_had) < rot_had) ++log_had;
  const float div = rot_had > 1 ? (float)std::sqrt((double)rot_had) : 1.0f;
  float rot_scale = 1.0f / div;  // the activation prep's 2^0 / sqrt(b)
  void* args[] = {(void*)&wc, (void*)&out, (void*)&ldo, (void*)&odt, (void*)&nseg, (void*)&segc,
                  (void*)&log_had, (void*)&rot_scale};
  const int64_t waves = w->n * nseg, per_block = kDqThreads / 64;
  SPECTRA_HIP_CHECK(hipLaunchKernel(kern, dim3((unsigned)((waves + per_block - 1) / per_block)), dim3(kDqThreads),
                                    args, 0, s));
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

// the prefill library path's weights: W_eff H_b / sqrt(b) rowwise in blocks of b = had, in the
// 16-bit out_dtype, row stride K; SPECTRA_ERR_UNSUPPORTED (nothing launched) when the row
// kernel does not serve the operands (then the activations are rotated instead)
int w4_dequant_rotated(const spectra_qweight_t* w, void* out, int out_dtype, int had, hipStream_t s) {
  if (out_dtype != SPECTRA_F16 && out_dtype != SPECTRA_BF16) return SPECTRA_ERR_UNSUPPORTED;
  return launch_dequant_rows(w, out, w->k, out_dtype, had, s);
}

}  // namespace spectra

extern "C" int spectra_w4_dequant(const spectra_qweight_t* w, void* out, int64_t ldo, int32_t out_dtype,
                                  spectra_stream_t stream) {
  int st = validate_qweight(w);
  if (st != SPECTRA_OK) return st;
  SPECTRA_REQUIRE(out != nullptr, "out is NULL");
  SPECTRA_REQUIRE(ldo >= w->k, "out row stride smaller than K");
  SPECTRA_REQUIRE(out_dtype >= SPECTRA_F16 && out_dtype <= SPECTRA_F32, "bad out dtype");
  const hipStream_t s = (hipStream_t)stream;
  st = launch_dequant_rows(w, out, ldo, (int)out_dtype, 0, s);
  if (st != SPECTRA_ERR_UNSUPPORTED) return st;
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
