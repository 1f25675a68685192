// Small-batch W4A16 family on MFMA (speculative-decoding verify, M = 2..16 rows):
//   out[m, :] = FWHT(x[m, :]) . W_eff^T + bias,   Format B (NF4, blocks of 64, CSR).
//
// Replaces the reference's batched GEMM path for small M (kernels.py:191-389, which runs
// M = 4..16 through 16-row tiles of a prefill-shaped kernel).  At these M the layer is
// HBM-bound: every weight byte is read once, so the kernel streams the packed tensor
// exactly like the decode GEMV and lets the matrix cores do the M-fold multiply.
//
// 1. skinny_prep_kernel (one workgroup per activation row): blockwise FWHT in fp32 (the
//    reference's butterfly order), division by sqrt(block), a power-of-two row scale
//    (max |x| -> [2^14, 2^15)) and fp16 rounding.  It writes the rows in the order the
//    MFMA A operand consumes them (xa) and, for CSR outliers, k-major (xk).
// 2. skinny_kernel<T, CPW>: a workgroup owns T tiles of 16 weight rows and all of K; wave
//    w owns CPW 128-k chunks per round.  Lane (n, g) = (lane % 16, lane / 16) loads 16
//    packed bytes of row n per chunk (4 lanes read 64 contiguous bytes = two NF4 blocks),
//    a v_permlane32_swap pair regroups the dwords so that every v_mfma_f32_16x16x32_f16
//    draws its 32 k from one 64-block, and each packed byte becomes an fp16 code pair
//    through the lane-replicated 256-entry LUT in LDS (lane l reads bank l).  The two
//    MFMAs of a block accumulate from zero; the block's absmax scales them into the
//    running fp32 sum (exact codes, one fp32 scale per block, as W_eff defines it up to
//    the fp32 summation order).  Waves meet in LDS in a fixed order (deterministic);
//    CSR outliers are staged in LDS; each output's entries are summed in parts by
//    adjacent lanes that meet in a fixed butterfly order.
#include <cmath>

#include "common.h"

namespace spectra {

typedef _Float16 sh8_t __attribute__((ext_vector_type(8)));
typedef float sf4_t __attribute__((ext_vector_type(4)));

constexpr int kSkPrepThreads = 256;
constexpr int kSkLut = 65536;

// k (inside a 128-k chunk) of element e = 2 i + h of the 8 A/B values that lane group g
// contributes to MFMA t of the chunk.  Lane group g0 loads chunk bytes [16 g0, 16 g0 + 16);
// after the swap lane group g holds, in register slot t, dword d0 of group g0 with
//   g0 = 2 (t >> 1) + (g & 1),  d0 = 2 (g >> 1) + (t & 1),
// so slots 0-1 come from bytes [0, 32) (block 2c) and slots 2-3 from [32, 64) (block 2c+1).
__host__ __device__ __forceinline__ int sk_chunk_k(int t, int g, int e, int marlin) {
  const int g0 = 2 * (t >> 1) + (g & 1), d0 = 2 * (g >> 1) + (t & 1);
  const int b = 16 * g0 + 4 * d0 + (e >> 1), h = e & 1;
  return marlin ? 32 * (b >> 4) + (b & 15) + 16 * h : 2 * b + h;
}

// ---------------------------------------------------------------------------
// activation pre-pass
// ---------------------------------------------------------------------------
constexpr int kSkSeg = 1024;  // activation elements per prep workgroup (whole Hadamard blocks)

// grid (segments, rows): workgroup (s, m) rotates elements [s * seg, s * seg + seg) of row m.
// The row's power-of-two scale comes from a bound every segment can compute alone:
// |FWHT_b(x)_i| / sqrt(b) <= sqrt(b) max|x|, so max |x_rot| * 2^F < 2^15 (no fp16 overflow);
// fp16 keeps 11 significant bits for every value in its normal range either way.
__global__ void __launch_bounds__(kSkPrepThreads) skinny_prep_kernel(const void* __restrict__ x, int64_t ldx, int dt,
                                                                      int k, int seg, int log_had, float div,
                                                                      int mp, int marlin, int want_xk,
                                                                      uint4* __restrict__ xa, uint16_t* __restrict__ xk,
                                                                      int32_t* __restrict__ fexp) {
  extern __shared__ float fs[];
  __shared__ float wmax[kSkPrepThreads / 64];
  const int sg = blockIdx.x, m = blockIdx.y;
  const int tid = threadIdx.x;
  const int k0 = sg * seg;
  const int len = min(seg, k - k0);
  const uint16_t* row = (const uint16_t*)x + (int64_t)m * ldx;
  // row max |x| (16-byte loads; K % 128 == 0 and the host checked the alignment)
  float mx = 0.0f;
  for (int i = tid * 8; i < k; i += kSkPrepThreads * 8) {
    const uint4 v = *(const uint4*)(row + i);
    const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      mx = fmaxf(mx, fabsf(to_f32_16((uint16_t)(u[j] & 0xffffu), dt)));
      mx = fmaxf(mx, fabsf(to_f32_16((uint16_t)(u[j] >> 16), dt)));
    }
  }
  for (int i = tid; i < len; i += kSkPrepThreads) fs[i] = to_f32_16(row[k0 + i], dt);
  mx = wave_max(mx);
  if ((tid & 63) == 0) wmax[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  if (log_had > 0) {
    // compressor.py:34-39: stages h = 1, 2, 4, ...: (u, v) -> (u + v, u - v), fp32
    const int had = 1 << log_had, npairs = len >> 1;
    for (int lh = 0; lh < log_had; ++lh) {
      const int h = 1 << lh;
      for (int q = tid; q < npairs; q += kSkPrepThreads) {
        const int blk = q >> (log_had - 1), w = q & ((had >> 1) - 1);
        const int i = (blk << log_had) + ((w >> lh) << (lh + 1)) + (w & (h - 1));
        const float u = fs[i], v = fs[i + h];
        fs[i] = u + v;
        fs[i + h] = u - v;
      }
      __syncthreads();
    }
    mx = mx * div;  // sqrt(b) max|x| (x div is exact for b = 4^j; the next line keeps margin)
    mx = mx * 1.0009765625f;
  }
  const uint32_t bits = __builtin_bit_cast(uint32_t, mx);
  const int eb = (int)(bits >> 23);
  const int E = eb == 0 ? -126 : eb - 127;
  int F = bits == 0 ? 0 : 14 - E;
  F = F < -126 ? -126 : (F > 126 ? 126 : F);
  const float f = __builtin_bit_cast(float, (uint32_t)(F + 127) << 23);
  // A-operand units of this segment: (chunk c, MFMA t, lane group g) -> 8 fp16 at [c][t][g][mp][8]
  // (a wave's load of one MFMA operand is 4 x mp x 16 contiguous bytes)
  const int units = (len >> 7) * 16, c0 = k0 >> 7;
  for (int u = tid; u < units; u += kSkPrepThreads) {
    const int c = u >> 4, t = (u >> 2) & 3, g = u & 3;
    uint32_t d[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = fs[c * 128 + sk_chunk_k(t, g, 2 * i, marlin)];
      const float hi = fs[c * 128 + sk_chunk_k(t, g, 2 * i + 1, marlin)];
      // the rotated value is (sum) / sqrt(b) (compressor.py:40-41), then the exact 2^F
      const float lo_r = log_had > 0 ? lo / div : lo, hi_r = log_had > 0 ? hi / div : hi;
      d[i] = (uint32_t)f2h(lo_r * f) | ((uint32_t)f2h(hi_r * f) << 16);
    }
    xa[(int64_t)((c0 + c) * 16 + (u & 15)) * mp + m] = make_uint4(d[0], d[1], d[2], d[3]);
  }
  if (want_xk)
    for (int i = tid; i < len; i += kSkPrepThreads) {
      const float v = log_had > 0 ? fs[i] / div : fs[i];
      xk[(int64_t)(k0 + i) * mp + m] = f2h(v * f);
    }
  if (sg == 0 && tid == 0) fexp[m] = F;
}

// The same pre-pass for Hadamard blocks of at most 512: one workgroup of 256 threads per
// 2048-element segment, thread t owning elements 8 t .. 8 t + 7.  The FWHT runs on register
// bits (h = 1, 2, 4) and across the lanes of a block (h = 8 .. 256: v_fmac_f32_dpp
// butterflies, the lane's sign and 1 / sqrt(b) riding on the output scale), with no
// barrier per stage; the scaled fp16 values pass through LDS once to reach the MFMA
// operand order.  Same scale bound, layout and outputs as skinny_prep_kernel.
constexpr int kSkSegFast = 8 * kSkPrepThreads;

__global__ void __launch_bounds__(kSkPrepThreads) skinny_prep_fast_kernel(
    const void* __restrict__ x, int64_t ldx, int dt, int k, int log_had, float div, int mp, int marlin, int want_xk,
    uint4* __restrict__ xa, uint16_t* __restrict__ xk, int32_t* __restrict__ fexp) {
  __shared__ __align__(16) uint16_t xs[kSkSegFast];
  __shared__ float wmax[kSkPrepThreads / 64];
  const int sg = blockIdx.x, m = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int k0 = sg * kSkSegFast;
  const int len = min(kSkSegFast, k - k0);
  const uint16_t* row = (const uint16_t*)x + (int64_t)m * ldx;
  // this thread's 8 elements (K % 128 == 0 and the host checked the alignment)
  float v[1][8];
  {
    uint4 q = make_uint4(0u, 0u, 0u, 0u);
    if (8 * tid < len) q = *(const uint4*)(row + k0 + 8 * tid);
    const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[0][2 * e] = to_f32_16((uint16_t)(w4[e] & 0xffffu), dt);
      v[0][2 * e + 1] = to_f32_16((uint16_t)(w4[e] >> 16), dt);
    }
  }
  // row max |x| (the whole row: every segment computes the same bound)
  float mx = 0.0f;
  for (int i = tid * 8; i < k; i += kSkPrepThreads * 8) {
    const uint4 q = *(const uint4*)(row + i);
    const uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      mx = fmaxf(mx, fabsf(to_f32_16((uint16_t)(u[j] & 0xffffu), dt)));
      mx = fmaxf(mx, fabsf(to_f32_16((uint16_t)(u[j] >> 16), dt)));
    }
  }
  mx = wave_max(mx);
  if (lane == 0) wmax[tid >> 6] = mx;
  // compressor.py:34-39: stages h = 1, 2, 4 on register bits, then across lanes
#pragma unroll
  for (int lh = 0; lh < 3; ++lh) {
    if (lh < log_had) {
      const int h = 1 << lh;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if ((e & h) == 0) {
          const float x0 = v[0][e], x1 = v[0][e | h];
          v[0][e] = x0 + x1;
          v[0][e | h] = x0 - x1;
        }
    }
  }
  float sgn = 1.0f;
  auto side = [&](int lb) { const bool hi = (tid & lb) != 0; if (hi) sgn = -sgn; return hi ? -1.0f : 1.0f; };
  if (log_had > 3) prep_fly<1>(v, side(1), lane);
  if (log_had > 4) prep_fly<2>(v, side(2), lane);
  if (log_had > 5) prep_fly<4>(v, side(4), lane);
  if (log_had > 6) prep_fly<8>(v, side(8), lane);
  if (log_had > 7) prep_fly<16>(v, side(16), lane);
  if (log_had > 8) prep_fly<32>(v, side(32), lane);
  __syncthreads();
  mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  if (log_had > 0) {
    mx = mx * div;  // sqrt(b) max|x| bounds the rotated row before the division
    mx = mx * 1.0009765625f;
  }
  const uint32_t bits = __builtin_bit_cast(uint32_t, mx);
  const int eb = (int)(bits >> 23);
  const int E = eb == 0 ? -126 : eb - 127;
  int F = bits == 0 ? 0 : 14 - E;
  F = F < -126 ? -126 : (F > 126 ? 126 : F);
  const float f2 = __builtin_bit_cast(float, (uint32_t)(F + 127) << 23);
  // (sum) / sqrt(b) (compressor.py:40-41) times 2^F, in one scale with the lane's sign
  const float fo = sgn * (log_had > 0 ? f2 / div : f2);
  {
    uint32_t d[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) d[e] = (uint32_t)f2h(v[0][2 * e] * fo) | ((uint32_t)f2h(v[0][2 * e + 1] * fo) << 16);
    *(uint4*)(xs + 8 * tid) = make_uint4(d[0], d[1], d[2], d[3]);
  }
  __syncthreads();
  // A-operand units of this segment: (chunk c, MFMA t, lane group g) -> 8 fp16 at [c][t][g][mp][8]
  const int units = (len >> 7) * 16, c0 = k0 >> 7;
  for (int u = tid; u < units; u += kSkPrepThreads) {
    const int c = u >> 4, t = (u >> 2) & 3, g = u & 3;
    uint32_t d[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      d[i] = (uint32_t)xs[c * 128 + sk_chunk_k(t, g, 2 * i, marlin)] |
             ((uint32_t)xs[c * 128 + sk_chunk_k(t, g, 2 * i + 1, marlin)] << 16);
    xa[(int64_t)((c0 + c) * 16 + (u & 15)) * mp + m] = make_uint4(d[0], d[1], d[2], d[3]);
  }
  if (want_xk)
    for (int i = tid; i < len; i += kSkPrepThreads) xk[(int64_t)(k0 + i) * mp + m] = xs[i];
  if (sg == 0 && tid == 0) fexp[m] = F;
}

// ---------------------------------------------------------------------------
// MFMA stream
// ---------------------------------------------------------------------------
struct SkinnyParams {
  const uint8_t* packed;
  int64_t ldp;             // bytes
  const uint32_t* scales;  // absmax pairs (blocks 2c, 2c + 1) as dwords
  int64_t lds32;           // row stride in dwords
  const uint4* xa;
  const uint16_t* xk;
  const int32_t* fexp;
  const int32_t* rowptr;
  const int32_t* ccol;
  const uint16_t* cval;
  const void* bias;
  void* out;
  int64_t ldo;
  int m, mp, n, k, nchunks, nrounds, csr_nnz, okind, bias_dt, act_dt, ecap;
  uint32_t off_rp, off_bias, off_fx, off_xe, off_ve, off_sums, off_csum;
};

template <int T, int CPW>
__global__ void __launch_bounds__(512) skinny_kernel(const SkinnyParams p) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw = __builtin_amdgcn_readfirstlane((int)(blockDim.x >> 6));
  const int BD = nw * 64;
  const int n16 = lane & 15, g = lane >> 4;
  constexpr int R = 16 * T;
  const int r0 = blockIdx.x * R;
  const int Rw = min(R, p.n - r0);
  const bool csr = p.okind == SPECTRA_OUTLIERS_CSR;
  const int mrow = n16 & (p.mp - 1);  // A-operand row of this lane (rows >= mp repeat)
  // every argument the prologue needs, fetched in one round trip before the first load
  asm volatile("" ::"s"(p.packed), "s"(p.ldp), "s"(p.scales), "s"(p.lds32), "s"(p.xa), "s"(p.rowptr),
               "s"(p.bias), "s"(p.n), "s"(p.mp), "s"(p.nchunks), "s"(p.nrounds), "s"(p.okind), "s"(p.bias_dt),
               "s"(p.csr_nnz), "s"(p.ccol), "s"(p.cval));

  // ---- (1) loads the tail needs first (wait counts are in issue order) ----
  // lanes 0/1: the workgroup's first / end CSR row pointer (packed bytes when no CSR)
  const int rpe = *(csr ? p.rowptr + r0 + (lane == 1 ? Rw : 0) : (const int32_t*)p.packed);
  const int rp_v = *(csr ? p.rowptr + r0 + min(tid, Rw) : (const int32_t*)p.packed);
  // the activation rows' exponents (lanes m < M), stored to LDS in the tail
  const int32_t fx_reg = p.fexp[min(tid, p.m - 1)];
  uint32_t bias_raw = 0;
  if (p.bias != nullptr) {
    const int64_t bi = r0 + (tid < Rw ? tid : 0);
    if (p.bias_dt == SPECTRA_F32) bias_raw = ((const uint32_t*)p.bias)[bi];
    else bias_raw = ((const uint16_t*)p.bias)[bi];
  }

  int64_t rowoff[T];
#pragma unroll
  for (int t = 0; t < T; ++t) rowoff[t] = r0 + min(16 * t + n16, Rw - 1);

  sf4_t acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = sf4_t{0.0f, 0.0f, 0.0f, 0.0f};

  int4 ocv = {0, 0, 0, 0};
  uint2 ovv = {0, 0};
  int e0 = 0, e1 = 0;
  const uint32_t lanebits = (uint32_t)lane << 2;
  constexpr int NJ = (CPW + 3) / 4;

  // units (chunk c, tile t) of a round in consumption order u = c * T + t; the first D0
  // units' weights are issued before the LUT is built, each later one while an earlier
  // unit is decoded, so the LDS-bound decode runs under the stream instead of after it
  constexpr int U = CPW * T;
  constexpr int D0 = U < 4 ? U : (U + 1) / 2;
  for (int rd = 0; rd < p.nrounds; ++rd) {
    const int cb = (rd * nw + wave) * CPW;  // first chunk of this wave in this round
    // loads start at cbl = min(cb, nchunks - CPW) so every address is in bounds and chunk
    // c of the wave sits at a constant offset; slots below cb (only in a last, partial
    // round) belong to another wave and are masked
    const int cbl = min(cb, p.nchunks - CPW);
    // ---- (2) scales (one dword = the two block absmax of a chunk; lane group g loads
    //      chunk cb + 4 j + g of its row, redistributed per chunk with ds_bpermute),
    //      then activations, then the first weight units ----
    uint32_t scw[T][NJ];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        scw[t][j] = p.scales[rowoff[t] * p.lds32 + min(cbl + 4 * j + g, p.nchunks - 1)];
    uint4 xr[CPW][4];
    const uint4* xbase = p.xa + (int64_t)(cbl * 16 + g) * p.mp + mrow;
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
#pragma unroll
      for (int s = 0; s < 4; ++s) xr[c][s] = xbase[(c * 16 + s * 4) * p.mp];
    }
    uint4 wq[U];
    const uint8_t* wbase[T];
#pragma unroll
    for (int t = 0; t < T; ++t) wbase[t] = p.packed + rowoff[t] * p.ldp + (int64_t)cbl * 64 + 16 * g;
    auto issue = [&](int u) { wq[u] = *(const uint4*)(wbase[u % T] + (u / T) * 64); };
#pragma unroll
    for (int u = 0; u < D0; ++u) issue(u);

    if (rd == 0) {
      // ---- (3) CSR entries of this workgroup: four per thread from the 4-aligned entry
      //      below e0 (one dwordx4 of columns, one dwordx2 of values), consumed in the tail
      if (csr) {
        e0 = __builtin_amdgcn_readlane(rpe, 0);
        e1 = __builtin_amdgcn_readlane(rpe, 1);
      }
      {
        const int g4 = (e0 & ~3) + 4 * tid;
        // (arrays of fewer than 4 entries are never read this way: nothing is staged then)
        const bool big = csr && p.csr_nnz >= 4;
        const int gc = (big && g4 < e1 && g4 + 4 <= p.csr_nnz) ? g4 : 0;
        ocv = *(big ? (const int4*)(p.ccol + gc) : (const int4*)p.packed);
        ovv = *(big ? (const uint2*)(p.cval + gc) : (const uint2*)p.packed);
      }
      // ---- (4) nibble-pair LUT (from registers, no LDS reads) ----
      build_pair_lut<SPECTRA_FMT_NF4>(smem, wave, nw, lane);
      __syncthreads();  // LUT complete
    }

    // ---- (5) decode + MFMA unit by unit as the stream arrives ----
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (u + D0 < U) issue(u + D0);
      const int c = u / T, t = u % T;
      const bool cvalid = cbl + c >= cb;  // wave-uniform
      const uint4 w = wq[u];
      // lower lanes keep dwords 0-1 and take the upper lanes' 0-1; upper lanes take
      // the lower lanes' 2-3 and keep their own 2-3
      const auto sxz = __builtin_amdgcn_permlane32_swap(w.x, w.z, false, false);
      const auto syw = __builtin_amdgcn_permlane32_swap(w.y, w.w, false, false);
      const uint32_t slot[4] = {sxz[0], syw[0], sxz[1], syw[1]};
      uint32_t bv[4][4];
#pragma unroll
      for (int sl = 0; sl < 4; ++sl)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t addr = __builtin_amdgcn_perm(slot[sl], lanebits, 0x0c0c0000u | ((4u + i) << 8));
          bv[sl][i] = *(const __attribute__((address_space(3))) uint32_t*)(uintptr_t)addr;
        }
      sf4_t t0 = {0.0f, 0.0f, 0.0f, 0.0f}, t1 = {0.0f, 0.0f, 0.0f, 0.0f};
      t0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(sh8_t, xr[c][0]),
                                                  __builtin_bit_cast(sh8_t, bv[0]), t0, 0, 0, 0);
      t1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(sh8_t, xr[c][2]),
                                                  __builtin_bit_cast(sh8_t, bv[2]), t1, 0, 0, 0);
      t0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(sh8_t, xr[c][1]),
                                                  __builtin_bit_cast(sh8_t, bv[1]), t0, 0, 0, 0);
      t1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(sh8_t, xr[c][3]),
                                                  __builtin_bit_cast(sh8_t, bv[3]), t1, 0, 0, 0);
      const uint32_t sd = (uint32_t)__builtin_amdgcn_ds_bpermute((n16 + 16 * (c & 3)) << 2, (int)scw[t][c >> 2]);
      const float s0 = h2f((uint16_t)(sd & 0xffffu)), s1 = h2f((uint16_t)(sd >> 16));
      if (cvalid) {
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][r] = __builtin_fmaf(t1[r], s1, __builtin_fmaf(t0[r], s0, acc[t][r]));
      }
    }
  }

  // ---- (6) CSR staging loads first (their latency runs under the barrier below): the mp
  //      activations of each of this thread's four entries' columns (k-major copy), every
  //      lane loading from an in-bounds address; the stores to LDS are predicated ----
  const int e_stage = csr ? min(min(e1, e0 + p.ecap), p.csr_nnz & ~3) : 0;
  const int g4 = (e0 & ~3) + 4 * tid;
  // Two 16-byte loads per entry whatever the row count (no branches between the loads and
  // the stores, whose register moves would wait for the loads): mp = 16 reads the column's
  // 32 bytes; mp = 8 its 16 bytes twice; mp = 4 the aligned 16 bytes holding the column
  // and its even/odd neighbour (K is even, so both are in the tensor).  Without CSR the
  // loads re-read the first 32 bytes of the k-major copy and nothing is stored.
  auto gload = [&](int c, uint4& a, uint4& b) __attribute__((always_inline)) {
    const uint32_t col = csr ? min((uint32_t)c, (uint32_t)(p.k - 1)) : 0u;
    const uint32_t oa = p.mp == 4 ? (col * 8u) & ~15u : col * (uint32_t)p.mp * 2u;
    const uint32_t ob = p.mp == 16 ? oa + 16u : oa;
    a = *(const uint4*)((const uint8_t*)p.xk + oa);
    b = *(const uint4*)((const uint8_t*)p.xk + ob);
  };
  uint4 ga0, gb0, ga1, gb1, ga2, gb2, ga3, gb3;
  gload(ocv.x, ga0, gb0);
  gload(ocv.y, ga1, gb1);
  gload(ocv.z, ga2, gb2);
  gload(ocv.w, ga3, gb3);
  // ---- (7) wave partials -> LDS (the LUT is dead once every wave has streamed) ----
  __syncthreads();
  sf4_t* red = (sf4_t*)smem;  // [wave][T][64 lanes]
#pragma unroll
  for (int t = 0; t < T; ++t) red[(wave * T + t) * 64 + lane] = acc[t];
  int32_t* rps = (int32_t*)(smem + p.off_rp);
  if (csr && tid <= Rw) rps[tid] = rp_v;
  float* bl = (float*)(smem + p.off_bias);
  if (p.bias != nullptr && tid < Rw)
    bl[tid] = p.bias_dt == SPECTRA_F32 ? __builtin_bit_cast(float, bias_raw) : to_f32_16((uint16_t)bias_raw, p.bias_dt);
  int32_t* fxs = (int32_t*)(smem + p.off_fx);
  if (tid < p.m) fxs[tid] = fx_reg;
  // CSR entries: the gathered mp activations of each entry's column, staged with the
  // value; entries beyond the staging capacity (or in a partial last group of the
  // array) are read directly in the per-output phase
  uint16_t* xe = (uint16_t*)(smem + p.off_xe);
  uint16_t* ve = (uint16_t*)(smem + p.off_ve);
  if (csr) {
    auto stage = [&](int u, int col, uint32_t val, const uint4& a, const uint4& b) __attribute__((always_inline)) {
      const int e = g4 + u;
      if (e >= e0 && e < e_stage && g4 + 4 <= p.csr_nnz) {
        const int el = e - e0;
        if (p.mp == 16) {
          ((uint4*)(xe + el * 16))[0] = a;
          ((uint4*)(xe + el * 16))[1] = b;
        } else if (p.mp == 8) {
          *(uint4*)(xe + el * 8) = a;
        } else {
          *(uint2*)(xe + el * 4) = (col & 1) ? make_uint2(a.z, a.w) : make_uint2(a.x, a.y);
        }
        ve[el] = (uint16_t)val;
      }
    };
    stage(0, ocv.x, ovv.x & 0xffffu, ga0, gb0);
    stage(1, ocv.y, ovv.x >> 16, ga1, gb1);
    stage(2, ocv.z, ovv.y & 0xffffu, ga2, gb2);
    stage(3, ocv.w, ovv.y >> 16, ga3, gb3);
  }
  __syncthreads();

  // ---- (8) cross-wave sums in a fixed wave order: thread (t, lane) adds the float4 of
  //      every wave (conflict-free 16-byte reads) into sums[m][row] (m-major) ----
  float* sums = (float*)(smem + p.off_sums);
  for (int i = tid; i < T * 64; i += BD) {
    const int t = i >> 6, l = i & 63;
    sf4_t v = red[t * 64 + l];
    for (int w = 1; w < nw; ++w) v += red[(w * T + t) * 64 + l];
    const int row = 16 * t + (l & 15), mq = 4 * (l >> 4);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (mq + r < p.m) sums[(mq + r) * R + row] = v[r];
  }
  // ---- (8b) CSR sums: thread (row, group of 4 m, part) takes a contiguous part of the
  //      row's entries (P parts on adjacent lanes), 4 activations per entry in one 8-byte
  //      read; the parts meet in a fixed butterfly order (deterministic) ----
  float* csums = (float*)(smem + p.off_csum);
  if (csr) {
    const int ng = p.mp >> 2;                       // groups of 4 activation rows
    const int pairs = Rw * ng;
    int P = 1;                                      // parts per (row, group): a power of two <= 64
    while (P < 64 && pairs * P * 2 <= BD) P *= 2;
    const int part = tid & (P - 1);
    for (int q = tid / P; q < (pairs + BD / P - 1) / (BD / P) * (BD / P); q += BD / P) {  // uniform trip count
      const bool okq = q < pairs;
      const int row = okq ? q / ng : 0, mg = okq ? q - (q / ng) * ng : 0;
      const int lo = rps[row], hi = rps[row + 1];
      const int hs = min(hi, e_stage);
      const int len = max(hs - lo, 0), per = (len + P - 1) / P;
      const int a = lo + part * per, b = min(a + per, hs);
      float acc4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int e = a; okq && e < b; ++e) {
        const float vv = h2f(ve[e - e0]);
        const uint2 xx = *(const uint2*)(xe + (e - e0) * p.mp + 4 * mg);
        acc4[0] += vv * h2f((uint16_t)(xx.x & 0xffffu));
        acc4[1] += vv * h2f((uint16_t)(xx.x >> 16));
        acc4[2] += vv * h2f((uint16_t)(xx.y & 0xffffu));
        acc4[3] += vv * h2f((uint16_t)(xx.y >> 16));
      }
      if (okq && part == 0)
        for (int e = max(lo, hs); e < hi; ++e) {  // beyond the staged entries: the side tensors directly
          const uint32_t col = min((uint32_t)p.ccol[e], (uint32_t)(p.k - 1));
          const float vv = h2f(p.cval[e]);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc4[i] += vv * h2f(p.xk[(int64_t)col * p.mp + 4 * mg + i]);
        }
      for (int o = 1; o < P; o <<= 1)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc4[i] += __shfl_xor(acc4[i], o);
      if (okq && part == 0)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (4 * mg + i < p.m) csums[(4 * mg + i) * R + row] = acc4[i];
    }
  }
  __syncthreads();

  // ---- (9) per output (row, m): dense sum + outliers, scale, bias, store ----
  for (int idx = tid; idx < Rw * p.m; idx += BD) {
    const int m = idx / Rw, row = idx - m * Rw;
    float v = sums[m * R + row];
    if (csr) v += csums[m * R + row];
    float y = v * __builtin_bit_cast(float, (uint32_t)(127 - fxs[m]) << 23);
    if (p.bias != nullptr) y += bl[row];
    ((uint16_t*)p.out)[(int64_t)m * p.ldo + r0 + row] = from_f32_16(y, p.act_dt);
  }
}

typedef void (*skinny_fn)(const SkinnyParams);

template <int T>
static skinny_fn pick_cpw(int cpw) {
  switch (cpw) {
    case 1: return skinny_kernel<T, 1>;
    case 2: return skinny_kernel<T, 2>;
    case 3: return skinny_kernel<T, 3>;
    case 4: return skinny_kernel<T, 4>;
    case 5: if constexpr (T <= 2) return skinny_kernel<T, 5>; else return nullptr;
    case 6: if constexpr (T <= 2) return skinny_kernel<T, 6>; else return nullptr;
    case 7: if constexpr (T == 1) return skinny_kernel<T, 7>; else return nullptr;
    case 8: if constexpr (T == 1) return skinny_kernel<T, 8>; else return nullptr;
    default: return nullptr;
  }
}

static skinny_fn pick_skinny(int T, int cpw) {
  if (T == 1) return pick_cpw<1>(cpw);
  if (T == 2) return pick_cpw<2>(cpw);
  return pick_cpw<4>(cpw);
}

static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

static int skinny_mp(int64_t m) { return m <= 4 ? 4 : (m <= 8 ? 8 : 16); }

// workspace of the small-batch path: xa + xk (K x mp fp16 each) + row exponents
size_t skinny_workspace(const spectra_qweight_t* w, int64_t m) {
  if (m < 1 || m > 16) return 0;
  const size_t mp = (size_t)skinny_mp(m);
  return 2 * al256((size_t)w->k * mp * 2) + al256(16 * 4);
}

struct SkinnyPlan {
  int T, cpw, nw, nrounds, grid;
};

static bool plan_skinny(int64_t n, int64_t k, SkinnyPlan* pl) {
  const int nchunks = (int)(k / 128);
  const int64_t tiles = (n + 15) / 16;
  const int ncu = device_cu_count();
  int T = (int)((tiles + ncu - 1) / ncu);
  T = T <= 1 ? 1 : (T <= 2 ? 2 : 4);
  const int cpw_max = T == 1 ? 8 : (T == 2 ? 6 : 4);
  const int nrounds = (nchunks + 8 * cpw_max - 1) / (8 * cpw_max);
  const int per_round = (nchunks + nrounds - 1) / nrounds;
  const int nw = per_round < 8 ? per_round : 8;
  const int cpw = (per_round + nw - 1) / nw;
  pl->T = T; pl->cpw = cpw; pl->nw = nw; pl->nrounds = nrounds;
  pl->grid = (int)((tiles + T - 1) / T);
  return cpw >= 1 && cpw <= cpw_max;
}

// Returns SPECTRA_ERR_UNSUPPORTED (and launches nothing) when the operands are not
// served by this family: the caller then uses the prefill GEMM.
// SPECTRA_OK when this family serves the operands (the descriptor already validated),
// SPECTRA_ERR_UNSUPPORTED with the reason otherwise
int skinny_supported(const spectra_qweight_t* w, const void* x, int64_t ldx, int64_t m) {
  if (m < 2 || m > 16) return fail(SPECTRA_ERR_UNSUPPORTED, "small-batch family serves 2 <= m <= 16");
  if (w->format != SPECTRA_FMT_NF4 || w->group_size != 64)
    return fail(SPECTRA_ERR_UNSUPPORTED, "small-batch family serves NF4 with blocks of 64");
  if (w->k % 128 != 0 || w->k > 32768)
    return fail(SPECTRA_ERR_UNSUPPORTED, "small-batch family needs K % 128 == 0 and K <= 32768");
  if (w->outlier_kind == SPECTRA_OUTLIERS_COLUMNS)
    return fail(SPECTRA_ERR_UNSUPPORTED, "small-batch family serves CSR outliers only");
  if ((reinterpret_cast<uintptr_t>(w->packed) % 16) != 0 || w->packed_stride % 16 != 0 ||
      (reinterpret_cast<uintptr_t>(w->scales) % 4) != 0 || w->scales_stride % 2 != 0)
    return fail(SPECTRA_ERR_UNSUPPORTED, "small-batch family needs 16-byte packed rows and 4-byte scale pairs");
  const bool csr = w->outlier_kind == SPECTRA_OUTLIERS_CSR && w->csr_nnz > 0;
  if (csr && ((reinterpret_cast<uintptr_t>(w->csr_col) % 16) != 0 || (reinterpret_cast<uintptr_t>(w->csr_val) % 8) != 0))
    return fail(SPECTRA_ERR_UNSUPPORTED, "small-batch family needs 16-byte CSR columns and 8-byte values");
  if (w->hadamard_block > 1024) return fail(SPECTRA_ERR_UNSUPPORTED, "hadamard_block too large");
  if ((reinterpret_cast<uintptr_t>(x) % 16) != 0 || ldx % 8 != 0)
    return fail(SPECTRA_ERR_UNSUPPORTED, "small-batch family needs 16-byte aligned activation rows");
  SkinnyPlan pl;
  if (!plan_skinny(w->n, w->k, &pl)) return fail(SPECTRA_ERR_UNSUPPORTED, "no small-batch plan for this shape");
  return SPECTRA_OK;
}

int skinny_launch(const spectra_qweight_t* w, const void* x, int64_t ldx, int64_t m, int act_dtype, void* out,
                  int64_t ldo, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const int sup = skinny_supported(w, x, ldx, m);
  if (sup != SPECTRA_OK) return sup;
  SkinnyPlan pl;
  plan_skinny(w->n, w->k, &pl);
  const bool csr = w->outlier_kind == SPECTRA_OUTLIERS_CSR && w->csr_nnz > 0;
  const size_t need = skinny_workspace(w, m);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(SPECTRA_ERR_WORKSPACE, "workspace missing or smaller than spectra_w4a16_gemm_workspace()");
  SPECTRA_REQUIRE((reinterpret_cast<uintptr_t>(workspace) % 256) == 0, "workspace must be 256-byte aligned");
  const int mp = skinny_mp(m);
  uint8_t* ws = (uint8_t*)workspace;
  uint4* xa = (uint4*)ws;
  uint16_t* xk = (uint16_t*)(ws + al256((size_t)w->k * mp * 2));
  int32_t* fexp = (int32_t*)(ws + 2 * al256((size_t)w->k * mp * 2));

  const int had = w->hadamard_block;
  int log_had = 0;
  while (had > 1 && (1 << log_had) < had) ++log_had;
  const float div = had > 1 ? (float)std::sqrt((double)had) : 1.0f;
  const int seg = had > kSkSeg ? had : kSkSeg;
  const int nseg = (int)((w->k + seg - 1) / seg);
  int st;
  if (log_had <= 9) {  // blocks up to 512: register / DPP butterflies
    const int nsegf = (int)((w->k + kSkSegFast - 1) / kSkSegFast);
    hipLaunchKernelGGL(skinny_prep_fast_kernel, dim3((unsigned)nsegf, (unsigned)m), dim3(kSkPrepThreads), 0, stream,
                       x, ldx, act_dtype, (int)w->k, log_had, div, mp, w->marlin_layout ? 1 : 0, csr ? 1 : 0, xa,
                       xk, fexp);
  } else {
    st = ensure_lds_limit((const void*)skinny_prep_kernel);
    if (st != SPECTRA_OK) return st;
    hipLaunchKernelGGL(skinny_prep_kernel, dim3((unsigned)nseg, (unsigned)m), dim3(kSkPrepThreads), (size_t)seg * 4,
                       stream, x, ldx, act_dtype, (int)w->k, seg, log_had, div, mp, w->marlin_layout ? 1 : 0,
                       csr ? 1 : 0, xa, xk, fexp);
  }
  SPECTRA_HIP_CHECK(hipGetLastError());

  SkinnyParams p;
  p.packed = w->packed; p.ldp = w->packed_stride;
  p.scales = (const uint32_t*)w->scales; p.lds32 = w->scales_stride / 2;
  p.xa = xa; p.xk = xk; p.fexp = fexp;
  p.rowptr = w->csr_rowptr; p.ccol = w->csr_col; p.cval = w->csr_val;
  p.bias = w->bias; p.out = out; p.ldo = ldo;
  p.m = (int)m; p.mp = mp; p.n = (int)w->n; p.k = (int)w->k; p.nchunks = (int)(w->k / 128);
  p.nrounds = pl.nrounds; p.csr_nnz = csr ? (int)w->csr_nnz : 0;
  p.okind = csr ? SPECTRA_OUTLIERS_CSR : SPECTRA_OUTLIERS_NONE;
  p.bias_dt = w->bias_dtype; p.act_dt = act_dtype;
  // LDS: the LUT (64 KB), reused after the stream for the wave partials and the staged
  // CSR entries; then the code tables and the row pointers
  const int BD = pl.nw * 64;
  const uint32_t red_bytes = (uint32_t)(pl.nw * pl.T * 1024);
  int ecap = 0;
  uint32_t stage_end = red_bytes;
  if (csr) {
    const double per_row = (double)w->csr_nnz / (double)w->n;
    int want = (int)(per_row * 16 * pl.T * 1.25) + 64;
    if (want > 4 * BD - 3) want = 4 * BD - 3;
    ecap = want;
    stage_end = red_bytes + (uint32_t)ecap * (uint32_t)(2 * mp + 2) + 32;
  }
  p.off_sums = (stage_end + 15u) & ~15u;  // [16][16 T] fp32 cross-wave sums
  p.off_csum = p.off_sums + (uint32_t)(16 * 16 * pl.T * 4);  // [16][16 T] fp32 outlier sums
  stage_end = p.off_csum + (uint32_t)(16 * 16 * pl.T * 4);
  const uint32_t base = stage_end > (uint32_t)kSkLut ? ((stage_end + 15u) & ~15u) : (uint32_t)kSkLut;
  p.off_xe = red_bytes;
  p.off_ve = (red_bytes + (uint32_t)ecap * (uint32_t)(2 * mp) + 15u) & ~15u;
  p.ecap = ecap;
  p.off_rp = base;
  p.off_bias = (p.off_rp + (uint32_t)(16 * pl.T + 1) * 4 + 15u) & ~15u;
  p.off_fx = (p.off_bias + (uint32_t)(16 * pl.T) * 4 + 15u) & ~15u;
  const uint32_t lds = p.off_fx + 16u * 4u;
  if (lds > 163840) return fail(SPECTRA_ERR_UNSUPPORTED, "small-batch LDS plan too large");
  skinny_fn fn = pick_skinny(pl.T, pl.cpw);
  if (fn == nullptr) return fail(SPECTRA_ERR_UNSUPPORTED, "no small-batch kernel for this plan");
  st = ensure_lds_limit((const void*)fn, true);
  if (st != SPECTRA_OK) return st;
  hipLaunchKernelGGL(fn, dim3((unsigned)pl.grid), dim3((unsigned)BD), (size_t)lds, stream, p);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

}  // namespace spectra
