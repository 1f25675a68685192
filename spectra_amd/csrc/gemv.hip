// Decode GEMV family for gfx950: out[m, :] = FWHT(x[m, :]) . W_eff^T + bias, m <= 4.
//
// Replaces the reference's single-row Triton GEMV (kernels.py:16-184).  Design:
//  * Workgroup = S x G waves (at most 8).  S = ceil(K / 2048) K-slices; G row groups.  A wave
//    owns one slice (each lane 32 k = 16 packed bytes, one dwordx4) of RPW rows.  All weight
//    loads of a wave are issued up front, after the activation loads, so waiting for x
//    never waits for the weight stream (vmcnt counts in issue order).
//  * VALU is the scarce resource while the stream is in flight, so every setup step is
//    sized per element, never per wave:
//    - activations: each thread owns one 32-element run of x: five butterfly stages in
//      registers, the stages across the 4 threads of a 128-block with DPP quad
//      permutes; the run is scaled by its own power of two (max |x| -> [2^14, 2^15)),
//      rounded to fp16 and stored in LDS in "pair order" (the two k's of packed byte j
//      side by side) with the run's inverse scale beside it; the 1/sqrt(block)
//      normalisation is applied once per output.
//    - nibble decode: a 256-entry LUT in LDS maps a packed byte to the fp16 pair
//      (code[lo], code[hi]) -- NF4 levels for Format B, the integers 0..15 for Format A.
//      It is replicated per lane (64 KB) so that lane l always reads bank l: the LDS
//      address is (byte << 8) | (lane << 2), built by one v_perm_b32.  Each wave fills
//      its share from a 16-entry table it wrote itself (no barrier, no select chains).
//  * Math per packed byte: v_perm + ds_read_b32 + v_dot2_f32_f16.  Scales are applied once
//    per 32 k: Format B acc * absmax * run_scale; Format A (acc - z * sum(x)) * s * run_scale.
//  * Lane partials of all rows are reduced across the wave with a transposed halving
//    reduction; per-row totals (slices, outliers, bias) are reduced by one wave per row in
//    a fixed order: the result is deterministic run to run.
#include <cmath>

#include "common.h"

namespace spectra {

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

constexpr int kRpwMax = 12;  // rows per wave held in registers
constexpr int kOj = 4;       // outlier entries per thread held in registers
constexpr int kLutBytes = 65536;
constexpr int kMaxWaves = 8;

struct GemvParams {
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
  const void* x;
  int64_t ldx;
  void* out;
  int64_t ldo;
  int n, k, m;
  int gshift;  // log2(group / block size)
  int had, log_had, marlin;
  int okind, n_out, ow_dt, bias_dt, act_dt;
  int R, S, G, ocap;
  uint32_t off_xp, off_xsc, off_part, off_codes, off_rp, off_bias, off_oprod;
  float out_scale;  // 1/sqrt(hadamard_block) (1 without rotation)
  float inv_n_out;  // 1/n_out (dense outlier columns)
};

__device__ __forceinline__ uint16_t nf4_f16_bits(int i) {
  // fp16 roundings of the NF4 levels (compressor.py:22-27)
  uint16_t r = 0xbc00;
  r = (i == 1) ? 0xb992 : r;
  r = (i == 2) ? 0xb833 : r;
  r = (i == 3) ? 0xb652 : r;
  r = (i == 4) ? 0xb48d : r;
  r = (i == 5) ? 0xb1ea : r;
  r = (i == 6) ? 0xadd4 : r;
  r = (i == 7) ? 0x0000 : r;
  r = (i == 8) ? 0x2d18 : r;
  r = (i == 9) ? 0x3126 : r;
  r = (i == 10) ? 0x33e0 : r;
  r = (i == 11) ? 0x3568 : r;
  r = (i == 12) ? 0x370d : r;
  r = (i == 13) ? 0x3880 : r;
  r = (i == 14) ? 0x39c9 : r;
  r = (i == 15) ? 0x3c00 : r;
  return r;
}

__device__ __forceinline__ float pow2f(int e) {  // e in [-126, 127]
  return __builtin_bit_cast(float, (uint32_t)(e + 127) << 23);
}

// fp16 position of element k inside one activation row of xp: run q = k / 32 holds 16
// (lo, hi) pairs (pair j = (k_j, k_j + 16) for the marlin nibble order, (2j, 2j+1)
// otherwise) in 4 16-byte chunks stored at [slice q / 64][chunk][lane q % 64]
__device__ __forceinline__ int xp_pos(int k, int marlin) {
  const int q = k >> 5, e = k & 31;
  const int j = marlin ? (e & 15) : (e >> 1), half = marlin ? (e >> 4) : (e & 1);
  return ((((q >> 6) * 4 + (j >> 2)) * 64 + (q & 63)) * 4 + (j & 3)) * 2 + half;
}

// value of lane (lane ^ MASK): DPP quad permutes for 1 and 2, ds_swizzle (xor mode, no
// address register) for 4..16, a cross-lane permute for 32
template <int MASK>
__device__ __forceinline__ float lane_xor_c(float v) {
  const int iv = __builtin_bit_cast(int, v);
  if constexpr (MASK == 1) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0xB1, 0xF, 0xF, false));
  else if constexpr (MASK == 2) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x4E, 0xF, 0xF, false));
  else if constexpr (MASK < 32) return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(iv, (MASK << 10) | 0x1F));
  else return __shfl_xor(v, MASK, 64);
}

// Transposed halving reduction of N values per lane across the 64 lanes: at the step
// with offset OFF the lanes with bit OFF set keep the upper half of their values and add
// their partner's upper half (the others the lower half), so N values cost N-1 exchanges
// instead of 6N.  Offsets go 1, 2, 4, ... so the steps that move the most values use the
// cheap DPP permutes.  At the end every lane holds the total number idx(lane).
template <int N, int OFF>
__device__ __forceinline__ void transposed_reduce(float* vals, int lane, int& idx) {
  if constexpr (OFF <= 32) {
    if constexpr (N > 1) {
      constexpr int H = N / 2;
      const bool upper = (lane & OFF) != 0;
#pragma unroll
      for (int q = 0; q < H; ++q) {
        const float send = upper ? vals[q] : vals[q + H];
        const float keep = upper ? vals[q + H] : vals[q];
        vals[q] = keep + lane_xor_c<OFF>(send);
      }
      if (upper) idx += H;
      transposed_reduce<H, OFF * 2>(vals, lane, idx);
    } else {
      vals[0] += lane_xor_c<OFF>(vals[0]);
      transposed_reduce<1, OFF * 2>(vals, lane, idx);
    }
  }
}

// Blockwise FWHT of one 32-element run (block 2^LOG): stages h = 1..16 inside the run,
// h = 32.. across the lanes of the block (partner lane ^ h/32), pairs (i, i+h) ->
// (u+v, u-v) in the reference's stage order (compressor.py:34-39).  Fully static.
template <int LOG>
__device__ __forceinline__ void fwht_run(float (&v)[32], int lane) {
  constexpr int IN = LOG < 5 ? LOG : 5;
#pragma unroll
  for (int st = 0; st < IN; ++st) {
    const int h = 1 << st;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      if ((e & h) == 0) {
        const float a = v[e], b = v[e + h];
        v[e] = a + b;
        v[e + h] = a - b;
      }
    }
  }
  if constexpr (LOG > 5) {
    constexpr int MSK = 1;
    const bool upper = (lane & MSK) != 0;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const float o = lane_xor_c<MSK>(v[e]);
      v[e] = upper ? (o - v[e]) : (v[e] + o);
    }
  }
  if constexpr (LOG > 6) {
    constexpr int MSK = 2;
    const bool upper = (lane & MSK) != 0;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const float o = lane_xor_c<MSK>(v[e]);
      v[e] = upper ? (o - v[e]) : (v[e] + o);
    }
  }
  if constexpr (LOG > 7) {
    constexpr int MSK = 4;
    const bool upper = (lane & MSK) != 0;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const float o = lane_xor_c<MSK>(v[e]);
      v[e] = upper ? (o - v[e]) : (v[e] + o);
    }
  }
  if constexpr (LOG > 8) {
    constexpr int MSK = 8;
    const bool upper = (lane & MSK) != 0;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const float o = lane_xor_c<MSK>(v[e]);
      v[e] = upper ? (o - v[e]) : (v[e] + o);
    }
  }
}

// one uniform branch into a straight-line transform
__device__ __forceinline__ void fwht_run_dispatch(float (&v)[32], int lane, int log_had) {
  switch (log_had) {
    case 1: fwht_run<1>(v, lane); break;
    case 2: fwht_run<2>(v, lane); break;
    case 3: fwht_run<3>(v, lane); break;
    case 4: fwht_run<4>(v, lane); break;
    case 5: fwht_run<5>(v, lane); break;
    case 6: fwht_run<6>(v, lane); break;
    case 7: fwht_run<7>(v, lane); break;
    case 8: fwht_run<8>(v, lane); break;
    case 9: fwht_run<9>(v, lane); break;
    default: break;
  }
}

// Sum over the 64 lanes with DPP only (no LDS): quad permutes, half-row and row mirrors,
// then row broadcasts; the total ends in lane 63 and is read back as a scalar.
__device__ __forceinline__ float wave_sum(float v) {
  int t;
  t = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  v += __builtin_bit_cast(float, t);
  t = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  v += __builtin_bit_cast(float, t);
  t = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false);  // row_half_mirror
  v += __builtin_bit_cast(float, t);
  t = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false);  // row_mirror
  v += __builtin_bit_cast(float, t);
  t = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false);  // row_bcast:15
  v += __builtin_bit_cast(float, t);
  t = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, false);  // row_bcast:31
  v += __builtin_bit_cast(float, t);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

template <int FMT, int MT, int RPW>
__global__ void __launch_bounds__(512) gemv_kernel(const GemvParams p) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int XQ = MT;  // 32-element activation runs per thread (at most)
  const int tid = threadIdx.x;
  const int BD = blockDim.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwaves = BD >> 6;
  const int s = wave % p.S, g = wave / p.S;
  const int r0 = blockIdx.x * p.R;
  const int Rw = min(p.R, p.n - r0);
  const int K = p.k;
  const int qpr = K >> 5;  // 32-element runs per activation row

  // ---------------- (1) activation runs, CSR row pointers, bias: raw bits, issued first ----------------
  uint4 xr[XQ][4];
  bool xok[XQ];
  int xm[XQ], xq[XQ];
#pragma unroll
  for (int i = 0; i < XQ; ++i) {
    const int qd = tid + i * BD;
    int m = 0;
#pragma unroll
    for (int mm = 1; mm < MT; ++mm) m += qd >= mm * qpr ? 1 : 0;
    xm[i] = m;
    xq[i] = qd - m * qpr;
    xok[i] = qd < MT * qpr && m < p.m;
    const uint4* src = (const uint4*)((const uint16_t*)p.x + (xok[i] ? (int64_t)m * p.ldx + (int64_t)xq[i] * 32 : 0));
#pragma unroll
    for (int c = 0; c < 4; ++c) xr[i][c] = src[c];
  }
  int rp_v = 0, e0 = 0, e1 = 0;
  if (p.okind == SPECTRA_OUTLIERS_CSR) {
    rp_v = p.rowptr[r0 + min(tid, Rw)];
    e0 = p.rowptr[r0];
    e1 = p.rowptr[r0 + Rw];
  }
  uint32_t bias_raw = 0;
  if (p.bias != nullptr) {
    const int64_t bi = r0 + (tid < Rw ? tid : 0);
    if (p.bias_dt == SPECTRA_F32) bias_raw = ((const uint32_t*)p.bias)[bi];
    else bias_raw = ((const uint16_t*)p.bias)[bi];
  }

  // ---------------- (2) the weight stream: every row of this wave, up front ----------------
  const int kb = s * 2048 + lane * 32;  // first k of this lane (one 32-run)
  const bool kvalid = kb < K;
  uint4 wq[RPW];
  uint16_t sc[RPW];
  uint8_t zq[RPW];
  bool wok[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int rl = g + i * p.G;
    wok[i] = (rl < Rw) && kvalid;
    const int64_t row = r0 + (wok[i] ? rl : 0);
    const int kk = wok[i] ? kb : 0;
    wq[i] = *(const uint4*)(p.packed + row * p.ldp + (kk >> 1));
    sc[i] = p.scales[row * p.lds + (kk >> p.gshift)];
    if (FMT == SPECTRA_FMT_ASYM_G32) zq[i] = p.zeros[row * p.ldz + (kk >> 5)];
  }

  // ---------------- (3) nibble-pair LUT from a wave-private 16-entry code table ----------------
  {
    uint16_t* codes = (uint16_t*)(smem + p.off_codes) + wave * 16;
    if (lane < 16) codes[lane] = FMT == SPECTRA_FMT_NF4 ? nf4_f16_bits(lane) : f2h((float)lane);
    // consecutive lanes fill consecutive 16-byte chunks (conflict-free stores); the 16
    // lanes of one 256-byte row read the same two codes (broadcast)
    uint4* lut = (uint4*)smem;
    for (int w = tid; w < 256 * 16; w += BD) {
      const int v = w >> 4;
      const uint32_t e = (uint32_t)codes[v & 15] | ((uint32_t)codes[v >> 4] << 16);
      lut[w] = make_uint4(e, e, e, e);
    }
  }

  // ---------------- (4) activation runs: FWHT, run scale, fp16 pairs -> LDS ----------------
  uint16_t* xp = (uint16_t*)(smem + p.off_xp);
  const int XS = ((K + 2047) >> 11) << 11;  // xp row stride: whole 2048-element slices
  float* xsc = (float*)(smem + p.off_xsc);
#pragma unroll
  for (int i = 0; i < XQ; ++i) {
    float v[32];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t u[4] = {xr[i][c].x, xr[i][c].y, xr[i][c].z, xr[i][c].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint16_t h = (uint16_t)(u[e >> 1] >> (16 * (e & 1)));
        v[c * 8 + e] = xok[i] ? to_f32_16(h, p.act_dt) : 0.0f;
      }
    }
    fwht_run_dispatch(v, lane, p.log_had);
    float mx = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; ++e) mx = fmaxf(mx, fabsf(v[e]));
    const uint32_t bits = __builtin_bit_cast(uint32_t, mx);
    const int eb = (int)(bits >> 23);
    const int E = eb == 0 ? -126 : eb - 127;   // floor(log2(mx)) for normal mx
    int F = bits == 0 ? 0 : 14 - E;            // mx * 2^F in [2^14, 2^15)
    F = F < -126 ? -126 : (F > 126 ? 126 : F);
    const float f = pow2f(F);
    uint32_t d[16];
    const bool mar = p.marlin != 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {  // static register indices for both layouts, then a select
      const float lo = mar ? v[j] : v[2 * j], hi = mar ? v[j + 16] : v[2 * j + 1];
      d[j] = (uint32_t)f2h(lo * f) | ((uint32_t)f2h(hi * f) << 16);
    }
    if (tid + i * BD < MT * qpr) {  // every run of rows 0..MT-1 (padded rows m >= p.m hold zeros)
      // run q is consumed by lane q % 64 of slice q / 64: stored as 4 16-byte chunks at
      // [m][slice][chunk][lane] so that each ds_read_b128 of the stream reads 1 KB contiguous
      uint4* dst = (uint4*)(xp + xm[i] * XS) + ((xq[i] >> 6) * 4) * 64 + (xq[i] & 63);
      dst[0] = make_uint4(d[0], d[1], d[2], d[3]);
      dst[64] = make_uint4(d[4], d[5], d[6], d[7]);
      dst[128] = make_uint4(d[8], d[9], d[10], d[11]);
      dst[192] = make_uint4(d[12], d[13], d[14], d[15]);
      xsc[xm[i] * qpr + xq[i]] = pow2f(-F);
    }
  }
  int32_t* rps = (int32_t*)(smem + p.off_rp);
  if (p.okind == SPECTRA_OUTLIERS_CSR && tid <= Rw) rps[tid] = rp_v;
  float* bl = (float*)(smem + p.off_bias);
  if (p.bias != nullptr && tid < Rw)
    bl[tid] = p.bias_dt == SPECTRA_F32 ? __builtin_bit_cast(float, bias_raw) : to_f32_16((uint16_t)bias_raw, p.bias_dt);

  // ---------------- (5) outlier entries of this workgroup (consumed after the stream) ----------------
  // raw bits, one 32-bit register per value; one branch-free load pair per entry:
  // CSR reads col/val, dense columns read the low dword of idx and the row's weight
  int ocol[kOj];
  uint32_t oraw[kOj];
  bool ook[kOj];
  {
    const bool has_o = p.okind != SPECTRA_OUTLIERS_NONE;
    const bool csr = p.okind == SPECTRA_OUTLIERS_CSR;
    const int n_out = p.n_out > 0 ? p.n_out : 1;
    const int cnt = !has_o ? 0 : (csr ? e1 - e0 : Rw * n_out);
#pragma unroll
    for (int jo = 0; jo < kOj; ++jo) {
      const int el = tid + jo * BD;
      ook[jo] = el < cnt;
      const int ei = ook[jo] ? el : 0;
      // (row, column) of a dense-column entry: float reciprocal, exact after one correction
      int r = (int)((float)ei * p.inv_n_out);
      int jj = ei - r * n_out;
      r = jj < 0 ? r - 1 : (jj >= n_out ? r + 1 : r);
      jj = ei - r * n_out;
      const int gi = ook[jo] ? e0 + el : 0;  // CSR entry; entry 0 exists whenever CSR is used (nnz > 0)
      // without outliers the loads read the first bytes of the packed/scale tensors
      // (always present) so that the load sequence, and the wait counts, never branch
      const int32_t* cptr = !has_o ? (const int32_t*)p.packed
                                   : (csr ? p.ccol + gi : (const int32_t*)(p.oidx + jj));
      const uint16_t* vptr = !has_o ? p.scales
                                    : (csr ? p.cval + gi : (const uint16_t*)p.ow + (int64_t)(r0 + r) * p.ldow + jj);
      ocol[jo] = *cptr;
      oraw[jo] = *vptr;
    }
  }

  __syncthreads();  // --- barrier 1: LUT, activation pairs and run scales

  // ---------------- (6) this lane's activation pairs and run scales ----------------
  uint32_t xpair[MT][16];
  float xs[MT], xsum[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const int kk = kvalid ? kb : 0;
    const int q = kk >> 5;  // this lane's run: lane (q & 63) of slice s
    const uint4* src = (const uint4*)(xp + m * XS) + ((q >> 6) * 4) * 64 + (q & 63);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint4 a = src[64 * c];
      xpair[m][4 * c] = a.x; xpair[m][4 * c + 1] = a.y; xpair[m][4 * c + 2] = a.z; xpair[m][4 * c + 3] = a.w;
    }
    xs[m] = xsc[m * qpr + (kk >> 5)];
    xsum[m] = 0.0f;
    if (FMT == SPECTRA_FMT_ASYM_G32) {
#pragma unroll
      for (int q = 0; q < 16; ++q)
        xsum[m] += h2f((uint16_t)xpair[m][q]) + h2f((uint16_t)(xpair[m][q] >> 16));
    }
  }

  // ---------------- (7) the stream: LUT decode + dot2 per packed byte ----------------
  constexpr int V = RPW * MT;
  constexpr int VP = V <= 1 ? 1 : V <= 2 ? 2 : V <= 4 ? 4 : V <= 8 ? 8 : V <= 16 ? 16 : V <= 32 ? 32 : 64;
  float vals[VP];
#pragma unroll
  for (int q = 0; q < VP; ++q) vals[q] = 0.0f;
  const uint32_t lanebits = (uint32_t)lane << 2;
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
    const uint32_t wd[4] = {wq[i].x, wq[i].y, wq[i].z, wq[i].w};
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      const uint32_t addr = __builtin_amdgcn_perm(wd[b >> 2], lanebits, 0x0c0c0000u | ((4u + (b & 3)) << 8));
      const uint32_t code2 = *(const uint32_t*)(smem + addr);
#pragma unroll
      for (int m = 0; m < MT; ++m)
        acc[m] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, code2),
                                        __builtin_bit_cast(f16x2_t, xpair[m][b]), acc[m], false);
    }
    const float sf = h2f(sc[i]);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      float v;
      if (FMT == SPECTRA_FMT_ASYM_G32) v = (acc[m] - (float)zq[i] * xsum[m]) * (sf * xs[m]);
      else v = acc[m] * (sf * xs[m]);
      vals[i * MT + m] = wok[i] ? v : 0.0f;
    }
  }

  // ---------------- (8) transposed halving reduction across the wave ----------------
  int idx = 0;
  transposed_reduce<VP, 1>(vals, lane, idx);
  // every lane now holds the total number idx (set by its low log2(VP) bits); lanes
  // 0..VP-1 write them
  float* part = (float*)(smem + p.off_part);
  if (lane < VP && idx < V) {
    const int i = idx / MT, m = idx - i * MT;
    const int rl = g + i * p.G;
    if (rl < Rw) part[(rl * p.S + s) * MT + m] = vals[0];
  }

  // ---------------- (9) outlier products, in the same scaled fp16 activation basis ----------------
  float* oprod = (float*)(smem + p.off_oprod);
  const int odt = p.okind == SPECTRA_OUTLIERS_CSR ? SPECTRA_F16 : p.ow_dt;
#pragma unroll
  for (int jo = 0; jo < kOj; ++jo) {
    const int el = tid + jo * BD;  // workgroup-local entry index
    if (ook[jo] && el < p.ocap) {
      const int pos = xp_pos(ocol[jo], p.marlin);
      const float ov = to_f32_16((uint16_t)oraw[jo], odt);
#pragma unroll
      for (int m = 0; m < MT; ++m)
        oprod[el * MT + m] = ov * (h2f(xp[m * XS + pos]) * xsc[m * qpr + (ocol[jo] >> 5)]);
    }
  }

  __syncthreads();  // --- barrier 2: slice partials and outlier products

  // ---------------- (10) per-row totals: one wave per row, fixed order ----------------
  for (int r = wave; r < Rw; r += nwaves) {
    int lo = 0, hi = 0;
    if (p.okind == SPECTRA_OUTLIERS_CSR) {
      lo = rps[r] - e0;
      hi = rps[r + 1] - e0;
    } else if (p.okind == SPECTRA_OUTLIERS_COLUMNS) {
      lo = r * p.n_out;
      hi = lo + p.n_out;
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m >= p.m) break;
      float v = lane < p.S ? part[(r * p.S + lane) * MT + m] : 0.0f;
      for (int el = lo + lane; el < hi; el += 64) {
        if (el < p.ocap) {
          v += oprod[el * MT + m];
        } else {  // beyond the register-staged entries: read the side tensor directly
          int col;
          float val;
          if (p.okind == SPECTRA_OUTLIERS_CSR) {
            col = p.ccol[e0 + el];
            val = h2f(p.cval[e0 + el]);
          } else {
            const int rr = el / p.n_out, jj = el - rr * p.n_out;
            col = (int)p.oidx[jj];
            val = load_elem(p.ow, (int64_t)(r0 + rr) * p.ldow + jj, p.ow_dt);
          }
          v += val * (h2f(xp[m * XS + xp_pos(col, p.marlin)]) * xsc[m * qpr + (col >> 5)]);
        }
      }
      v = wave_sum(v);
      if (lane == 0) {
        float y = v * p.out_scale;
        if (p.bias != nullptr) y += bl[r];
        ((uint16_t*)p.out)[(int64_t)m * p.ldo + r0 + r] = from_f32_16(y, p.act_dt);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host side: decomposition, LDS layout, launch
// ---------------------------------------------------------------------------
typedef void (*gemv_fn)(const GemvParams);

template <int FMT, int MT>
static gemv_fn pick_rpw(int rpw) {
  switch (rpw) {
    case 1: return gemv_kernel<FMT, MT, 1>;
    case 2: return gemv_kernel<FMT, MT, 2>;
    case 3: return gemv_kernel<FMT, MT, 3>;
    case 4: return gemv_kernel<FMT, MT, 4>;
    case 5: return gemv_kernel<FMT, MT, 5>;
    case 6: return gemv_kernel<FMT, MT, 6>;
    case 7: return gemv_kernel<FMT, MT, 7>;
    case 8: return gemv_kernel<FMT, MT, 8>;
    case 9: return gemv_kernel<FMT, MT, 9>;
    case 10: return gemv_kernel<FMT, MT, 10>;
    case 11: return gemv_kernel<FMT, MT, 11>;
    default: return gemv_kernel<FMT, MT, 12>;
  }
}

template <int FMT>
static gemv_fn pick_rpw4(int rpw) {
  switch (rpw) {
    case 1: return gemv_kernel<FMT, 4, 1>;
    case 2: return gemv_kernel<FMT, 4, 2>;
    case 3: return gemv_kernel<FMT, 4, 3>;
    case 4: return gemv_kernel<FMT, 4, 4>;
    case 5: return gemv_kernel<FMT, 4, 5>;
    case 6: return gemv_kernel<FMT, 4, 6>;
    case 7: return gemv_kernel<FMT, 4, 7>;
    default: return gemv_kernel<FMT, 4, 8>;
  }
}

template <int FMT>
static gemv_fn pick_kernel(int mt, int rpw) {
  if (mt == 1) return pick_rpw<FMT, 1>(rpw);
  if (mt == 2) return pick_rpw<FMT, 2>(rpw);
  return pick_rpw4<FMT>(rpw);
}

static uint32_t align16(uint32_t v) { return (v + 15u) & ~15u; }

struct GemvPlan {
  int mt, S, G, rpw, R, BD, grid, ocap;
  uint32_t off_xp, off_xsc, off_part, off_codes, off_rp, off_bias, off_oprod, lds_bytes;
};

// returns false when the shape does not fit this kernel family
static bool plan_gemv(int64_t n, int64_t k, int m, bool outliers, GemvPlan* pl) {
  const int mt = m <= 1 ? 1 : (m <= 2 ? 2 : 4);
  if (m > 4 || k > 16384 || k % 32) return false;
  const int S = (int)((k + 2047) / 2048);
  // at most 8 waves per workgroup: the setup work is per element, the stream per wave
  int G = kMaxWaves / S;
  const int64_t want = (n + 255) / 256;  // rows per workgroup for ~one workgroup per CU
  if (G > want) G = (int)want;
  if (G < 1) G = 1;
  int rpw = (int)((want + G - 1) / G);
  const int rpw_max = mt == 4 ? 8 : kRpwMax;
  rpw = rpw < 1 ? 1 : (rpw > rpw_max ? rpw_max : rpw);
  const int R = G * rpw;
  const int BD = 64 * S * G;
  // each thread stages at most mt 32-element activation runs
  const int64_t runs = (int64_t)mt * (k / 32);
  if (runs > (int64_t)BD * mt) return false;
  if (R + 1 > BD || R > 4096) return false;
  pl->mt = mt; pl->S = S; pl->G = G; pl->rpw = rpw; pl->R = R; pl->BD = BD;
  pl->grid = (int)((n + R - 1) / R);
  uint32_t off = kLutBytes;
  pl->off_xp = off;
  off = align16(off + (uint32_t)(mt * S * 2048 * 2));  // rows padded to whole slices
  pl->off_xsc = off;
  off = align16(off + (uint32_t)(mt * (k / 32) * 4));
  pl->off_part = off;
  off = align16(off + (uint32_t)(R * S * mt * 4));
  pl->off_codes = off;
  off = align16(off + (uint32_t)(kMaxWaves * 16 * 2));
  pl->off_rp = off;
  off = align16(off + (uint32_t)((R + 1) * 4));
  pl->off_bias = off;
  off = align16(off + (uint32_t)(R * 4));
  pl->off_oprod = off;
  if (off > 163840) return false;
  // outlier products staged in LDS: up to kOj per thread, as many as the LDS left holds
  // (entries beyond that are read from the side tensor in the per-row phase)
  int ocap = outliers ? kOj * BD : 0;
  const int fit = (int)((163840 - off) / (uint32_t)(mt * 4));
  if (ocap > fit) ocap = fit;
  pl->ocap = ocap;
  off = align16(off + (uint32_t)(ocap * mt * 4));
  pl->lds_bytes = off;
  return off <= 163840;
}

static bool ptr_aligned(const void* p, int a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int gemv_launch(const spectra_qweight_t* w, const void* x, int64_t ldx, int m, int act_dtype, void* out,
                int64_t ldo, hipStream_t stream) {
  const bool outliers = w->outlier_kind == SPECTRA_OUTLIERS_COLUMNS ||
                        (w->outlier_kind == SPECTRA_OUTLIERS_CSR && w->csr_nnz > 0);
  GemvPlan pl;
  if (!plan_gemv(w->n, w->k, m, outliers, &pl))
    return fail(SPECTRA_ERR_UNSUPPORTED, "shape not served by the GEMV family (use the GEMM family)");
  SPECTRA_REQUIRE(w->hadamard_block == 0 || w->hadamard_block <= 512, "GEMV serves hadamard_block <= 512");
  SPECTRA_REQUIRE(ptr_aligned(x, 16) && ldx % 8 == 0, "x must be 16-byte aligned with a row stride multiple of 8");
  SPECTRA_REQUIRE(ptr_aligned(w->packed, 16) && w->packed_stride % 16 == 0,
                  "packed weights must be 16-byte aligned with a row stride multiple of 16");
  if (w->format == SPECTRA_FMT_NF4 && w->group_size < 32)
    return fail(SPECTRA_ERR_UNSUPPORTED, "the GEMV family needs an NF4 block of at least 32");
  GemvParams p;
  p.packed = w->packed; p.ldp = w->packed_stride;
  p.scales = w->scales; p.lds = w->scales_stride;
  p.zeros = w->zeros; p.ldz = w->zeros_stride;
  p.oidx = w->outlier_idx; p.ow = w->outlier_w; p.ldow = w->outlier_w_stride;
  p.rowptr = w->csr_rowptr; p.ccol = w->csr_col; p.cval = w->csr_val;
  p.bias = w->bias;
  p.x = x; p.ldx = ldx; p.out = out; p.ldo = ldo;
  p.n = (int)w->n; p.k = (int)w->k; p.m = m;
  int gs = 0;
  while ((1 << gs) < w->group_size) ++gs;
  p.gshift = gs;
  p.had = w->hadamard_block; p.marlin = w->marlin_layout ? 1 : 0;
  p.log_had = 0;
  while (p.log_had < 30 && (1 << p.log_had) < w->hadamard_block) ++p.log_had;
  p.okind = outliers ? w->outlier_kind : SPECTRA_OUTLIERS_NONE;
  p.n_out = w->num_outliers; p.ow_dt = w->outlier_w_dtype; p.bias_dt = w->bias_dtype; p.act_dt = act_dtype;
  p.R = pl.R; p.S = pl.S; p.G = pl.G; p.ocap = pl.ocap;
  p.off_xp = pl.off_xp; p.off_xsc = pl.off_xsc; p.off_part = pl.off_part; p.off_codes = pl.off_codes;
  p.off_rp = pl.off_rp; p.off_bias = pl.off_bias; p.off_oprod = pl.off_oprod;
  p.out_scale = w->hadamard_block ? (float)(1.0 / std::sqrt((double)w->hadamard_block)) : 1.0f;
  p.inv_n_out = w->num_outliers > 0 ? 1.0f / (float)w->num_outliers : 1.0f;
  gemv_fn fn = w->format == SPECTRA_FMT_NF4 ? pick_kernel<SPECTRA_FMT_NF4>(pl.mt, pl.rpw)
                                            : pick_kernel<SPECTRA_FMT_ASYM_G32>(pl.mt, pl.rpw);
  const int st = ensure_lds_limit((const void*)fn);
  if (st != SPECTRA_OK) return st;
  hipLaunchKernelGGL(fn, dim3(pl.grid), dim3(pl.BD), pl.lds_bytes, stream, p);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

}  // namespace spectra

extern "C" int spectra_w4a16_gemv(const spectra_qweight_t* w, const void* x, int64_t ldx, int32_t m,
                                  int32_t act_dtype, void* out, int64_t ldo, spectra_stream_t stream) {
  int st = spectra::validate_qweight(w);
  if (st != SPECTRA_OK) return st;
  SPECTRA_REQUIRE(x != nullptr && out != nullptr, "x/out is NULL");
  SPECTRA_REQUIRE(m >= 1 && m <= 4, "the GEMV family serves 1 <= m <= 4");
  SPECTRA_REQUIRE(act_dtype == SPECTRA_F16 || act_dtype == SPECTRA_BF16, "activations must be fp16 or bf16");
  SPECTRA_REQUIRE(ldx >= w->k && ldo >= w->n, "row stride too small");
  return spectra::gemv_launch(w, x, ldx, m, act_dtype, out, ldo, (hipStream_t)stream);
}
