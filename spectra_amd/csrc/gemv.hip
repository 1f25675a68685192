// Decode GEMV family for gfx950: out[m, :] = FWHT(x[m, :]) . W_eff^T + bias, m <= 4.
//
// Replaces the reference's single-row Triton GEMV (kernels.py:16-184).  Design:
//  * Workgroup = S x G waves.  S = ceil(K / 1024) K-slices; G row groups.  A wave owns
//    one slice (each lane 16 k = 8 packed bytes, one dwordx2) of RPW rows.  All weight
//    loads of a wave are issued up front, after the activation loads, so waiting for x
//    never waits for the weight stream (vmcnt is in issue order).
//  * Activations: each workgroup rotates x itself (blockwise FWHT in fp32, butterflies
//    across lanes with xor-shuffles), scales each row by a power of two so the largest
//    |x| lands in [2^14, 2^15), rounds to fp16 and stores the result in LDS in
//    "pair order" (the two k's of packed byte j side by side).
//  * Nibble decode: a 256-entry LUT in LDS maps a packed byte to the fp16 pair
//    (code[lo], code[hi]) -- NF4 levels for Format B, the integers 0..15 for Format A.
//    The table is replicated per lane (64 KB) so that lane l always reads bank l:
//    the LDS address is (byte << 8) | (lane << 2), built by one v_perm_b32.
//  * Math per packed byte: v_perm + ds_read_b32 + v_dot2_f32_f16.  The per-block scale
//    is applied once per 16 k: Format B acc * absmax; Format A (acc - z * sum(x)) * s.
//  * Lane partials of all rows are reduced across the wave with a transposed halving
//    reduction, slices are summed in a fixed order, outliers are added per row in
//    index order: the result is deterministic run to run.
#include <cmath>

#include "common.h"

namespace spectra {

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

constexpr int kRpwMax = 8;   // rows per wave held in registers
constexpr int kOj = 2;       // outlier entries per thread held in registers
constexpr int kLutBytes = 65536;
constexpr int kMaxWaves = 16;

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
  int had, marlin;
  int okind, n_out, ow_dt, bias_dt, act_dt;
  int R, S, G, xch, ocap;
  uint32_t off_xp, off_part, off_smax, off_rp, off_oprod;
  float had_div;
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

template <int FMT>
__device__ __forceinline__ uint32_t lut_entry(int v) {
  const int lo = v & 15, hi = v >> 4;
  if (FMT == SPECTRA_FMT_NF4) return (uint32_t)nf4_f16_bits(lo) | ((uint32_t)nf4_f16_bits(hi) << 16);
  return (uint32_t)f2h((float)lo) | ((uint32_t)f2h((float)hi) << 16);
}

__device__ __forceinline__ float pow2f(int e) {  // e in [-126, 127]
  return __builtin_bit_cast(float, (uint32_t)(e + 127) << 23);
}

// fp16 pair-order position of element k inside a row of xp
__device__ __forceinline__ int xp_pos(int k, int marlin) {
  return marlin ? ((((k >> 5) << 4) + (k & 15)) << 1) + ((k >> 4) & 1) : k;
}

template <int FMT, int MT, int RPW>
__global__ void __launch_bounds__(1024) gemv_kernel(const GemvParams p) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int XCH = MT < 2 ? 2 : 4;
  const int tid = threadIdx.x;
  const int BD = blockDim.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwaves = BD >> 6;
  const int s = wave % p.S, g = wave / p.S;
  const int r0 = blockIdx.x * p.R;
  const int Rw = min(p.R, p.n - r0);
  const int K = p.k;
  const int cpr = K >> 3;  // activation chunks of 8 elements per row

  // ---------------- (1) activation chunks, CSR row pointers, bias ----------------
  uint4 xr[XCH];
  bool xok[XCH];
#pragma unroll
  for (int j = 0; j < XCH; ++j) {
    const int c = tid + j * BD;
    const int mrow = c / cpr;
    xok[j] = (j < p.xch) && (mrow < p.m);
    const int64_t off = xok[j] ? (int64_t)mrow * p.ldx + (int64_t)(c - mrow * cpr) * 8 : 0;
    xr[j] = *(const uint4*)((const uint16_t*)p.x + off);
  }
  int rp_v = 0, e0 = 0, e1 = 0;
  if (p.okind == SPECTRA_OUTLIERS_CSR) {
    rp_v = p.rowptr[r0 + min(tid, Rw)];
    e0 = p.rowptr[r0];
    e1 = p.rowptr[r0 + Rw];
  }
  // raw bits only: converting here would make the compiler wait for this load (and,
  // vmcnt being in issue order, for everything issued before it)
  uint32_t bias_raw = 0;
  bool bias_ok = false;
  if (p.bias != nullptr) {
    const int r = tid % p.R;
    bias_ok = tid < p.R * MT && r < Rw;
    const int64_t bi = r0 + (bias_ok ? r : 0);
    if (p.bias_dt == SPECTRA_F32) bias_raw = ((const uint32_t*)p.bias)[bi];
    else bias_raw = ((const uint16_t*)p.bias)[bi];
  }

  // ---------------- (2) the weight stream: every row of this wave, up front ----------------
  const int kb = s * 1024 + lane * 16;  // first k of this lane
  const bool kvalid = kb < K;
  uint2 wq[RPW];
  uint16_t sc[RPW];
  uint8_t zq[RPW];
  bool wok[RPW];
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int rl = g + i * p.G;
    wok[i] = (rl < Rw) && kvalid;
    const int64_t row = r0 + (wok[i] ? rl : 0);
    const int kk = wok[i] ? kb : 0;
    wq[i] = *(const uint2*)(p.packed + row * p.ldp + (kk >> 1));
    sc[i] = p.scales[row * p.lds + (kk >> p.gshift)];
    if (FMT == SPECTRA_FMT_ASYM_G32) zq[i] = p.zeros[row * p.ldz + (kk >> 5)];
  }

  // ---------------- (3) nibble-pair LUT, replicated per lane ----------------
  {
    uint32_t* lut = (uint32_t*)smem;
    for (int w = tid; w < 256 * 16; w += BD) {
      const int v = w >> 4, cq = w & 15;
      const uint32_t e = lut_entry<FMT>(v);
      *(uint4*)(lut + v * 64 + cq * 4) = make_uint4(e, e, e, e);
    }
  }

  // ---------------- (4) blockwise FWHT of the activations (fp32) ----------------
  float xv[XCH][8];
  float lmax[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) lmax[m] = 0.0f;
#pragma unroll
  for (int j = 0; j < XCH; ++j) {
    const uint32_t u[4] = {xr[j].x, xr[j].y, xr[j].z, xr[j].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint16_t h = (uint16_t)(u[e >> 1] >> (16 * (e & 1)));
      xv[j][e] = xok[j] ? to_f32_16(h, p.act_dt) : 0.0f;
    }
    if (j < p.xch && p.had) {
      // butterfly stages h = 1, 2, 4 inside the chunk, then across lanes (compressor.py:34-39)
#pragma unroll
      for (int h = 1; h < 8; h <<= 1) {
        if (h < p.had) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            if ((e & h) == 0) {
              const float a = xv[j][e], b = xv[j][e + h];
              xv[j][e] = a + b;
              xv[j][e + h] = a - b;
            }
          }
        }
      }
      for (int h = 8; h < p.had; h <<= 1) {
        const int msk = h >> 3;
        const bool upper = (lane & msk) != 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float o = __shfl_xor(xv[j][e], msk, 64);
          xv[j][e] = upper ? (o - xv[j][e]) : (xv[j][e] + o);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[j][e] = xv[j][e] / p.had_div;
    }
    const int mrow = (tid + j * BD) / cpr;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m == mrow && xok[j]) {
#pragma unroll
        for (int e = 0; e < 8; ++e) lmax[m] = fmaxf(lmax[m], fabsf(xv[j][e]));
      }
    }
  }
  float* smaxw = (float*)(smem + p.off_smax);  // [MT][kMaxWaves]
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    float v = lmax[m];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    if (lane == 0) smaxw[m * kMaxWaves + wave] = v;
  }
  int32_t* rps = (int32_t*)(smem + p.off_rp);
  if (p.okind == SPECTRA_OUTLIERS_CSR && tid <= Rw) rps[tid] = rp_v;

  // ---------------- (5) outlier entries of this workgroup (consumed after the stream) ----------------
  // (raw bits again, one 32-bit register per value, consumed after the weight stream;
  // one branch-free load pair per entry: CSR reads col/val, dense columns read the low
  // dword of idx and the row's outlier weight)
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
      const int r = ei / n_out, jj = ei - r * n_out;
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

  __syncthreads();  // --- barrier 0: per-wave maxima, LUT

  // ---------------- (6) power-of-two row scale, fp16 activations in pair order ----------------
  int fexp[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    float mx = 0.0f;
    for (int w = 0; w < nwaves; ++w) mx = fmaxf(mx, smaxw[m * kMaxWaves + w]);
    const uint32_t bits = __builtin_bit_cast(uint32_t, mx);
    const int eb = (int)(bits >> 23);             // mx >= 0
    const int E = eb == 0 ? -126 : eb - 127;      // floor(log2(mx)) for normal mx
    int F = bits == 0 ? 0 : 14 - E;               // mx * 2^F in [2^14, 2^15)
    F = F < -126 ? -126 : (F > 126 ? 126 : F);
    fexp[m] = F;
  }
  uint16_t* xp = (uint16_t*)(smem + p.off_xp);
#pragma unroll
  for (int j = 0; j < XCH; ++j) {
    const int c = tid + j * BD;
    if (j < p.xch && c < MT * cpr) {
      const int mrow = c / cpr;
      int F = 0;
#pragma unroll
      for (int m = 0; m < MT; ++m) F = (m == mrow) ? fexp[m] : F;
      const float f = pow2f(F);
      const int kc = (c - mrow * cpr) * 8;
#pragma unroll
      for (int e = 0; e < 8; ++e) xp[mrow * K + xp_pos(kc + e, p.marlin)] = f2h(xv[j][e] * f);
    }
  }

  __syncthreads();  // --- barrier 1: xp ready

  // ---------------- (7) this lane's activation pairs ----------------
  uint32_t xpair[MT][8];
  float xsum[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const uint4* src = (const uint4*)(xp + m * K + (kvalid ? kb : 0));
    const uint4 a = src[0], b = src[1];
    xpair[m][0] = a.x; xpair[m][1] = a.y; xpair[m][2] = a.z; xpair[m][3] = a.w;
    xpair[m][4] = b.x; xpair[m][5] = b.y; xpair[m][6] = b.z; xpair[m][7] = b.w;
    xsum[m] = 0.0f;
    if (FMT == SPECTRA_FMT_ASYM_G32) {
#pragma unroll
      for (int q = 0; q < 8; ++q)
        xsum[m] += h2f((uint16_t)xpair[m][q]) + h2f((uint16_t)(xpair[m][q] >> 16));
    }
  }

  // ---------------- (8) the stream: LUT decode + dot2 per packed byte ----------------
  constexpr int V = RPW * MT;
  constexpr int VP = V <= 1 ? 1 : V <= 2 ? 2 : V <= 4 ? 4 : V <= 8 ? 8 : V <= 16 ? 16 : 32;
  float vals[VP];
#pragma unroll
  for (int q = 0; q < VP; ++q) vals[q] = 0.0f;
  const uint32_t lanebits = (uint32_t)lane << 2;
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
    const uint32_t wd[2] = {wq[i].x, wq[i].y};
#pragma unroll
    for (int b = 0; b < 8; ++b) {
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
      if (FMT == SPECTRA_FMT_ASYM_G32) v = (acc[m] - (float)zq[i] * xsum[m]) * sf;
      else v = acc[m] * sf;
      vals[i * MT + m] = wok[i] ? v : 0.0f;
    }
  }

  // ---------------- (9) transposed halving reduction across the wave ----------------
  int n_left = VP;
  int idx = 0;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    if (n_left > 1) {
      const int half = n_left >> 1;
      const bool upper = (lane & off) != 0;
#pragma unroll
      for (int q = 0; q < VP / 2; ++q) {
        if (q < half) {
          const float send = upper ? vals[q] : vals[q + half];
          const float keep = upper ? vals[q + half] : vals[q];
          vals[q] = keep + __shfl_xor(send, off, 64);
        }
      }
      if (upper) idx += half;
      n_left = half;
    } else {
      vals[0] += __shfl_xor(vals[0], off, 64);
    }
  }
  // lanes sharing idx now hold the same total; the lowest of them writes it
  constexpr int lowbits = 64 / VP;  // lanes per result group
  float* part = (float*)(smem + p.off_part);
  if ((lane & (lowbits - 1)) == 0 && idx < V) {
    const int i = idx / MT, m = idx - i * MT;
    const int rl = g + i * p.G;
    if (rl < Rw) part[(rl * p.S + s) * MT + m] = vals[0];
  }

  // ---------------- (10) outlier products (x taken from the same scaled fp16 row) ----------------
  float* oprod = (float*)(smem + p.off_oprod);
  const int odt = p.okind == SPECTRA_OUTLIERS_CSR ? SPECTRA_F16 : p.ow_dt;
#pragma unroll
  for (int jo = 0; jo < kOj; ++jo) {
    if (ook[jo]) {
      const int el = tid + jo * BD;  // workgroup-local entry index
      const int pos = xp_pos(ocol[jo], p.marlin);
      const float ov = to_f32_16((uint16_t)oraw[jo], odt);
#pragma unroll
      for (int m = 0; m < MT; ++m) oprod[el * MT + m] = ov * h2f(xp[m * K + pos]);
    }
  }

  __syncthreads();  // --- barrier 2: slice partials and outlier products

  // ---------------- (11) per-row totals ----------------
  for (int t = tid; t < p.R * MT; t += BD) {
    const int r = t % p.R, m = t / p.R;
    if (r >= Rw || m >= p.m) continue;
    float y = 0.0f;
    for (int ss = 0; ss < p.S; ++ss) y += part[(r * p.S + ss) * MT + m];
    if (p.okind != SPECTRA_OUTLIERS_NONE) {
      int lo, hi;
      if (p.okind == SPECTRA_OUTLIERS_CSR) {
        lo = rps[r] - e0;
        hi = rps[r + 1] - e0;
      } else {
        lo = r * p.n_out;
        hi = lo + p.n_out;
      }
      float os = 0.0f;
      for (int el = lo; el < hi; ++el) {
        if (el < p.ocap) {
          os += oprod[el * MT + m];
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
          os += val * h2f(xp[m * K + xp_pos(col, p.marlin)]);
        }
      }
      y += os;
    }
    int F = 0;
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) F = (mm == m) ? fexp[mm] : F;
    y = y * pow2f(-F);
    if (p.bias != nullptr && t == tid && bias_ok)
      y += p.bias_dt == SPECTRA_F32 ? __builtin_bit_cast(float, bias_raw) : to_f32_16((uint16_t)bias_raw, p.bias_dt);
    const int64_t oi = (int64_t)m * p.ldo + r0 + r;
    ((uint16_t*)p.out)[oi] = from_f32_16(y, p.act_dt);
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
    default: return gemv_kernel<FMT, MT, 8>;
  }
}

template <int FMT>
static gemv_fn pick_kernel(int mt, int rpw) {
  if (mt == 1) return pick_rpw<FMT, 1>(rpw);
  if (mt == 2) return pick_rpw<FMT, 2>(rpw);
  return pick_rpw<FMT, 4>(rpw);
}

static uint32_t align16(uint32_t v) { return (v + 15u) & ~15u; }

struct GemvPlan {
  int mt, S, G, rpw, R, BD, xch, grid, ocap;
  uint32_t off_xp, off_part, off_smax, off_rp, off_oprod, lds_bytes;
};

// returns false when the shape does not fit this kernel family
static bool plan_gemv(int64_t n, int64_t k, int m, bool outliers, GemvPlan* pl) {
  const int mt = m <= 1 ? 1 : (m <= 2 ? 2 : 4);
  if (m > 4 || k > 16384) return false;
  const int S = (int)((k + 1023) / 1024);
  const int gmax = kMaxWaves / S;
  const int64_t want = (n + 255) / 256;  // rows per workgroup for ~one workgroup per CU
  int G = (int)(want < gmax ? want : gmax);
  if (G < 1) G = 1;
  int rpw = (int)((want + G - 1) / G);
  rpw = rpw < 1 ? 1 : (rpw > kRpwMax ? kRpwMax : rpw);
  const int R = G * rpw;
  const int BD = 64 * S * G;
  const int xch_max = mt < 2 ? 2 : 4;
  const int64_t chunks = (int64_t)mt * (k / 8);
  const int xch = (int)((chunks + BD - 1) / BD);
  if (xch > xch_max) return false;
  if (R * mt > BD || R + 1 > BD) return false;
  pl->mt = mt; pl->S = S; pl->G = G; pl->rpw = rpw; pl->R = R; pl->BD = BD; pl->xch = xch;
  pl->grid = (int)((n + R - 1) / R);
  pl->ocap = outliers ? kOj * BD : 0;
  uint32_t off = kLutBytes;
  pl->off_xp = off;
  off = align16(off + (uint32_t)(mt * k * 2));
  pl->off_part = off;
  off = align16(off + (uint32_t)(R * S * mt * 4));
  pl->off_smax = off;
  off = align16(off + (uint32_t)(mt * kMaxWaves * 4));
  pl->off_rp = off;
  off = align16(off + (uint32_t)((R + 1) * 4));
  pl->off_oprod = off;
  off = align16(off + (uint32_t)(pl->ocap * mt * 4));
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
  SPECTRA_REQUIRE(ptr_aligned(w->packed, 8) && w->packed_stride % 8 == 0,
                  "packed weights must be 8-byte aligned with a row stride multiple of 8");
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
  p.okind = outliers ? w->outlier_kind : SPECTRA_OUTLIERS_NONE;
  p.n_out = w->num_outliers; p.ow_dt = w->outlier_w_dtype; p.bias_dt = w->bias_dtype; p.act_dt = act_dtype;
  p.R = pl.R; p.S = pl.S; p.G = pl.G; p.xch = pl.xch; p.ocap = pl.ocap;
  p.off_xp = pl.off_xp; p.off_part = pl.off_part; p.off_smax = pl.off_smax; p.off_rp = pl.off_rp;
  p.off_oprod = pl.off_oprod;
  p.had_div = w->hadamard_block ? (float)std::sqrt((double)w->hadamard_block) : 1.0f;
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
