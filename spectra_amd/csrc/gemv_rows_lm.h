// One-row decode GEMV for NF4 weights with many rows per CU (the lm_head: N = 128256): the
// row-owning kernel of gemv_rows.h run in passes.
//
// With one workgroup per CU the row kernel's plan holds R = ceil(N / CUs) rows per workgroup;
// past ~64 rows its lane groups run out of registers and waves.  Giving each workgroup a
// few dozen rows instead (thousands of workgroups, several rounds per CU) repeats the fixed
// work of a workgroup -- the activation loads, the 64 KB LUT, the rotation -- once per
// round.  Here one workgroup per CU does that work once and then streams its R rows in
// passes of 8 waves x RW rows (lane groups of G lanes owning RPG = 2 rows each, as in the
// row kernel; eight waves leave each 256 registers, enough for two passes' loads):
//
//  * pass P + 1's weight runs, block scales (one fp16 per run, read with the run: the LDS
//    holds no scales) and CSR extents (scalar loads) are issued when pass P starts, its CSR
//    entries once pass P's products are done (the extents have landed by then), so the
//    stream never waits for a pass boundary; two register buffers alternate;
//  * each pass: the run's activations read once for the group's rows, LUT decode and
//    v_dot2 per packed byte, the CSR outliers, the group sum, the store;
//  * the greedy pick (optional): each lane keeps the best key of the outputs it stored,
//    each wave merges its lanes' keys and makes one atomic max at the end, as the
//    multi-row kernel does (same slots, same key).
#pragma once

#include "gemv_kernel.h"  // argmax_key
#include "gemv_rows.h"

namespace spectra {

template <int G, int SPR, int RPG_>
struct LmBuf {
  static constexpr int RPG = RPG_, NS = SPR * RPG, RW = RPG * (64 / G);
  uint4 wq[NS];
  uint16_t am[NS];
  int sx[RW + 1];
  int ocol[RPG], e0[RPG], cnt[RPG];
  uint32_t oval[RPG];
};

constexpr int kLmWaves = 8;  // two waves per SIMD: 256 VGPRs each, room for two passes' loads

template <int G, int SPR, int RPG_, int XC, bool BF, int PRO>
__global__ void __launch_bounds__(64 * kLmWaves, 1) gemv_rows_lm_kernel(const RowsParams p, int R,
                                                                         unsigned long long* __restrict__ akey) {
  extern __shared__ __align__(16) uint8_t smem[];
  typedef LmBuf<G, SPR, RPG_> Buf;
  constexpr int RPG = Buf::RPG, NS = Buf::NS, RW = Buf::RW;
  asm volatile("" ::"s"(p.x), "s"(p.packed), "s"(p.ldp), "s"(p.absmax), "s"(p.lda), "s"(p.csr), "s"(p.rowptr),
               "s"(p.ccol), "s"(p.cval), "s"(p.n), "s"(p.k), "s"(p.W), "s"(R), "s"(akey));
  const int tid = threadIdx.x;
  const int W = p.W;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  RowsCtx c;
  c.tid = tid;
  c.lane = lane;
  c.wave = wave;
  c.W = W;
  c.K = p.k;
  c.Q = p.k >> 5;
  c.r0 = blockIdx.x * R;
  c.Rw = min(R, p.n - c.r0);
  c.gi = lane / G;
  c.li = lane % G;
  c.grow0 = 0;
  const int PR = W * RW;  // rows per pass
  const int npass = (c.Rw + PR - 1) / PR;
  const uint8_t* wbase = p.packed + (int64_t)c.r0 * p.ldp;
  const uint8_t* abase = (const uint8_t*)p.absmax + (int64_t)c.r0 * p.lda * 2;
  // ---- a pass's loads: weight runs, their block scales and the wave's CSR extents
  auto load_main = [&](Buf& b, int P) __attribute__((always_inline)) {
    const int base = P * PR + wave * RW;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int j = s / SPR, ch = s % SPR;
      const int row = base + c.gi * RPG + j;
      const uint32_t ro = row < c.Rw ? (uint32_t)row : 0u;
      const int run = ch * G + c.li;
      b.wq[s] = load_nt_u4(wbase + ro * (uint32_t)p.ldp + (uint32_t)run * 16u);
      b.am[s] = load_at<uint16_t>(abase, (ro * (uint32_t)p.lda + (uint32_t)((run * 32) >> p.gshift)) * 2u);
    }
    typedef const __attribute__((address_space(4))) int32_t* crp_t;
    const crp_t rpc = (crp_t)p.rowptr;
#pragma unroll
    for (int i = 0; i <= RW; ++i) b.sx[i] = p.csr ? rpc[c.r0 + min(base + i, c.Rw)] : 0;
  };
  // ---- a pass's CSR entries: lane li of row j stages entry e0 + li (dummy: entry 0)
  auto load_entries = [&](Buf& b, int P) __attribute__((always_inline)) {
    const int base = P * PR + wave * RW;
#pragma unroll
    for (int j = 0; j < RPG; ++j) {
      const int a = G == 32 ? ((lane >> 5) ? b.sx[RPG + j] : b.sx[j]) : b.sx[j];
      const int e = G == 32 ? ((lane >> 5) ? b.sx[RPG + j + 1] : b.sx[j + 1]) : b.sx[j + 1];  // (RW = 2 RPG)
      const bool live = base + c.gi * RPG + j < c.Rw;
      b.e0[j] = a;
      b.cnt[j] = live ? e - a : 0;
      const bool ok = p.csr && c.li < b.cnt[j];
      const uint32_t ei = ok ? (uint32_t)(a + c.li) : 0u;
      b.ocol[j] = p.csr ? load_at<int>(p.ccol, 4u * ei) : 0;
      b.oval[j] = p.csr ? load_at<uint16_t>(p.cval, 2u * ei) : 0u;
    }
  };
  // ---- producer loads (activation chunks; no scale staging: p.R is 0), pass 0's loads
  ProducerRegs<XC, PRO> pr;
  rows_producer_loads<XC, PRO>(p, c, wave, W, tid, pr);
  Buf b0, b1;
  load_main(b0, 0);
  // ---- LUT and rotated activations, then pass 0's entries
  build_pair_lut32<SPECTRA_FMT_NF4>(smem, wave, W, lane);
  rows_rotate<XC, BF, PRO>(p, c, smem, wave, W, tid, pr);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  load_entries(b0, 0);
  float inv = 1.0f;  // kProRms: rsqrt(mean(h^2) + eps)
  if constexpr (PRO == kProRms) {
    const float* ss = (const float*)(smem + p.off_ss);
    float t = 0.0f;
    for (int w = 0; w < W; ++w) t += ss[w];
    inv = 1.0f / sqrtf(t / (float)c.K + p.eps);
  }
  const uint32_t lanebits = (uint32_t)(lane & 31) << 2;
  const uint16_t* xp16 = (const uint16_t*)(smem + p.off_xp);
  const float* xsc = (const float*)(smem + p.off_xsc);
  constexpr int odt = BF ? SPECTRA_BF16 : SPECTRA_F16;
  unsigned long long best = 0ull;
  // ---- one pass: products, outliers, row totals, stores; `next` gets its entries once the
  //      products are done
  auto process = [&](Buf& b, int P, Buf& next, bool has_next) __attribute__((always_inline)) {
    float acc[RPG];
#pragma unroll
    for (int j = 0; j < RPG; ++j) acc[j] = 0.0f;
#pragma unroll
    for (int ch = 0; ch < SPR; ++ch) {
      const XRun xr = rows_xrun<G>(p, c, smem, ch);
#pragma unroll
      for (int j = 0; j < RPG; ++j) {
        const int s = j * SPR + ch;
        uint32_t dec[16];
        rows_decode(b.wq[s], lanebits, dec);
        float d = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e)
          d = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, dec[e]), __builtin_bit_cast(f16x2_t, xr.xpair[e]), d,
                                     false);
        acc[j] += d * (h2f(b.am[s]) * xr.xs);
      }
    }
    if (has_next) load_entries(next, P + 1);
    if (p.csr) {
#pragma unroll
      for (int j = 0; j < RPG; ++j) {
        int col = b.ocol[j];
        uint32_t ov = b.oval[j];
        asm volatile("" : "+v"(col), "+v"(ov)::"memory");  // consumed here, after the products
        if (c.li < b.cnt[j]) acc[j] += h2f((uint16_t)ov) * (h2f(xp16[xs_pos(col, p.marlin, c.Q)]) * xsc[col >> 7]);
        for (int el = G + c.li; el < b.cnt[j]; el += G) {  // rows of more than G entries (rare)
          const int cl = p.ccol[b.e0[j] + el];
          acc[j] += h2f(p.cval[b.e0[j] + el]) * (h2f(xp16[xs_pos(cl, p.marlin, c.Q)]) * xsc[cl >> 7]);
        }
      }
    }
    const int base = P * PR + wave * RW;
#pragma unroll
    for (int j = 0; j < RPG; ++j) {
      const float v = group_sum<G>(acc[j], lane);
      const int row = base + c.gi * RPG + j;
      if (c.li == 0 && row < c.Rw) {
        float y = v * p.out_scale;
        if constexpr (PRO == kProRms) y *= inv;
        const uint16_t o = from_f32_16(y, odt);
        ((uint16_t*)p.out)[c.r0 + row] = o;
        if (akey != nullptr) {
          const unsigned long long k = argmax_key(to_f32_16(o, odt), c.r0 + row);
          best = k > best ? k : best;
        }
      }
    }
  };
  for (int P = 0; P < npass; P += 2) {
    const bool h1 = P + 1 < npass;
    if (h1) load_main(b1, P + 1);
    process(b0, P, b1, h1);
    if (!h1) break;
    const bool h2 = P + 2 < npass;
    if (h2) load_main(b0, P + 2);
    process(b1, P + 1, b0, h2);
  }
  // ---- greedy pick: the wave's best key (group leaders: lanes 0 and, at G = 32, 32), one
  //      atomic max into the wave's slot
  if (akey != nullptr) {  // (uniform)
    unsigned long long kw = best;
    if constexpr (G == 32) {
      const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)best, 32);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(best >> 32), 32);
      const unsigned long long t = ((unsigned long long)hi << 32) | lo;
      kw = t > kw ? t : kw;
    }
    if (lane == 0 && kw != 0)
      __hip_atomic_fetch_max(akey + ((blockIdx.x * W + wave) & (SPECTRA_ARGMAX_SLOTS - 1)) * SPECTRA_ARGMAX_STRIDE, kw,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

typedef void (*gemv_rows_lm_fn)(const RowsParams, int, unsigned long long*);

// instantiated in gemv_rows_lm.hip: (G, SPR) = (32, 3) (K = 3072), (64, 1) (2048), (64, 2)
// (4096), two rows per lane group; fp16 or bf16 activations; no prologue or the fused
// RMSNorm.  (K = 8192 would need more registers than two passes of loads leave.)
gemv_rows_lm_fn gemv_rows_lm_pick(int g, int spr, bool bf, int pro);

}  // namespace spectra
