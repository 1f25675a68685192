// One-row decode GEMV for NF4 weights, stream-first:
//   out[0, :] = FWHT(x) . W_eff^T (+ CSR outliers, bias, residual), fp32 accumulation.
//
// Replaces the reference's single-row Triton GEMV (kernels.py:16-184) for Format B operands
// at M = 1, the decode hot path.  A launch is bound by HBM: the point of this design is that
// the weight stream starts as soon as the kernel arguments arrive and that little work is
// left after its last byte lands.
//
//  * Workgroup = W waves (W <= 16, one workgroup per CU), R rows of W, all of K.  K is cut in
//    P = K / 1024 pieces of 32 lanes x 32 k; half-wave h owns piece h % P of row group h / P
//    (RG = 2W / P row groups), so a lane streams one fixed 32-run q of every row
//    rg + RG i (slot i < NS): its 16 activation pairs stay in registers for all slots.
//  * Issue order per wave: the activation half-runs, every weight unit (one dwordx4 per slot),
//    the block scales, then the small tail operands (row pointers, bias, residual).  Nothing
//    ahead of the weights depends on a memory round trip.  The workgroup's CSR extent
//    [e0, e1) is loaded with the activations (ahead of the weights, so waiting for it never
//    waits for the stream); the CSR entries are issued after the activation rotation, behind
//    the weights, and consumed after the stream.
//  * While the weights are in flight: the 64 KB nibble-pair LUT is built from registers and
//    the activations are rotated once per workgroup (one half-run of 16 values per thread,
//    register stages plus DPP butterflies), scaled per 32-run by a power of two and stored as
//    fp16 pairs in LDS ([chunk][run] 16-byte units).
//  * Stream, per slot: 16 x (v_perm -> LDS LUT read -> v_dot2_f32_f16), then one multiply by
//    absmax * run scale.
//  * Tail: a transposed halving reduction over each half-wave (32 lanes), the piece partials
//    and the outlier products (entry value x rotated activation) to LDS, one barrier, then
//    16 lanes per row add the row's pieces and its outlier products in a fixed order:
//    deterministic run to run.
#pragma once

#include "gemv_kernel.h"

namespace spectra {

struct StreamParams {
  const uint8_t* packed;
  int64_t ldp;
  const uint16_t* absmax;
  int64_t lda;
  const int32_t* rowptr;
  const int32_t* ccol;
  const uint16_t* cval;
  const void* bias;
  const void* x;
  void* out;
  const uint16_t* nw;  // kProRms: RMSNorm weight fp16 [K]
  const void* res;     // optional residual [N] (act dtype, may alias out): out = res + out
  float eps;           // kProRms
  float out_scale;     // 1/sqrt(hadamard_block) (1 without rotation)
  int n, k;
  int W;               // waves per workgroup
  int R;               // rows per workgroup
  int P;               // 1024-k pieces per row
  int RG;              // row groups per slot (2W / P)
  int pmagic;          // ceil(65536 / P): h / P == (h * pmagic) >> 16 for h < 32
  int gshift;          // log2(NF4 block)
  int log_had, marlin;
  int csr;             // CSR outliers present (nnz > 0)
  int csr_nnz;
  int bias_dt;
  int ocap;            // outlier products staged in LDS
  int cpr;             // 16-byte chunks of absmax per row (K / block / 8)
  int cmagic;          // ceil(65536 / cpr): t / cpr == (t * cmagic) >> 16 for t < 1024
  uint32_t off_xp, off_xsc, off_part, off_rp, off_bias, off_res, off_ss, off_op, off_sc;
};

constexpr int kStreamMaxSlots = 8;
// slots decoded (LUT reads) before the activations are ready: their dot products need only
// the rotated activations after the barrier
#ifndef SPECTRA_STREAM_PREDECODE
#define SPECTRA_STREAM_PREDECODE 0
#endif
constexpr int kStreamPredecode = SPECTRA_STREAM_PREDECODE;
constexpr int kStreamOutlierLoads = 2;  // staged CSR entries per thread

// transposed halving reduction over lane-logical bits KB..4 (a half-wave of 32 lanes)
template <int N, int KB>
__device__ __forceinline__ void transposed_reduce32(float* vals, int lane, int lam, int& idx) {
  if constexpr (KB <= 4) {
    if constexpr (N > 1) {
      constexpr int H = N / 2;
      const bool upper = (lam >> KB) & 1;
#pragma unroll
      for (int q = 0; q < H; ++q) {
        const float send = upper ? vals[q] : vals[q + H];
        const float keep = upper ? vals[q + H] : vals[q];
        vals[q] = keep + lane_partner<KB>(send, lane);
      }
      if (upper) idx += H;
      transposed_reduce32<H, KB + 1>(vals, lane, lam, idx);
    } else {
      vals[0] += lane_partner<KB>(vals[0], lane);
      transposed_reduce32<1, KB + 1>(vals, lane, lam, idx);
    }
  }
}

// fp16 index of activation element k in the [chunk][run] pair layout (Q runs per row)
__device__ __forceinline__ int xs_pos(int k, int marlin, int Q) {
  const int q = k >> 5, e = k & 31;
  const int j = marlin ? (e & 15) : (e >> 1), half = marlin ? (e >> 4) : (e & 1);
  return (((j >> 2) * Q + q) * 4 + (j & 3)) * 2 + half;
}

// 16 bytes streamed once: a nontemporal load (no reuse expected in the caches)
__device__ __forceinline__ uint4 load_nt_u4(const uint8_t* p) {
  typedef uint32_t v4_t __attribute__((ext_vector_type(4)));
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load((const __attribute__((address_space(1))) v4_t*)p));
}

// fp16 pair (lo, hi) -> (lo + hi, lo - hi) in fp32: the conversion and the butterfly on
// element bit 0 in one v_fma_mix_f32 each (lo * 1 + (+-hi), rounded once: the fp32 sum)
__device__ __forceinline__ void fly0_from_f16(uint32_t u, float& a, float& b) {
  asm("v_fma_mix_f32 %0, %1, 1.0, %1 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(a) : "v"(u));
  asm("v_fma_mix_f32 %0, %1, 1.0, -%1 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(b) : "v"(u));
}

// fp16 pair (RNE(lo * f), RNE(hi * f)) in one dword: two v_fma_mix{lo,hi}_f16 (the product
// by a power of two is exact, so each value rounds once)
__device__ __forceinline__ uint32_t pack_scaled(float lo, float hi, float f) {
  uint32_t r;  // the low half is written first: the old high half is never used
  asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[0,0,0]" : "=v"(r) : "v"(lo), "v"(f));
  asm("v_fma_mixhi_f16 %0, %1, %2, 0 op_sel_hi:[0,0,0]" : "+v"(r) : "v"(hi), "v"(f));
  return r;
}

// fwht_half_t without its first stage (done by fly0_from_f16)
template <bool MAR>
__device__ __forceinline__ void fwht128_after0(float (&v)[16], int cl) {
  const auto sgn = [&](int kb) { return ((cl >> kb) & 1) ? -1.0f : 1.0f; };
  fly_in<1>(v);
  fly_in<2>(v);
  if constexpr (MAR) {
    fly_x<0>(v, sgn(0));
    fly_in<3>(v);
  } else {
    fly_in<3>(v);
    fly_x<0>(v, sgn(0));
  }
  fly_x<1>(v, sgn(1));
  fly_x<2>(v, sgn(2));
}

template <int NS, bool BF, int PRO>
__global__ void __launch_bounds__(1024, 1) gemv_stream_kernel(const StreamParams p) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int VP = NS <= 1 ? 1 : NS <= 2 ? 2 : NS <= 4 ? 4 : 8;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int T = 64 * p.W;
  const int K = p.k, Q = K >> 5;
  const int r0 = blockIdx.x * p.R;
  const int Rw = min(p.R, p.n - r0);
  // every argument the issue phase needs, fetched in one round trip before the first load
  asm volatile("" ::"s"(p.x), "s"(p.packed), "s"(p.ldp), "s"(p.absmax), "s"(p.lda), "s"(p.log_had), "s"(p.marlin),
               "s"(p.RG), "s"(p.pmagic), "s"(p.P), "s"(p.gshift), "s"(p.csr), "s"(p.rowptr), "s"(p.bias),
               "s"(p.res), "s"(p.bias_dt));

  // Wait counts: the compiler counts, for each load waited on, the loads issued after it; a
  // load under a condition is counted as absent, so a wait would then also cover it.  The
  // loads issued under per-wave or per-thread conditions therefore come first (they are
  // waited on only at the end), and every later load is issued by every wave, from a
  // dummy in-bounds address where the wave has nothing to load.

  // ---------------- (0) conditional loads: block scales and tail operands ----------------
  // the workgroup's block scales, 16 bytes per thread (row t / cpr, chunk t % cpr), staged in
  // LDS before the first barrier (rows past the workgroup's read row 0)
  const int srow = (tid * p.cmagic) >> 16;
  const bool sthr = tid < p.R * p.cpr;
  uint4 scv;
  if (wave * 64 < p.R * p.cpr) {
    const int sr = srow < Rw ? srow : 0;
    scv = load_at<uint4>(p.absmax + (int64_t)r0 * p.lda,
                         (uint32_t)(sr * p.lda) * 2u + (uint32_t)(tid - srow * p.cpr) * 16u);
  }
  // row pointers, bias and residual of the workgroup's rows (threads <= Rw: wave 0 when Rw < 64)
  const uint32_t ti = (uint32_t)(tid <= Rw ? tid : 0);
  int rp_v = 0;
  uint32_t bias_raw = 0;
  uint16_t res_raw = 0;
  if (wave * 64 <= Rw) {
    if (p.csr) rp_v = load_at<int>(p.rowptr + r0, 4u * ti);
    if (p.bias != nullptr) {
      const uint32_t bi = tid < Rw ? ti : 0u;
      if (p.bias_dt == SPECTRA_F32) bias_raw = load_at<uint32_t>((const uint32_t*)p.bias + r0, 4u * bi);
      else bias_raw = load_at<uint16_t>((const uint16_t*)p.bias + r0, 2u * bi);
    }
    if (p.res != nullptr) res_raw = load_at<uint16_t>((const uint16_t*)p.res + r0, 2u * (tid < Rw ? ti : 0u));
  }

  // ---------------- (1) activation half-runs (raw bits), every wave ----------------
  // half-run hd = tid of the K / 16; inside a Hadamard block of 2^bL lanes the lane holds
  // logical chunk reflect_chunk (bit 0 = which half of its 32-run); threads past the last
  // half-run read half-run 0 (discarded)
  const int hpr = K >> 4;  // a multiple of 64: whole waves take part or none
  const bool xwave = wave * 64 < hpr;
  const int bL = p.log_had >= 5 ? p.log_had - 4 : (p.marlin && p.log_had == 4 ? 1 : 0);
  const int bm = (1 << bL) - 1;
  const int cl = (tid & ~bm) | reflect_chunk(lane & bm, bL);
  const int xq = cl >> 1, xhf = cl & 1;
  uint4 xr[2], xu[PRO == kProSiluMul ? 2 : 1], nwv[PRO == kProRms ? 2 : 1];
  {
    const uint32_t xo = xwave ? (uint32_t)xq * 64u : 0u;
    const uint32_t o0 = 2u * (p.marlin ? 8 * xhf : 16 * xhf), o1 = 2u * (p.marlin ? 16 + 8 * xhf : 16 * xhf + 8);
    xr[0] = load_at<uint4>(p.x, xo + o0);
    xr[1] = load_at<uint4>(p.x, xo + o1);
    if constexpr (PRO == kProSiluMul) {
      xu[0] = load_at<uint4>(p.x, xo + 2u * K + o0);
      xu[1] = load_at<uint4>(p.x, xo + 2u * K + o1);
    }
    if constexpr (PRO == kProRms) {
      nwv[0] = load_at<uint4>(p.nw, xo + o0);
      nwv[1] = load_at<uint4>(p.nw, xo + o1);
    }
  }

  // this workgroup's CSR extent [e0, e1): lane 0 reads rowptr[r0], the others rowptr[r0 + Rw]
  // (without outliers: a word of the workgroup's own first weight row, unused -- dummy
  // addresses stay inside the workgroup's own data, so no line is read by every workgroup)
  const int rpe = load_at<int>(p.csr ? (const void*)(p.rowptr + r0) : (const void*)(p.packed + (int64_t)r0 * p.ldp),
                               p.csr ? (lane != 0 ? 4u * (uint32_t)Rw : 0u) : 4u * (uint32_t)lane);

  constexpr int PDC = NS < kStreamPredecode ? NS : (NS == 8 && kStreamPredecode > 4 ? 4 : kStreamPredecode);
  if constexpr (PDC > 0) {
    // ---------------- (3) nibble-pair LUT (from registers) ----------------
    // read while the weights arrive (pre-decode): every wave waits for it here, ahead of the
    // weight loads, where no wave is held up by a load issue yet
    build_pair_lut<SPECTRA_FMT_NF4>(smem, wave, p.W, lane);
    __syncthreads();
  }

  // ---------------- (2) the weight stream: every slot of this lane, up front ----------------
  const int h = tid >> 5;
  const int rg = (h * p.pmagic) >> 16;  // h / P
  const int q = (h - rg * p.P) * 32 + (tid & 31);  // this lane's 32-run, the same in every slot
  const uint8_t* wbase = p.packed + (int64_t)r0 * p.ldp;
  const uint32_t wstep = (uint32_t)(p.RG * p.ldp);
  const uint32_t w0 = (uint32_t)(rg * p.ldp) + (uint32_t)q * 16u;
  uint4 wq[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const bool ok = rg + p.RG * i < Rw;  // rows past the workgroup's read row r0 (discarded)
    wq[i] = load_nt_u4(wbase + (ok ? w0 + (uint32_t)i * wstep : (uint32_t)q * 16u));
  }


  if constexpr (PDC == 0) build_pair_lut<SPECTRA_FMT_NF4>(smem, wave, p.W, lane);  // read after barrier 1

  // ---------------- (4) activations: FWHT, run scale, fp16 pairs -> LDS ----------------
  uint4* xp4 = (uint4*)(smem + p.off_xp);
  float* xsc = (float*)(smem + p.off_xsc);
  float ssq = 0.0f;
  uint16_t* scl = (uint16_t*)(smem + p.off_sc);
  if (sthr) ((uint4*)scl)[tid] = scv;  // [R][K / block] fp16
  if (xwave) {
    float v[16];
    const uint32_t u[8] = {xr[0].x, xr[0].y, xr[0].z, xr[0].w, xr[1].x, xr[1].y, xr[1].z, xr[1].w};
    const bool mar = p.marlin != 0;
    const int xcl = cl & bm;
    // fp16 input rotated by 128: the first butterfly stage fused with the conversion
    const bool fused0 = !BF && PRO == kProNone && p.log_had == 7;
    if (fused0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) fly0_from_f16(u[e], v[2 * e], v[2 * e + 1]);
      if (mar) fwht128_after0<true>(v, xcl);
      else fwht128_after0<false>(v, xcl);
    } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if constexpr (BF) {
        v[2 * e] = __builtin_bit_cast(float, u[e] << 16);
        v[2 * e + 1] = __builtin_bit_cast(float, u[e] & 0xffff0000u);
      } else {
        v[2 * e] = h2f((uint16_t)u[e]);
        v[2 * e + 1] = h2f((uint16_t)(u[e] >> 16));
      }
    }
    if constexpr (PRO == kProSiluMul) {  // fp16(silu(g) * u), the silu_mul arithmetic
      const uint32_t uu[8] = {xu[0].x, xu[0].y, xu[0].z, xu[0].w, xu[1].x, xu[1].y, xu[1].z, xu[1].w};
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float g = v[e], uv = h2f((uint16_t)(uu[e >> 1] >> (16 * (e & 1))));
        v[e] = h2f(f2h(g / (1.0f + __expf(-g)) * uv));
      }
    }
    if constexpr (PRO == kProRms) {
#pragma unroll
      for (int e = 0; e < 16; ++e) ssq += v[e] * v[e];
      const uint32_t nw[8] = {nwv[0].x, nwv[0].y, nwv[0].z, nwv[0].w, nwv[1].x, nwv[1].y, nwv[1].z, nwv[1].w};
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] *= h2f((uint16_t)(nw[e >> 1] >> (16 * (e & 1))));
    }
    if (p.log_had == 7) {
      if (mar) fwht_half_t<7, true>(v, xcl);
      else fwht_half_t<7, false>(v, xcl);
    } else if (p.log_had != 0) {
      fwht_half(v, p.log_had, mar, xcl);
    }
    }
    float mx = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fabsf(v[r]));
    // the other half of the run: the partner across lane bit 0
    mx = fmaxf(mx, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, mx), 0xB1, 0xF, 0xF, false)));
    const uint32_t bits = __builtin_bit_cast(uint32_t, mx);
    const int eb = (int)(bits >> 23);
    const int E = eb == 0 ? -126 : eb - 127;  // floor(log2(mx)) for normal mx
    int F = bits == 0 ? 0 : 14 - E;           // mx * 2^F in [2^14, 2^15)
    F = F < -126 ? -126 : (F > 126 ? 126 : F);
    // the lane's butterfly sign rides on the (exact) power-of-two scale
    const float f = (__builtin_popcount(xcl) & 1) ? -pow2f(F) : pow2f(F);
    uint32_t d[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {  // pair jj of this half: plain (2jj, 2jj+1), marlin (jj, jj+8)
      const float lo = mar ? v[jj] : v[2 * jj], hi = mar ? v[jj + 8] : v[2 * jj + 1];
      d[jj] = pack_scaled(lo, hi, f);
    }
    // run xq's pairs 8 hf .. 8 hf + 7: chunks 2 hf and 2 hf + 1
    xp4[(2 * xhf) * Q + xq] = make_uint4(d[0], d[1], d[2], d[3]);
    xp4[(2 * xhf + 1) * Q + xq] = make_uint4(d[4], d[5], d[6], d[7]);
    if (xhf == 0) xsc[xq] = pow2f(-F);
  }
  if constexpr (PRO == kProRms) {  // per-wave sums of h^2, fixed order
    ssq = wave_sum(ssq);
    if (lane == 0) ((float*)(smem + p.off_ss))[wave] = ssq;
  }

  // ---------------- (5) this workgroup's CSR entries (behind the weights) ----------------
  // thread tid stages entries el = tid + T u (el = e - e0); arrays without entries, and
  // lanes past the staged range, read entry 0 of the packed tensor (discarded)
  const int e0 = p.csr ? __builtin_amdgcn_readlane(rpe, 0) : 0;
  const int cnt = p.csr ? __builtin_amdgcn_readlane(rpe, 1) - e0 : 0;
  int ocol[kStreamOutlierLoads];
  uint16_t oval[kStreamOutlierLoads];
  {
    // lanes past the staged entries re-read one of the workgroup's first 64 entries (or, without
    // entries, a word of its own first weight row)
    const int64_t wrow = (int64_t)r0 * p.ldp;
    const void* cb = p.csr ? (const void*)p.ccol : (const void*)(p.packed + wrow);
    const void* vb = p.csr ? (const void*)p.cval : (const void*)(p.packed + wrow);
    const int ostaged = min(cnt, p.ocap);
    const int elast = p.csr_nnz - 1;
#pragma unroll
    for (int u = 0; u < kStreamOutlierLoads; ++u) {
      const int el = tid + T * u;
      const uint32_t e = !p.csr ? (uint32_t)lane : el < ostaged ? (uint32_t)(e0 + el) : (uint32_t)min(e0 + lane, elast);
      ocol[u] = load_at<int>(cb, 4u * e);
      oval[u] = load_at<uint16_t>(vb, 2u * e);
    }
  }

  // ---------------- (5b) pre-decode: LUT reads of the first slots as their weights land ----------------
  // (at most 5, 4 with 8 slots: within 128 VGPRs)
  constexpr int PD = PDC;
  const uint32_t lanebits = (uint32_t)lane << 2;  // this lane's LUT copy: conflict-free reads
  const int rg_lo = __builtin_amdgcn_readlane(rg, 0), rg_hi = __builtin_amdgcn_readlane(rg, 32);
  uint32_t dec[PD > 0 ? PD : 1][16];
#pragma unroll
  for (int i = 0; i < PD; ++i) {
    if (min(rg_lo, rg_hi) + p.RG * i >= Rw) continue;  // slots with no row in either half-wave
    const uint32_t wd[4] = {wq[i].x, wq[i].y, wq[i].z, wq[i].w};
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      const uint32_t addr = __builtin_amdgcn_perm(wd[b >> 2], lanebits, 0x0c0c0000u | ((4u + (b & 3)) << 8));
      dec[i][b] = *(const __attribute__((address_space(3))) uint32_t*)(uintptr_t)addr;
    }
  }

  __syncthreads();  // --- barrier 1: activation pairs, run scales, block scales

  // ---------------- (6) this lane's activation pairs and run scale ----------------
  uint32_t xpair[16];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const uint4 a = xp4[c * Q + q];
    xpair[4 * c] = a.x; xpair[4 * c + 1] = a.y; xpair[4 * c + 2] = a.z; xpair[4 * c + 3] = a.w;
  }
  const float xs = xsc[q];

  // ---------------- (7) the stream: LUT decode + dot2 per packed byte ----------------
  float vals[VP];
#pragma unroll
  for (int i = 0; i < VP; ++i) vals[i] = 0.0f;
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    // slots where neither half-wave has a row are skipped (a wave-uniform branch)
    if (min(rg_lo, rg_hi) + p.RG * i >= Rw) continue;
    float acc = 0.0f;
    const uint32_t wd[4] = {wq[i].x, wq[i].y, wq[i].z, wq[i].w};
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      uint32_t code2;
      if (i < PD) {
        code2 = dec[i < PD ? i : 0][b];
      } else {
        const uint32_t addr = __builtin_amdgcn_perm(wd[b >> 2], lanebits, 0x0c0c0000u | ((4u + (b & 3)) << 8));
        // the LUT starts at LDS address 0 (the kernel has no static LDS; the host checks)
        code2 = *(const __attribute__((address_space(3))) uint32_t*)(uintptr_t)addr;
      }
      acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, code2), __builtin_bit_cast(f16x2_t, xpair[b]), acc,
                                   false);
    }
    const int rl = rg + p.RG * i;
    const float v = acc * (h2f(scl[(rl < Rw ? rl : 0) * (p.cpr * 8) + (q >> (p.gshift - 5))]) * xs);
    vals[i] = rl < Rw ? v : 0.0f;
  }

  // ---------------- (8) per half-wave totals of each slot ----------------
  int idx = 0;
  const int lam = reflect_chunk(lane & 15, 4) | (lane & 16);
  transposed_reduce32<VP, 0>(vals, lane, lam, idx);
  float* part = (float*)(smem + p.off_part);
  const int piece = q >> 5;
  if ((lam & 31) < VP && idx < NS) {
    const int rl = rg + p.RG * idx;
    if (rl < Rw) part[rl * p.P + piece] = vals[0];
  }

  // ---------------- (9) outlier products, row pointers, bias and residual to LDS ----------------
  float* oprod = (float*)(smem + p.off_op);
  const uint16_t* xp16 = (const uint16_t*)xp4;
#pragma unroll
  for (int u = 0; u < kStreamOutlierLoads; ++u) {
    const int el = tid + T * u;
    if (el < cnt && el < p.ocap) {
      const int col = ocol[u];
      oprod[el] = h2f(oval[u]) * (h2f(xp16[xs_pos(col, p.marlin, Q)]) * xsc[col >> 5]);
    }
  }
  int32_t* rps = (int32_t*)(smem + p.off_rp);
  if (p.csr && tid <= Rw) rps[tid] = rp_v;
  float* bl = (float*)(smem + p.off_bias);
  if (p.bias != nullptr && tid < Rw)
    bl[tid] = p.bias_dt == SPECTRA_F32 ? __builtin_bit_cast(float, bias_raw) : to_f32_16((uint16_t)bias_raw, p.bias_dt);
  uint16_t* rsl = (uint16_t*)(smem + p.off_res);
  if (p.res != nullptr && tid < Rw) rsl[tid] = res_raw;

  __syncthreads();  // --- barrier 2: piece partials and outlier products

  // ---------------- (10) per-row totals: 16 lanes per row, fixed order ----------------
  float inv = 1.0f;  // kProRms: rsqrt(mean(h^2) + eps)
  if constexpr (PRO == kProRms) {
    const float* ss = (const float*)(smem + p.off_ss);
    float t = 0.0f;
    for (int w = 0; w < p.W; ++w) t += ss[w];
    inv = 1.0f / sqrtf(t / (float)K + p.eps);
  }
  const int gl = tid & 15;
  for (int r = tid >> 4; r < Rw; r += 4 * p.W) {
    float v = gl < p.P ? part[r * p.P + gl] : 0.0f;
    if (p.csr) {
      const int lo = rps[r] - e0, hi = rps[r + 1] - e0;
      for (int el = lo + gl; el < hi; el += 16) {
        if (el < p.ocap) {
          v += oprod[el];
        } else {  // beyond the staged entries: read the side tensor directly
          const int col = p.ccol[e0 + el];
          v += h2f(p.cval[e0 + el]) * (h2f(xp16[xs_pos(col, p.marlin, Q)]) * xsc[col >> 5]);
        }
      }
    }
    v = row16_sum(v);
    if (gl == 0) {
      constexpr int odt = BF ? SPECTRA_BF16 : SPECTRA_F16;
      float y = v * p.out_scale;
      if constexpr (PRO == kProRms) y *= inv;
      if (p.bias != nullptr) y += bl[r];
      if (p.res != nullptr) y = to_f32_16(from_f32_16(y, odt), odt) + to_f32_16(rsl[r], odt);
      ((uint16_t*)p.out)[r0 + r] = from_f32_16(y, odt);
    }
  }
}

typedef void (*gemv_stream_fn)(const StreamParams);

gemv_stream_fn gemv_stream_pick_f16(int ns, int pro);
gemv_stream_fn gemv_stream_pick_bf16(int ns);

template <bool BF, int PRO>
gemv_stream_fn stream_pick_ns(int ns) {
  switch (ns) {
    case 1: return gemv_stream_kernel<1, BF, PRO>;
    case 2: return gemv_stream_kernel<2, BF, PRO>;
    case 3: return gemv_stream_kernel<3, BF, PRO>;
    case 4: return gemv_stream_kernel<4, BF, PRO>;
    case 5: return gemv_stream_kernel<5, BF, PRO>;
    case 6: return gemv_stream_kernel<6, BF, PRO>;
    case 7: return gemv_stream_kernel<7, BF, PRO>;
    default: return gemv_stream_kernel<8, BF, PRO>;
  }
}

}  // namespace spectra
