// Decode GEMV family for gfx950: out[m, :] = FWHT(x[m, :]) . W_eff^T + bias, m <= 4.
//
// Replaces the reference's single-row Triton GEMV (kernels.py:16-184).  Design:
//  * Workgroup = S x G waves (at most 8).  S = ceil(K / 2048) K-slices; G row groups.  A wave
//    owns one slice (each lane 32 k = 16 packed bytes, one dwordx4) of RPW rows.  All weight
//    loads of a wave are issued up front, after the activation loads, so waiting for x
//    never waits for the weight stream (vmcnt counts in issue order).
//  * VALU is the scarce resource while the stream is in flight, so every setup step is
//    sized per element, never per wave:
//    - activations: each thread owns half of a 32-element run of x (16 values), so every
//      wave shares the work: butterfly stages on register bits in registers, the stages
//      across lanes as one v_fmac_f32 with a DPP-permuted source per value (lanes of a
//      Hadamard block are numbered in a reflected order so that the quad permutes and
//      the half-row / row mirrors pair exactly the lanes each stage needs; the high side
//      of a cross-lane butterfly keeps the negated difference and the lane's sign is
//      applied with the run scale); the run is scaled by its own power of two
//      (max |x| -> [2^14, 2^15)), rounded to fp16 and stored in LDS in "pair order" (the
//      two k's of packed byte j side by side) with the run's inverse scale beside it; the
//      1/sqrt(block) normalisation is applied once per output.
//    - nibble decode: a 256-entry LUT in LDS maps a packed byte to the fp16 pair
//      (code[lo], code[hi]) -- NF4 levels for Format B, the integers 0..15 for Format A.
//      It is replicated per lane (64 KB) so that lane l always reads bank l: the LDS
//      address is (byte << 8) | (lane << 2), built by one v_perm_b32.  The waves fill it
//      from registers (the high code of a row group is wave-uniform), with no LDS reads.
//  * Math per packed byte: v_perm + ds_read_b32 + v_dot2_f32_f16.  Scales are applied once
//    per 32 k: Format B acc * absmax * run_scale; Format A (acc - z * sum(x)) * s * run_scale.
//  * Lane partials of all rows are reduced across the wave with a transposed halving
//    reduction; per-row totals (slices, outliers, bias) are reduced by one wave per row in
//    a fixed order: the result is deterministic run to run.
#pragma once

#include "common.h"

namespace spectra {

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

constexpr int kRpwMax = 11;  // rows per wave held in registers (<= 128 VGPRs: two 8-wave workgroups per CU)
constexpr int kLutBytes = 65536;
constexpr int kMaxWaves = 16;  // waves per workgroup: 8 (two per SIMD) or 16 (four per SIMD)
constexpr int kRpwWide = 6;    // rows per wave of the 16-wave kernels (<= 128 VGPRs)

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
  int csr_nnz;
  int R, S, G, ocap;
  int s_magic;      // ceil(256 / S): wave / S == (wave * s_magic) >> 8 for wave < 8
  uint32_t off_xp, off_xsc, off_part, off_rp, off_bias, off_oprod, off_ss, off_res;
  float out_scale;  // 1/sqrt(hadamard_block) (1 without rotation)
  float inv_n_out;  // 1/n_out (dense outlier columns)
  // fusions (kernels with PRO != 0 serve one fp16 row)
  const uint16_t* nw;  // PRO 2: RMSNorm weight fp16 [K]
  float eps;        // PRO 2
  const void* res;  // optional residual [m, N] (act dtype, may alias out): out = res + out
  int64_t ldr;
  unsigned long long* akey;  // optional (m = 1): greedy-pick slots, merged with an atomic max
};

// Greedy-pick key of an output: the value's order (NaN above every number, -0 == +0) in the
// high word, the complement of the index in the low word, so that the largest key is the
// largest value and, among equal values, the lowest index (torch.argmax's rule).  0 is
// below every key (the slots' empty state).
__device__ __forceinline__ unsigned long long argmax_key(float f, int idx) {
  uint32_t b = __builtin_bit_cast(uint32_t, f);
  uint32_t o;
  if (f != f) {
    o = 0xffffffffu;
  } else {
    if (f == 0.0f) b = 0u;
    o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  }
  return ((unsigned long long)o << 32) | (unsigned long long)(0xffffffffu - (uint32_t)idx);
}

// activation prologues fused into the GEMV
constexpr int kProNone = 0;     // x as given
constexpr int kProSiluMul = 1;  // x row = [g | u] (2K values): fp16(silu(g) * u)
constexpr int kProRms = 2;      // x = h: h * w_norm, times rsqrt(mean(h^2) + eps) in the epilogue

// Rows per wave of the one-row 8-wave kernels when two workgroups share a CU (large N):
// four waves per SIMD leave 128 VGPRs per wave, and these are the largest row counts that
// compile within that without spilling (the fused prologues and Format A's zero points
// hold more registers per row).  Those kernels are built for four waves per SIMD.
constexpr int gemv_rpw_two_per_cu(int fmt, int pro) {
  return fmt != SPECTRA_FMT_NF4 ? 8 : pro == kProRms ? 8 : pro == kProSiluMul ? 9 : kRpwMax;
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

// Value of the partner lane across lane-logical bit KB of the reduction's lane numbering
// lam = reflect_chunk(lane & 15, 4) | (lane & 48): DPP quad permutes for bits 0 and 1, the
// half-row and row mirrors for bits 2 and 3, and the VALU row swaps v_permlane16_swap
// (lane ^ 16) and v_permlane32_swap (lane ^ 32) for bits 4 and 5 -- no LDS traffic.
template <int KB>
__device__ __forceinline__ float lane_partner(float v, int lane) {
  const int iv = __builtin_bit_cast(int, v);
  if constexpr (KB == 0) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0xB1, 0xF, 0xF, false));
  else if constexpr (KB == 1) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x4E, 0xF, 0xF, false));
  else if constexpr (KB == 2) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x141, 0xF, 0xF, false));
  else if constexpr (KB == 3) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x140, 0xF, 0xF, false));
  else if constexpr (KB == 4) {  // (v, v) -> rows [v0 v0 v2 v2] / [v1 v1 v3 v3]
    const auto r = __builtin_amdgcn_permlane16_swap(iv, iv, false, false);
    return __builtin_bit_cast(float, (int)((lane & 16) ? r[0] : r[1]));
  } else {  // (v, v) -> halves [lo lo] / [hi hi]
    const auto r = __builtin_amdgcn_permlane32_swap(iv, iv, false, false);
    return __builtin_bit_cast(float, (int)((lane & 32) ? r[0] : r[1]));
  }
}

// Transposed halving reduction of N values per lane across the 64 lanes: at the step on
// lane-logical bit KB the lanes with that bit of lam set keep the upper half of their
// values and add their partner's upper half (the others the lower half), so N values
// cost N-1 exchanges instead of 6N.  Partners differ from each other only in bit KB of
// lam, so both hold the same value indices when they combine.  At the end every lane
// holds the total number idx, a bijection of the low log2(N) bits of lam.
template <int N, int KB>
__device__ __forceinline__ void transposed_reduce(float* vals, int lane, int lam, int& idx) {
  if constexpr (KB <= 5) {
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
      transposed_reduce<H, KB + 1>(vals, lane, lam, idx);
    } else {
      vals[0] += lane_partner<KB>(vals[0], lane);
      transposed_reduce<1, KB + 1>(vals, lane, lam, idx);
    }
  }
}

// Lane j of a Hadamard block of 2^b lanes holds logical chunk reflect_chunk(j, b):
// identity inside a quad, and for a top bit t >= 2 the chunk of the mirrored lane
// (2^(t+1) - 1 - j) with bit t set.  With this numbering lane-logical bit 0/1 pairs the
// lanes of DPP quad_perm [1,0,3,2] / [2,3,0,1], bit 2 the lanes of row_half_mirror, bit 3
// those of row_mirror, bit 4 those of a 32-lane mirror (j <-> 31 - j) and bit 5 those of
// the 64-lane mirror (j <-> 63 - j).
__device__ __forceinline__ int reflect_chunk(int j, int b) {
  int out = 0;
#pragma unroll
  for (int t = 5; t >= 2; --t) {
    if (t < b && ((j >> t) & 1)) {
      out |= 1 << t;
      j ^= (1 << t) - 1;
    }
    j &= (1 << t) - 1;
  }
  return out | j;
}

// Butterfly on register bit RB of the 16 values of a thread (stage pairs (u, v) ->
// (u + v, u - v), compressor.py:34-39).
template <int RB>
__device__ __forceinline__ void fly_in(float (&v)[16]) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    if ((r & (1 << RB)) == 0) {
      const float a = v[r], b = v[r | (1 << RB)];
      v[r] = a + b;
      v[r | (1 << RB)] = a - b;
    }
  }
}

#define SPECTRA_XFLY(CTRL)                                                                      \
  asm volatile("s_nop 1\n"                                                                      \
               "v_fmac_f32_dpp %0, %0, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"              \
               "v_fmac_f32_dpp %1, %1, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"              \
               "v_fmac_f32_dpp %2, %2, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"              \
               "v_fmac_f32_dpp %3, %3, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"              \
               "v_fmac_f32_dpp %4, %4, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"              \
               "v_fmac_f32_dpp %5, %5, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"              \
               "v_fmac_f32_dpp %6, %6, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"              \
               "v_fmac_f32_dpp %7, %7, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"              \
               "v_fmac_f32_dpp %8, %8, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"              \
               "v_fmac_f32_dpp %9, %9, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"              \
               "v_fmac_f32_dpp %10, %10, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"            \
               "v_fmac_f32_dpp %11, %11, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"            \
               "v_fmac_f32_dpp %12, %12, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"            \
               "v_fmac_f32_dpp %13, %13, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"            \
               "v_fmac_f32_dpp %14, %14, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"            \
               "v_fmac_f32_dpp %15, %15, %16 " CTRL " row_mask:0xf bank_mask:0xf\n"            \
               : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),        \
                 "+v"(v[6]), "+v"(v[7]), "+v"(v[8]), "+v"(v[9]), "+v"(v[10]), "+v"(v[11]),      \
                 "+v"(v[12]), "+v"(v[13]), "+v"(v[14]), "+v"(v[15])                             \
               : "v"(c))

// Butterfly across the lanes on lane-logical bit KB: v += c * v(partner) with c = +1 on
// the low side and -1 on the high side, which leaves u + v on the low side and
// -(u - v) on the high side (the product by +-1 is exact and the fma rounds once, as
// the reference's add/subtract does).  Partners carry equal signs before every stage
// (they differ only in bit KB), so the lane's sign after all stages is
// (-1)^popcount(chunk bits).  The DPP source needs two wait states after the VALU write
// that produced it: the s_nop 1 at the head of the block provides them.
template <int KB>
__device__ __forceinline__ void fly_x(float (&v)[16], float c) {
  if constexpr (KB == 0) SPECTRA_XFLY("quad_perm:[1,0,3,2]");
  else if constexpr (KB == 1) SPECTRA_XFLY("quad_perm:[2,3,0,1]");
  else if constexpr (KB == 2) SPECTRA_XFLY("row_half_mirror");
  else if constexpr (KB == 3) SPECTRA_XFLY("row_mirror");
  else {
#pragma unroll
    for (int r = 0; r < 16; ++r) {  // lane j <-> 31 - j: ds_swizzle xor 0x1F
      const float o = __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v[r]), 0x7C1F));
      v[r] = __builtin_fmaf(o, c, v[r]);
    }
  }
}

// fwht_half for a block size known at compile time: straight-line, no stage branches
template <int LOG, bool MAR>
__device__ __forceinline__ void fwht_half_t(float (&v)[16], int cl) {
  const auto sgn = [&](int kb) { return ((cl >> kb) & 1) ? -1.0f : 1.0f; };
  if constexpr (LOG > 0) fly_in<0>(v);
  if constexpr (LOG > 1) fly_in<1>(v);
  if constexpr (LOG > 2) fly_in<2>(v);
  if constexpr (MAR) {
    if constexpr (LOG > 3) fly_x<0>(v, sgn(0));
    if constexpr (LOG > 4) fly_in<3>(v);
  } else {
    if constexpr (LOG > 3) fly_in<3>(v);
    if constexpr (LOG > 4) fly_x<0>(v, sgn(0));
  }
  if constexpr (LOG > 5) fly_x<1>(v, sgn(1));
  if constexpr (LOG > 6) fly_x<2>(v, sgn(2));
  if constexpr (LOG > 7) fly_x<3>(v, sgn(3));
  if constexpr (LOG > 8) fly_x<4>(v, sgn(4));
}

// Blockwise FWHT (block 2^log_had) of the 16 values of a half-run, in the reference's
// stage order h = 1, 2, 4, ... (compressor.py:34-39).  Element e of the 32-run sits in
// register r of half `hf`: plain order e = 16 hf + r (stages h = 1..8 on register bits,
// h = 16 across the half pair); marlin order e = (r & 7) + 8 hf + 16 (r >> 3) (h = 1..4
// and 16 on register bits, h = 8 across the half pair).  h >= 32 runs across the lanes
// of the block.  `cl` is the lane's logical chunk inside its block (bit 0 = hf).
__device__ __forceinline__ void fwht_half(float (&v)[16], int log_had, bool marlin, int cl) {
  const auto sgn = [&](int kb) { return ((cl >> kb) & 1) ? -1.0f : 1.0f; };
  if (log_had > 0) fly_in<0>(v);
  if (log_had > 1) fly_in<1>(v);
  if (log_had > 2) fly_in<2>(v);
  if (marlin) {
    if (log_had > 3) fly_x<0>(v, sgn(0));
    if (log_had > 4) fly_in<3>(v);
  } else {
    if (log_had > 3) fly_in<3>(v);
    if (log_had > 4) fly_x<0>(v, sgn(0));
  }
  if (log_had > 5) fly_x<1>(v, sgn(1));
  if (log_had > 6) fly_x<2>(v, sgn(2));
  if (log_had > 7) fly_x<3>(v, sgn(3));
  if (log_had > 8) fly_x<4>(v, sgn(4));
}

// Sum over each 16-lane row with DPP only: quad permutes, then the half-row and row
// mirrors; every lane of the row ends with the row's total.
__device__ __forceinline__ float row16_sum(float v) {
  int t;
  t = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  v += __builtin_bit_cast(float, t);
  t = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  v += __builtin_bit_cast(float, t);
  t = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false);  // row_half_mirror
  v += __builtin_bit_cast(float, t);
  t = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false);  // row_mirror
  v += __builtin_bit_cast(float, t);
  return v;
}

// One-row 8-wave kernels run two workgroups per CU in the large-N plans: four waves per
// SIMD, i.e. at most 128 VGPRs (one more and the second workgroup no longer fits).
template <int FMT, int MT, int RPW, bool BF, int PRO = kProNone, int LB = 512>
__global__ void __launch_bounds__(LB, (MT == 1 && LB == 512 && RPW <= gemv_rpw_two_per_cu(FMT, PRO) ? 4 : 1))
    gemv_kernel(const GemvParams p) {
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int XH = 2 * MT;  // 16-element half-runs of activations per thread (at most)
  const int tid = threadIdx.x;
  const int BD = 64 * p.S * p.G;  // == blockDim.x (the launch uses S x G waves), without the implicit-argument load
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwaves = BD >> 6;
  const int g = (wave * p.s_magic) >> 8, s = wave - g * p.S;  // wave / S, wave % S
  const int r0 = blockIdx.x * p.R;
  const int Rw = min(p.R, p.n - r0);
  const int K = p.k;
  const int qpr = K >> 5;  // 32-element runs per activation row
  // every argument the prologue needs, fetched in one round trip before the first load
  asm volatile("" ::"s"(p.x), "s"(p.ldx), "s"(p.packed), "s"(p.ldp), "s"(p.scales), "s"(p.lds), "s"(p.m),
               "s"(p.gshift), "s"(p.log_had), "s"(p.marlin), "s"(p.zeros), "s"(p.ldz), "s"(p.rowptr), "s"(p.okind), "s"(p.bias), "s"(p.bias_dt));

  // One workgroup per CU (the 16-wave kernels): the outlier entries are loaded ahead of the
  // weights and their products formed right after barrier 1, while the weights are still
  // in flight.  Several workgroups per CU (8 waves): each would wait a round trip for its
  // row pointers before its weights, so there they are loaded behind the weights and the
  // products formed after the stream.
  constexpr bool kEarlyOutl = LB > 512;
  // this workgroup's CSR entries [e0, e1): scalar (constant-cache) loads, issued first so
  // that their latency overlaps the activation address arithmetic
  const bool has_o = p.okind != SPECTRA_OUTLIERS_NONE;
  int e0 = 0, e1 = 0;
  if constexpr (FMT == SPECTRA_FMT_NF4 && kEarlyOutl) {
    if (p.okind == SPECTRA_OUTLIERS_CSR) {
      const __attribute__((address_space(4))) int32_t* rpc = (const __attribute__((address_space(4))) int32_t*)p.rowptr;
      e0 = rpc[r0];
      e1 = rpc[r0 + Rw];
    }
  }

  // ---------------- (1) activation runs: raw bits, issued first ----------------
  // half-run hr = tid + i * BD of the MT x (K / 16) half-runs; inside a Hadamard block of
  // 2^bL lanes the lane holds logical chunk reflect_chunk (bit 0 = which half of its run)
  const int hpr = K >> 4;  // half-runs per activation row
  const int bL = p.log_had >= 5 ? p.log_had - 4 : (p.marlin && p.log_had == 4 ? 1 : 0);
  uint4 xr[XH][2];
  uint4 xu[PRO == kProSiluMul ? XH : 1][2];   // the u half of a fused gate_up row
  uint4 nwv[PRO == kProRms ? XH : 1][2];      // RMSNorm weights of the half-run (fp16)
  int xm[XH], xq[XH], xcl[XH], xhf[XH];
  const int bm = (1 << bL) - 1;
  // block offsets of every slot (BD, hpr) are multiples of 2^bL, so the reflected chunk
  // inside the block depends on the lane alone: computed once
  const int rc = reflect_chunk(lane & bm, bL);
#pragma unroll
  for (int i = 0; i < XH; ++i) {
    const int hd = tid + i * BD;
    int m = 0;
#pragma unroll
    for (int mm = 1; mm < MT; ++mm) m += hd >= mm * hpr ? 1 : 0;
    const int hrr = hd - m * hpr;
    const int cl = (hrr & ~bm) | rc;
    xm[i] = m;
    xq[i] = cl >> 1;
    xcl[i] = cl & bm;  // the bits of the cross-lane stages (their signs)
    const int hf = cl & 1;
    xhf[i] = hf;
    // padded rows (m >= p.m) and slots past the last half-run read row 0: finite values
    // whose results are never stored
    const bool ok = hd < MT * hpr && m < p.m;
    // byte offset from the uniform base (the host keeps x within 2^31 bytes)
    const uint32_t xo = ok ? (uint32_t)(m * p.ldx + (cl >> 1) * 32) * 2u : 0u;
    // waves with no half-run in this slot skip its loads (a wave-uniform branch; the
    // loads come before every other load, so later wait counts are unaffected)
    // (left undefined otherwise: those values are never read, and no copy or wait is
    // needed where the branch joins)
    if (i == 0 || wave * 64 + i * BD < MT * hpr) {
      const uint32_t o0 = 2u * (p.marlin ? 8 * hf : 16 * hf), o1 = 2u * (p.marlin ? 16 + 8 * hf : 16 * hf + 8);
      xr[i][0] = load_at<uint4>(p.x, xo + o0);
      xr[i][1] = load_at<uint4>(p.x, xo + o1);
      if constexpr (PRO == kProSiluMul) {
        xu[i][0] = load_at<uint4>(p.x, xo + 2u * K + o0);
        xu[i][1] = load_at<uint4>(p.x, xo + 2u * K + o1);
      }
      if constexpr (PRO == kProRms) {
        const uint32_t no = ok ? (uint32_t)(cl >> 1) * 64u : 0u;
        nwv[i][0] = load_at<uint4>(p.nw, no + o0);
        nwv[i][1] = load_at<uint4>(p.nw, no + o1);
      }
    }
  }

  // row pointers through the vector path (lane 0 the first, lane 1 the last), issued before
  // the weights (the 8-wave kernels)
  int rpe = 0;
  if constexpr (FMT == SPECTRA_FMT_NF4 && !kEarlyOutl)
    rpe = p.okind == SPECTRA_OUTLIERS_CSR ? load_at<int>(p.rowptr + r0, lane == 1 ? 4u * Rw : 0u)
                                          : load_at<int>(p.packed, 0u);
  int olim = 0;
  int4 ocv;
  uint2 ovv;
  int obase = 0;  // el of this thread's first entry
  // ---------------- (1b) outlier entries of this workgroup ----------------
  // Raw loaded words only (extracted where they are used, so nothing here waits for
  // them), one unconditional load pair per thread (the wait counts never branch):
  //  * Format B, CSR: four consecutive entries from the 4-aligned entry below e0 (a
  //    dwordx4 of columns, a dwordx2 of fp16 values; entry e is el = e - e0).  The
  //    entries of a partial last group of the array are read in the per-row phase.
  //  * Format A, dense columns: entry el = tid, row el / n_out, column el % n_out (the
  //    low dword of the int64 index, the 16-bit weight).
  // Without outliers the loads read the first bytes of the packed tensor.  Entries
  // el < olim have their products staged in LDS; the rest (beyond the LDS share, or in a
  // partial last CSR group) are read from the side tensors per row.
  auto load_outliers = [&]() __attribute__((always_inline)) {
  if constexpr (FMT == SPECTRA_FMT_NF4 && !kEarlyOutl) {
    e0 = has_o ? __builtin_amdgcn_readlane(rpe, 0) : 0;
    e1 = has_o ? __builtin_amdgcn_readlane(rpe, 1) : 0;
  }
  olim = FMT == SPECTRA_FMT_NF4 ? min(p.ocap, (p.csr_nnz & ~3) - e0) : p.ocap;
  if constexpr (FMT == SPECTRA_FMT_NF4) {
    const int g0 = e0 & ~3, g4 = g0 + 4 * tid;
    // groups past this workgroup's entries (or the array end) re-read the first group (the
    // workgroup's own, or the array's when that one is partial), a cached line, so the
    // stream carries no CSR bytes beyond the workgroup's own
    // (arrays of fewer than 4 entries are never read this way: olim is 0 then)
    const bool big = has_o && p.csr_nnz >= 4;
    const bool ok4 = big && g4 < e1 && g4 + 4 <= p.csr_nnz;
    const int gb = big && g0 + 4 <= p.csr_nnz ? g0 : 0;  // wave-uniform base group
    // one load each, from a wave-uniform base (selected in scalar registers)
    const void* cbase = big ? (const void*)(p.ccol + gb) : (const void*)p.packed;
    const void* vbase = big ? (const void*)(p.cval + gb) : (const void*)p.packed;
    const uint32_t eo = ok4 ? (uint32_t)(g4 - gb) : 0u;
    ocv = load_at<int4>(cbase, 4u * eo);
    ovv = load_at<uint2>(vbase, 2u * eo);
    obase = g4 - e0;
  } else {
    const int n_out = p.n_out > 0 ? p.n_out : 1;
    // (row, column) of entry tid: float reciprocal, exact after one correction
    const int ei = tid < Rw * n_out ? tid : 0;
    int r = (int)((float)ei * p.inv_n_out);
    int jj = ei - r * n_out;
    r = jj < 0 ? r - 1 : (jj >= n_out ? r + 1 : r);
    jj = ei - r * n_out;
    ocv.x = has_o ? load_at<int>(p.oidx, 8u * (uint32_t)jj) : load_at<int>(p.packed, 0u);
    ovv.x = has_o ? load_at<uint16_t>((const uint16_t*)p.ow + (int64_t)r0 * p.ldow, 2u * (uint32_t)(r * p.ldow + jj))
                  : load_at<uint16_t>(p.packed, 0u);
    obase = tid;
  }
  };
  if constexpr (kEarlyOutl) load_outliers();

  // ---------------- (2) the weight stream: every row of this wave, up front ----------------
  const int kb = s * 2048 + lane * 32;  // first k of this lane (one 32-run)
  const bool kvalid = kb < K;
  constexpr int RP2 = (RPW + 1) / 2;
  uint4 wq[RPW];
  uint32_t sc[RPW];   // one scale per row (blocks of 32)
  uint16_t sc2[RP2];  // two rows per load (blocks of 64 and more)
  uint8_t zq[RPW];
  bool wok[RPW];
  const int kk = kvalid ? kb : 0;
  // Every address below is a wave-uniform row base (scalar arithmetic) plus one 32-bit
  // per-lane byte offset shared by all rows: no per-lane 64-bit address math per load.
  const uint32_t wo = (uint32_t)(kk >> 1);
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    const int rl = g + i * p.G;
    const bool rok = rl < Rw;
    wok[i] = rok && kvalid;
    const int64_t row = r0 + (rok ? rl : 0);
    wq[i] = load_at<uint4>(p.packed + row * p.ldp, wo);
    if (FMT == SPECTRA_FMT_ASYM_G32) zq[i] = load_at<uint8_t>(p.zeros + row * p.ldz, (uint32_t)(kk >> 5));
  }
  // Scales after the weights.  With blocks of 64 or more, lanes 2j and 2j+1 share a
  // block: one load serves rows 2t (even lanes) and 2t+1 (odd lanes), and a DPP quad
  // broadcast hands each lane its row's value (in the stream).
  constexpr bool pair_sc = FMT == SPECTRA_FMT_NF4;  // the host serves NF4 blocks >= 64 only
  const uint32_t so = (uint32_t)(kk >> p.gshift) * 2u;
  if constexpr (pair_sc) {
    const uint16_t* sbase = p.scales + (int64_t)r0 * p.lds;
    const bool odd = lane & 1;
#pragma unroll
    for (int t = 0; t < RP2; ++t) {
      const int ie = 2 * t, io = 2 * t + 1 < RPW ? 2 * t + 1 : 2 * t;
      const int rle = g + ie * p.G, rlo = g + io * p.G;
      const uint32_t oe = __builtin_amdgcn_readfirstlane((uint32_t)((rle < Rw ? rle : 0) * p.lds) * 2u);
      const uint32_t oo = __builtin_amdgcn_readfirstlane((uint32_t)((rlo < Rw ? rlo : 0) * p.lds) * 2u);
      sc2[t] = load_at<uint16_t>(sbase, (odd ? oo : oe) + so);
    }
  } else {
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int rl = g + i * p.G;
      const int64_t row = r0 + (rl < Rw ? rl : 0);
      sc[i] = load_at<uint16_t>(p.scales + row * p.lds, so);
    }
  }

  // ---------------- (2b) row pointers and bias: consumed after the stream ----------------
  int rp_v = 0;  // row pointers of this workgroup's rows, for the per-row phase
  if (p.okind == SPECTRA_OUTLIERS_CSR) rp_v = load_at<int>(p.rowptr + r0, 4u * (uint32_t)min(tid, Rw));
  uint32_t bias_raw = 0;
  if (p.bias != nullptr) {
    const uint32_t bi = (uint32_t)(tid < Rw ? tid : 0);
    if (p.bias_dt == SPECTRA_F32) bias_raw = load_at<uint32_t>((const uint32_t*)p.bias + r0, 4u * bi);
    else bias_raw = load_at<uint16_t>((const uint16_t*)p.bias + r0, 2u * bi);
  }
  // residual of output (row tid / Rw, column r0 + tid % Rw), read before any output is written
  uint16_t res_raw = 0;
  if (p.res != nullptr) {
    const int mm = tid / Rw, rr = tid - mm * Rw;
    res_raw = ((const uint16_t*)p.res)[mm < p.m ? (int64_t)mm * p.ldr + r0 + rr : 0];
  }

  // ---------------- (3) nibble-pair LUT (from registers, no LDS reads) ----------------
  build_pair_lut<FMT>(smem, wave, nwaves, lane);

  // ---------------- (4) activation half-runs: FWHT, run scale, fp16 pairs -> LDS ----------------
  uint16_t* xp = (uint16_t*)(smem + p.off_xp);
  const int XS = ((K + 2047) >> 11) << 11;  // xp row stride: whole 2048-element slices
  float* xsc = (float*)(smem + p.off_xsc);
  float ssq = 0.0f;  // PRO kProRms: sum of h^2 over this thread's half-runs
#pragma unroll
  for (int i = 0; i < XH; ++i) {
    // wave-uniform guard: the cross-lane stages need every lane of the wave
    if (wave * 64 + i * BD >= MT * hpr) break;
    float v[16];
    const uint32_t u[8] = {xr[i][0].x, xr[i][0].y, xr[i][0].z, xr[i][0].w,
                           xr[i][1].x, xr[i][1].y, xr[i][1].z, xr[i][1].w};
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
      const uint32_t uu[8] = {xu[i][0].x, xu[i][0].y, xu[i][0].z, xu[i][0].w,
                              xu[i][1].x, xu[i][1].y, xu[i][1].z, xu[i][1].w};
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float g = v[e], u = h2f((uint16_t)(uu[e >> 1] >> (16 * (e & 1))));
        v[e] = h2f(f2h(g / (1.0f + __expf(-g)) * u));
      }
    }
    if constexpr (PRO == kProRms) {
      if (tid + i * BD < MT * hpr) {
#pragma unroll
        for (int e = 0; e < 16; ++e) ssq += v[e] * v[e];
      }
      const uint32_t nw[8] = {nwv[i][0].x, nwv[i][0].y, nwv[i][0].z, nwv[i][0].w,
                              nwv[i][1].x, nwv[i][1].y, nwv[i][1].z, nwv[i][1].w};
#pragma unroll
      for (int e = 0; e < 16; ++e) v[e] *= h2f((uint16_t)(nw[e >> 1] >> (16 * (e & 1))));
    }
    const bool mar = p.marlin != 0;
    // straight-line code for the common blocks (none, 128), stage branches otherwise
    if (p.log_had == 7) {
      if (mar) fwht_half_t<7, true>(v, xcl[i]);
      else fwht_half_t<7, false>(v, xcl[i]);
    } else if (p.log_had != 0) {
      fwht_half(v, p.log_had, mar, xcl[i]);
    }
    float mx = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fabsf(v[r]));
    mx = fmaxf(mx, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, mx), 0xB1, 0xF, 0xF,
                                                                       false)));  // the other half of the run
    const uint32_t bits = __builtin_bit_cast(uint32_t, mx);
    const int eb = (int)(bits >> 23);
    const int E = eb == 0 ? -126 : eb - 127;   // floor(log2(mx)) for normal mx
    int F = bits == 0 ? 0 : 14 - E;            // mx * 2^F in [2^14, 2^15)
    F = F < -126 ? -126 : (F > 126 ? 126 : F);
    // the lane's butterfly sign rides on the (exact) power-of-two scale
    const float f = (__builtin_popcount(xcl[i]) & 1) ? -pow2f(F) : pow2f(F);
    uint32_t d[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // pair j of this half: plain (2j, 2j+1), marlin (j, j+8)
      const float lo = mar ? v[j] : v[2 * j], hi = mar ? v[j + 8] : v[2 * j + 1];
      d[j] = (uint32_t)f2h(lo * f) | ((uint32_t)f2h(hi * f) << 16);
    }
    if (tid + i * BD < MT * hpr) {
      // run q is consumed by lane q % 64 of slice q / 64: 4 16-byte chunks at
      // [m][slice][chunk][lane] (each ds_read_b128 of the stream reads 1 KB contiguous);
      // half hf of the run owns chunks 2 hf and 2 hf + 1
      const int q = xq[i], hf = xhf[i];
      uint4* dst = (uint4*)(xp + xm[i] * XS) + ((q >> 6) * 4 + 2 * hf) * 64 + (q & 63);
      dst[0] = make_uint4(d[0], d[1], d[2], d[3]);
      dst[64] = make_uint4(d[4], d[5], d[6], d[7]);
      if (hf == 0) xsc[xm[i] * qpr + q] = pow2f(-F);
    }
  }

  if constexpr (!kEarlyOutl) load_outliers();

  if constexpr (PRO == kProRms) {  // per-wave sums of h^2, fixed order
    ssq = wave_sum(ssq);
    if (lane == 0) ((float*)(smem + p.off_ss))[wave] = ssq;
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

  // ---------------- (6b) outlier products, in the same scaled fp16 activation basis ----------------
  // (before the stream in the 16-wave kernels, after it in the others)
  float* oprod = (float*)(smem + p.off_oprod);
  auto outlier_products = [&]() __attribute__((always_inline)) {
  {
    const int cnt = !has_o ? 0 : (FMT == SPECTRA_FMT_NF4 ? e1 - e0 : Rw * p.n_out);
    const int odt = FMT == SPECTRA_FMT_NF4 ? SPECTRA_F16 : p.ow_dt;
    constexpr int NE = FMT == SPECTRA_FMT_NF4 ? 4 : 1;
    const int cols[4] = {ocv.x, ocv.y, ocv.z, ocv.w};
    const uint32_t vals4[4] = {ovv.x & 0xffffu, ovv.x >> 16, ovv.y & 0xffffu, ovv.y >> 16};
#pragma unroll
    for (int u = 0; u < NE; ++u) {
      const int el = obase + u;  // workgroup-local entry index
      if (el >= 0 && el < cnt && el < olim) {
        const int col = cols[u];
        const int pos = xp_pos(col, p.marlin);
        const float ov = to_f32_16((uint16_t)vals4[u], odt);
#pragma unroll
        for (int m = 0; m < MT; ++m)
          oprod[el * MT + m] = ov * (h2f(xp[m * XS + pos]) * xsc[m * qpr + (col >> 5)]);
      }
    }
  }
  };
  if constexpr (kEarlyOutl) outlier_products();

  // ---------------- (7) the stream: LUT decode + dot2 per packed byte ----------------
  constexpr int V = RPW * MT;
  constexpr int VP = V <= 1 ? 1 : V <= 2 ? 2 : V <= 4 ? 4 : V <= 8 ? 8 : V <= 16 ? 16 : V <= 32 ? 32 : 64;
  float vals[VP];
#pragma unroll
  for (int q = 0; q < VP; ++q) vals[q] = 0.0f;
  const uint32_t lanebits = (uint32_t)lane << 2;  // this lane's LUT copy: conflict-free reads
#pragma unroll
  for (int i = 0; i < RPW; ++i) {
    // the plan may leave the last row of some waves empty (R < G x RPW): the 16-wave kernels
    // skip its decode (a wave-uniform branch; in the 8-wave kernels with more rows the branch
    // costs spills, so there the row is decoded and zeroed)
    if (LB > 512 && i == RPW - 1 && g + i * p.G >= Rw) {
#pragma unroll
      for (int m = 0; m < MT; ++m) vals[i * MT + m] = 0.0f;
      continue;
    }
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.0f;
    const uint32_t wd[4] = {wq[i].x, wq[i].y, wq[i].z, wq[i].w};
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      const uint32_t addr = __builtin_amdgcn_perm(wd[b >> 2], lanebits, 0x0c0c0000u | ((4u + (b & 3)) << 8));
      // the LUT starts at LDS address 0 (the kernel has no static LDS; the host checks)
      const uint32_t code2 = *(const __attribute__((address_space(3))) uint32_t*)(uintptr_t)addr;
#pragma unroll
      for (int m = 0; m < MT; ++m)
        acc[m] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, code2),
                                        __builtin_bit_cast(f16x2_t, xpair[m][b]), acc[m], false);
    }
    // quad_perm [0,0,2,2] / [1,1,3,3]: the even / odd lane of each pair
    // the empty asm pins the use here: no conversion of a scale can be hoisted above the
    // barrier, where it would wait for the whole stream
    uint16_t spr = sc2[i >> 1];
    asm volatile("" : "+v"(spr));
    const int sp = (int)spr;
    const uint32_t sw = !pair_sc ? sc[i]
                                 : (uint32_t)((i & 1) ? __builtin_amdgcn_mov_dpp(sp, 0xF5, 0xF, 0xF, false)
                                                      : __builtin_amdgcn_mov_dpp(sp, 0xA0, 0xF, 0xF, false));
    const float sf = h2f((uint16_t)sw);
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
  const int lam = reflect_chunk(lane & 15, 4) | (lane & 48);
  transposed_reduce<VP, 0>(vals, lane, lam, idx);
  // every lane now holds the total number idx (set by the low log2(VP) bits of lam); the
  // lanes with lam < VP write them
  float* part = (float*)(smem + p.off_part);
  if (lam < VP && idx < V) {
    const int i = idx / MT, m = idx - i * MT;
    const int rl = g + i * p.G;
    if (rl < Rw) part[(rl * p.S + s) * MT + m] = vals[0];
  }

  if constexpr (!kEarlyOutl) outlier_products();
  int32_t* rps = (int32_t*)(smem + p.off_rp);
  if (p.okind == SPECTRA_OUTLIERS_CSR && tid <= Rw) rps[tid] = rp_v;
  float* bl = (float*)(smem + p.off_bias);
  if (p.bias != nullptr && tid < Rw)
    bl[tid] = p.bias_dt == SPECTRA_F32 ? __builtin_bit_cast(float, bias_raw) : to_f32_16((uint16_t)bias_raw, p.bias_dt);
  uint16_t* rl = (uint16_t*)(smem + p.off_res);
  if (p.res != nullptr && tid < Rw * p.m) rl[tid] = res_raw;

  __syncthreads();  // --- barrier 2: slice partials and outlier products

  // ---------------- (10) per-row totals: 16 lanes per row, four rows per wave per pass ----------------
  // fixed order (deterministic): lane gl of a group takes slice gl and outlier entries
  // gl, gl + 16, ... of its row, then a DPP tree sums the 16 lanes
  unsigned long long best_key = 0;  // (11): this lane's greedy pick
  {
    float inv = 1.0f;  // PRO kProRms: rsqrt(mean(h^2) + eps) of the row
    if constexpr (PRO == kProRms) {
      const float* ss = (const float*)(smem + p.off_ss);
      float t = 0.0f;
      for (int w = 0; w < nwaves; ++w) t += ss[w];
      inv = 1.0f / sqrtf(t / (float)K + p.eps);
    }
    const int grp = lane >> 4, gl = lane & 15;
    for (int rb = wave * 4; rb < Rw; rb += nwaves * 4) {
      const int r = rb + grp;
      const bool rv = r < Rw;
      const int rr = rv ? r : Rw - 1;  // groups past the last row compute but do not store
      int lo = 0, hi = 0;
      if (p.okind == SPECTRA_OUTLIERS_CSR) {
        lo = rps[rr] - e0;
        hi = rps[rr + 1] - e0;
      } else if (p.okind == SPECTRA_OUTLIERS_COLUMNS) {
        lo = rr * p.n_out;
        hi = lo + p.n_out;
      }
      if (!rv) hi = lo;
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m >= p.m) break;
        float v = (gl < p.S && rv) ? part[(rr * p.S + gl) * MT + m] : 0.0f;
        // staged entries gl, gl + 16, gl + 32, gl + 48 of the row: four reads issued together
        // (in-bounds dummy index otherwise: the plan always holds one staged entry)
        float o[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int el = lo + gl + 16 * u;
          const bool st = el < hi && el < olim;
          const float t = oprod[(st ? el : 0) * MT + m];
          o[u] = st ? t : 0.0f;
        }
        v += (o[0] + o[1]) + (o[2] + o[3]);
        // the rest: entries past the first 64 of the row, and any not staged in LDS
        for (int el = lo + gl; el < hi; el += 16) {
          if (el < lo + 64 && el < olim) continue;
          if (el < olim) {
            v += oprod[el * MT + m];
          } else {  // beyond the staged entries: read the side tensor directly
            int col;
            float val;
            if (p.okind == SPECTRA_OUTLIERS_CSR) {
              col = p.ccol[e0 + el];
              val = h2f(p.cval[e0 + el]);
            } else {
              const int rw = el / p.n_out, jj = el - rw * p.n_out;
              col = (int)p.oidx[jj];
              val = load_elem(p.ow, (int64_t)(r0 + rw) * p.ldow + jj, p.ow_dt);
            }
            v += val * (h2f(xp[m * XS + xp_pos(col, p.marlin)]) * xsc[m * qpr + (col >> 5)]);
          }
        }
        v = row16_sum(v);
        if (gl == 0 && rv) {
          constexpr int odt = BF ? SPECTRA_BF16 : SPECTRA_F16;
          float y = v * p.out_scale;
          if constexpr (PRO == kProRms) y *= inv;
          if (p.bias != nullptr) y += bl[rr];
          if (p.res != nullptr) y = to_f32_16(from_f32_16(y, odt), odt) + to_f32_16(rl[m * Rw + rr], odt);
          const uint16_t yo = from_f32_16(y, odt);
          ((uint16_t*)p.out)[(int64_t)m * p.ldo + r0 + rr] = yo;
          if (m == 0) {  // greedy pick of the stored value
            const unsigned long long kk = argmax_key(to_f32_16(yo, odt), r0 + rr);
            best_key = kk > best_key ? kk : best_key;
          }
        }
      }
    }
  }
  // ---------------- (11) greedy pick: one atomic max per wave, no barrier ----------------
  // (the keys sit in lanes 0, 16, 32, 48: the groups' store lanes)
  if (p.akey != nullptr) {  // (uniform)
    unsigned long long kw = best_key;
#pragma unroll
    for (int l = 16; l < 64; l += 16) {
      const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)best_key, l);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(best_key >> 32), l);
      const unsigned long long t = ((unsigned long long)hi << 32) | lo;
      kw = t > kw ? t : kw;
    }
    if (lane == 0 && kw != 0)
      __hip_atomic_fetch_max(p.akey + ((blockIdx.x * nwaves + wave) & (SPECTRA_ARGMAX_SLOTS - 1)) * SPECTRA_ARGMAX_STRIDE,
                             kw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------
// kernel selection (instantiated per activation dtype in gemv_f16.hip / gemv_bf16.hip)
// ---------------------------------------------------------------------------
typedef void (*gemv_fn)(const GemvParams);

// wide: the 16-wave kernels (one activation row, rpw <= kRpwWide)
gemv_fn gemv_pick_f16(int fmt, int mt, int rpw, bool wide);
gemv_fn gemv_pick_bf16(int fmt, int mt, int rpw, bool wide);
gemv_fn gemv_pick_f16_pro(int pro, int rpw, bool wide);  // one fp16 row, NF4, fused prologue


template <int FMT, int MT, bool BF>
gemv_fn pick_rpw(int rpw) {
  switch (rpw) {
    case 1: return gemv_kernel<FMT, MT, 1, BF>;
    case 2: return gemv_kernel<FMT, MT, 2, BF>;
    case 3: return gemv_kernel<FMT, MT, 3, BF>;
    case 4: return gemv_kernel<FMT, MT, 4, BF>;
    case 5: return gemv_kernel<FMT, MT, 5, BF>;
    case 6: return gemv_kernel<FMT, MT, 6, BF>;
    case 7: return gemv_kernel<FMT, MT, 7, BF>;
    case 8: return gemv_kernel<FMT, MT, 8, BF>;
    case 9: return gemv_kernel<FMT, MT, 9, BF>;
    case 10: return gemv_kernel<FMT, MT, 10, BF>;
    default: return gemv_kernel<FMT, MT, 11, BF>;
  }
}

// one-row fp16 NF4 kernels with a fused prologue
template <int PRO>
gemv_fn pick_pro_rpw(int rpw) {
  switch (rpw) {
    case 1: return gemv_kernel<SPECTRA_FMT_NF4, 1, 1, false, PRO>;
    case 2: return gemv_kernel<SPECTRA_FMT_NF4, 1, 2, false, PRO>;
    case 3: return gemv_kernel<SPECTRA_FMT_NF4, 1, 3, false, PRO>;
    case 4: return gemv_kernel<SPECTRA_FMT_NF4, 1, 4, false, PRO>;
    case 5: return gemv_kernel<SPECTRA_FMT_NF4, 1, 5, false, PRO>;
    case 6: return gemv_kernel<SPECTRA_FMT_NF4, 1, 6, false, PRO>;
    case 7: return gemv_kernel<SPECTRA_FMT_NF4, 1, 7, false, PRO>;
    case 8: return gemv_kernel<SPECTRA_FMT_NF4, 1, 8, false, PRO>;
    case 9: return gemv_kernel<SPECTRA_FMT_NF4, 1, 9, false, PRO>;
    case 10: return gemv_kernel<SPECTRA_FMT_NF4, 1, 10, false, PRO>;
    default: return gemv_kernel<SPECTRA_FMT_NF4, 1, 11, false, PRO>;
  }
}

template <int FMT, bool BF>
gemv_fn pick_rpw4(int rpw) {
  switch (rpw) {
    case 1: return gemv_kernel<FMT, 4, 1, BF>;
    case 2: return gemv_kernel<FMT, 4, 2, BF>;
    case 3: return gemv_kernel<FMT, 4, 3, BF>;
    case 4: return gemv_kernel<FMT, 4, 4, BF>;
    case 5: return gemv_kernel<FMT, 4, 5, BF>;
    case 6: return gemv_kernel<FMT, 4, 6, BF>;
    case 7: return gemv_kernel<FMT, 4, 7, BF>;
    default: return gemv_kernel<FMT, 4, 8, BF>;
  }
}

// 16-wave kernels (launch bound 1024: four waves per SIMD)
template <int FMT, bool BF, int PRO>
gemv_fn pick_wide(int rpw) {
  switch (rpw) {
    case 1: return gemv_kernel<FMT, 1, 1, BF, PRO, 1024>;
    case 2: return gemv_kernel<FMT, 1, 2, BF, PRO, 1024>;
    case 3: return gemv_kernel<FMT, 1, 3, BF, PRO, 1024>;
    case 4: return gemv_kernel<FMT, 1, 4, BF, PRO, 1024>;
    case 5: return gemv_kernel<FMT, 1, 5, BF, PRO, 1024>;
    default: return gemv_kernel<FMT, 1, 6, BF, PRO, 1024>;
  }
}

template <int FMT, bool BF>
gemv_fn pick_kernel(int mt, int rpw, bool wide) {
  if (wide) return pick_wide<FMT, BF, kProNone>(rpw);
  if (mt == 1) return pick_rpw<FMT, 1, BF>(rpw);
  if (mt == 2) return pick_rpw<FMT, 2, BF>(rpw);
  return pick_rpw4<FMT, BF>(rpw);
}

}  // namespace spectra
