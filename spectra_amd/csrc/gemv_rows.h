// Decode GEMV for NF4 weights, rows owned by lane groups, one to four activation rows:
//   out[m, :] = FWHT_128(x[m]) . W_eff^T (+ CSR outliers, bias, residual), fp32 accumulation.
//
// Replaces the reference's single-row Triton GEMV (kernels.py:16-184) for Format B operands
// at M = 1 with a Hadamard block of 128 (or none), the decode hot path, and its small-batch
// path (kernels.py:191-389 at M = 2 .. 4, no prologue): each weight slot is
// decoded once for the MR rows, and each row's rotated activations get an LDS slot of
// their own.  A launch is bound
// by HBM, and what keeps it from the bound is work that cannot overlap the weight stream:
// the rotated activations must exist before the first dot product, and every cross-wave
// reduction after the last byte lands is on the critical path.  This design keeps both
// short.
//
//  * A lane group (G = 64 lanes, or 32 when K / 1024 is odd) owns RPG whole rows: slot
//    s = j * SPR + c streams the 16-byte run c * G + li of row j, so a row's dot product
//    never leaves its group.  The tail is one in-group butterfly sum per row, with no
//    cross-wave reduction and no per-row phase.
//  * The activations are rotated on the matrix cores: with H_128 = H_4 (x) H_32, a chunk of
//    512 values (16 sub-blocks of 32) times H_32 is two v_mfma_f32_16x16x32 (columns of
//    H_32 in the pair order the packed bytes use), and the H_4 factor combines the four
//    sub-blocks of a 128-block that the MFMA output leaves in one lane.  Without rotation
//    the same MFMAs multiply by a permutation (exact), so one code path serves both.
//    Each 128-block gets a power-of-two scale (max |x| -> [2^14, 2^15)) before the fp16
//    packing; the scale is exact and undone per slot.
//  * Roles (SPLIT): the waves past the row waves are producers.  They issue the
//    activation chunks and the staging loads (block scales, bias, residual) before a
//    start barrier, so those requests sit ahead of every weight request in the CU's memory
//    queue; after it they build the nibble-pair LUT, rotate the chunks, stage the scales
//    and count themselves done on an LDS counter.  The row waves issue their weight runs
//    right after the barrier, then the CSR entries of their rows (extents from scalar
//    loads issued at entry), and wait on the counter before the first dot product.  A row
//    wave held in its load issue (the CU's memory queue fills while the weights stream)
//    holds up nobody else, which a second workgroup barrier would.  The wait is bounded
//    (a counter that never completes gives wrong output, never a hang).
//    Without spare waves (!SPLIT) every wave does both jobs: loads first, then the
//    producer work, then a barrier.
//  * Every wait on a weight run is exact and never covers a later load: the loads under
//    per-thread conditions come first, every later load is issued by every lane of the
//    path (dummy in-bounds addresses where a lane has nothing to load).
//  * Decode: the 256-entry nibble-pair LUT in LDS in 32 copies (lane l reads bank l & 31;
//    the LDS serves the two 32-lane halves of a read in turn, so no conflicts), one
//    v_perm + ds_read_b32 + v_dot2_f32_f16 per packed byte.
#pragma once

#include <type_traits>

#include "gemv_stream.h"  // shared helpers: load_nt_u4, pack_scaled, xs_pos

namespace spectra {

struct RowsParams {
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
  float out_scale;     // 1/sqrt(128) with rotation, 1 without
  int n, k;
  int R;               // rows per workgroup
  int nchunk;          // K / 512
  int gshift;          // log2(NF4 block), >= 5
  int had;             // 128 or 0
  int marlin;
  int csr;             // CSR outliers present (nnz > 0)
  int csr_nnz;
  int bias_dt;
  int cpr;             // 16-byte absmax chunks per row (K / block / 8)
  int cmagic;          // ceil(65536 / cpr): t / cpr == (t * cmagic) >> 16 for t < 1024
  int wr;              // row waves (waves wr .. W-1 are producers when split)
  int W;               // waves per workgroup (blockDim.x / 64, passed so the kernel reads no implicit argument)
  uint32_t off_xp, off_xsc, off_sc, off_ss, off_bias, off_res;
  // several activation rows (MR > 1): row m of x at x + m ldx, of out at out + m ldo
  // (elements); its rotated pairs and block scales at off_xp + m xp_row, off_xsc + m xsc_row
  // (the residual's rows ldr apart, read by the row waves themselves)
  int64_t ldx, ldo, ldr;
  uint32_t xp_row, xsc_row;
};

constexpr int kRowsSpinLimit = 1 << 20;  // s_sleep rounds a row wave waits for the producers, at most
// LDS byte offset of the producers' counters (at most 5): the unused upper half of the nibble-pair
// LUT's first 256-byte row (the 32 copies fill bytes 0..127 of each row), a constant so
// that zeroing them waits for no kernel argument
constexpr uint32_t kRowsCounterOff = 128;

typedef _Float16 rh8_t __attribute__((ext_vector_type(8)));
typedef __bf16 rb8_t __attribute__((ext_vector_type(8)));
typedef float rf4_t __attribute__((ext_vector_type(4)));

// Max over each 16-lane row with DPP only (every lane of the row ends with the row's max).
__device__ __forceinline__ float row16_max(float v) {
  int t;
  t = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  v = fmaxf(v, __builtin_bit_cast(float, t));
  t = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  v = fmaxf(v, __builtin_bit_cast(float, t));
  t = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false);  // row_half_mirror
  v = fmaxf(v, __builtin_bit_cast(float, t));
  t = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false);  // row_mirror
  return fmaxf(v, __builtin_bit_cast(float, t));
}

// Sum over a lane group of G lanes (32: a half-wave, 64: the wave), same value in every lane.
template <int G>
__device__ __forceinline__ float group_sum(float v, int lane) {
  if constexpr (G == 64) v += lane_xor<32>(v, lane);
  v += lane_xor<16>(v, lane);
  v += lane_xor<8>(v, lane);
  v += lane_xor<4>(v, lane);
  v += lane_xor<2>(v, lane);
  return v + lane_xor<1>(v, lane);
}

// ---------------------------------------------------------------------------
// the kernel's phases (forced inline: the registers they hand over stay in registers)
// ---------------------------------------------------------------------------
struct RowsCtx {
  int tid, lane, wave, W, K, Q, r0, Rw, gi, li, grow0;
};

// producer loads: the activation chunks pw + np i (lane (i, g) = (lane & 15, lane >> 4)
// holds elements 32 i + 8 g .. + 7 of the chunk, the MFMA A operand; chunks past the last
// read chunk 0), then the workgroup's block scales (one 16-byte chunk per producer thread
// below R * cpr), bias and residual (producer threads below Rw)
template <int XC, int PRO>
struct ProducerRegs {
  uint4 scv;
  uint32_t bias_raw = 0;
  uint16_t res_raw = 0;
  uint4 xr[XC], xu[PRO == kProSiluMul ? XC : 1], nwr[PRO == kProRms ? XC : 1];
};

// the activation chunks of one row (x: its first element)
template <int XC, int PRO>
__device__ __forceinline__ void rows_producer_xloads(const RowsParams& p, const RowsCtx& c, const void* x, int pw,
                                                     int np, ProducerRegs<XC, PRO>& r) {
  const uint32_t xlo = 64u * (uint32_t)(c.lane & 15) + 16u * (uint32_t)(c.lane >> 4);
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int ch = pw + np * i;
    const uint32_t o = (ch < p.nchunk ? (uint32_t)ch * 1024u : 0u) + xlo;
    r.xr[i] = load_at<uint4>(x, o);
    if constexpr (PRO == kProSiluMul) r.xu[i] = load_at<uint4>(x, o + 2u * (uint32_t)c.K);
    if constexpr (PRO == kProRms) r.nwr[i] = load_at<uint4>(p.nw, o);
  }
}

// the workgroup's block scales, bias and residual (producer threads)
template <int XC, int PRO>
__device__ __forceinline__ void rows_producer_sloads(const RowsParams& p, const RowsCtx& c, int pw, int ptid,
                                                     ProducerRegs<XC, PRO>& r) {
  const int srow = (ptid * p.cmagic) >> 16;  // ptid / cpr
  if (pw * 64 < p.R * p.cpr) {
    const int sr = srow < c.Rw ? srow : 0;
    r.scv = load_at<uint4>(p.absmax + (int64_t)c.r0 * p.lda,
                           (uint32_t)(sr * p.lda) * 2u + (uint32_t)(ptid - srow * p.cpr) * 16u);
  }
  if (pw * 64 < c.Rw) {
    const uint32_t ti = (uint32_t)(ptid < c.Rw ? ptid : 0);
    if (p.bias != nullptr) {
      if (p.bias_dt == SPECTRA_F32) r.bias_raw = load_at<uint32_t>((const uint32_t*)p.bias + c.r0, 4u * ti);
      else r.bias_raw = load_at<uint16_t>((const uint16_t*)p.bias + c.r0, 2u * ti);
    }
    if (p.res != nullptr) r.res_raw = load_at<uint16_t>((const uint16_t*)p.res + c.r0, 2u * ti);
  }
}

template <int XC, int PRO>
__device__ __forceinline__ void rows_producer_loads(const RowsParams& p, const RowsCtx& c, int pw, int np, int ptid,
                                                    ProducerRegs<XC, PRO>& r) {
  // the activation chunks first: the rotation waits for them, and a wait counts every load
  // issued before the one it waits for (the block scales below come from HBM, cold)
  rows_producer_xloads<XC, PRO>(p, c, p.x, pw, np, r);
  rows_producer_sloads<XC, PRO>(p, c, pw, ptid, r);
}

// producer work after the LUT: the rotated chunks as fp16 pairs with one power-of-two scale
// per 128-block, block scales (fp32), bias, residual, RMSNorm partials
// (activation row m: its pairs and scales into row m's LDS slots; row 0 also stages the block
// scales, bias, residual and the RMSNorm partials)
// RM (several rows, one chunk per wave): chain t is activation row t of chunk pw (its
// pairs and scales into row t's slots), the chains interleaved as the chunks are
template <int XC, bool BF, int PRO, bool RM = false>
__device__ __forceinline__ void rows_rotate(const RowsParams& p, const RowsCtx& c, uint8_t* smem, int pw, int np,
                                             int ptid, const ProducerRegs<XC, PRO>& r, int m = 0) {
  static_assert(!RM || PRO == kProNone, "rows mode: no prologue");
  uint32_t* xpd = (uint32_t*)(smem + p.off_xp + (uint32_t)m * p.xp_row);  // [pair / 4][run][pair % 4] dwords
  float* xsc = (float*)(smem + p.off_xsc + (uint32_t)m * p.xsc_row);       // one scale per 128-block
  const int lane = c.lane, Q = c.Q;
  // B operands: column j of MFMA 1 / 2 is H_32 column (or unit column) pi1(j) / pi2(j),
  // the low / high position of packed pair j (marlin: j, j + 16; plain: 2 j, 2 j + 1)
  const int jj = lane & 15, g = lane >> 4;
  const int pi1 = p.marlin ? jj : 2 * jj;
  const uint32_t one = BF ? 0x3f80u : 0x3c00u;
  uint32_t b1[4], b2[4];
  if (p.had) {
    // sign of H_32[8 g + t][pi] = parity(g & pi >> 3) ^ parity(t & pi & 7): the byte of
    // Walsh row pi & 7 over t, complemented when the high parity is odd
    uint32_t w8 = (uint32_t)(0x963c5af066ccaa00ull >> (8 * (pi1 & 7))) & 0xffu;
    if (__builtin_popcount(g & (pi1 >> 3)) & 1) w8 ^= 0xffu;
#pragma unroll
    for (int t2 = 0; t2 < 4; ++t2)
      b1[t2] = (one | (one << 16)) | (((w8 >> (2 * t2)) & 1u) << 15) | (((w8 >> (2 * t2 + 1)) & 1u) << 31);
    // pi2 = pi1 + 16 (marlin: flips with bit 4 of k, i.e. bit 1 of g) or pi1 + 1 (plain:
    // flips with bit 0 of k, the high half of every dword)
    const uint32_t f2 = p.marlin ? ((g & 2) ? 0x80008000u : 0u) : 0x80000000u;
#pragma unroll
    for (int t2 = 0; t2 < 4; ++t2) b2[t2] = b1[t2] ^ f2;
  } else {
    // unit columns: B[k][j] = (k == pi(j)), k = 8 g + 2 t2 (+1)
    const int pi2 = p.marlin ? jj + 16 : 2 * jj + 1;
#pragma unroll
    for (int t2 = 0; t2 < 4; ++t2) {
      const int k0 = 8 * g + 2 * t2;
      b1[t2] = (k0 == pi1 ? one : 0u) | (k0 + 1 == pi1 ? one << 16 : 0u);
      b2[t2] = (k0 == pi2 ? one : 0u) | (k0 + 1 == pi2 ? one << 16 : 0u);
    }
  }
  float ssq = 0.0f;
  // every chunk's operand and MFMAs first, then the per-chunk VALU work: the XC chains are
  // independent, so their latencies overlap (chunks past the last one compute on the dummy
  // registers the loads left and are not written)
  uint32_t a[XC][4];
#pragma unroll
  for (int t = 0; t < XC; ++t) {
    const uint4 xi = r.xr[t];
    a[t][0] = xi.x; a[t][1] = xi.y; a[t][2] = xi.z; a[t][3] = xi.w;
    if constexpr (PRO == kProSiluMul) {  // fp16(silu(g) * u), the silu_mul arithmetic
      const uint4 ui = r.xu[t];
      const uint32_t uu[4] = {ui.x, ui.y, ui.z, ui.w};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        uint32_t v = 0;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const float gv = h2f((uint16_t)(a[t][d] >> (16 * hh))), uv = h2f((uint16_t)(uu[d] >> (16 * hh)));
          v |= (uint32_t)f2h(gv / (1.0f + __expf(-gv)) * uv) << (16 * hh);
        }
        a[t][d] = v;
      }
    }
    if constexpr (PRO == kProRms) {  // h^2 summed in fp32; h * w rounded once to fp16
      const uint4 ni = r.nwr[t];
      const uint32_t nn[4] = {ni.x, ni.y, ni.z, ni.w};
      const bool live = pw + np * t < p.nchunk;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float h0 = h2f((uint16_t)a[t][d]), h1 = h2f((uint16_t)(a[t][d] >> 16));
        if (live) {
          ssq += h0 * h0;
          ssq += h1 * h1;
        }
        const float w0 = h2f((uint16_t)nn[d]), w1 = h2f((uint16_t)(nn[d] >> 16));
        a[t][d] = (uint32_t)f2h(h0 * w0) | ((uint32_t)f2h(h1 * w1) << 16);
      }
    }
  }
  rf4_t d1[XC], d2[XC];
#pragma unroll
  for (int t = 0; t < XC; ++t) {
    d1[t] = rf4_t{0.0f, 0.0f, 0.0f, 0.0f};
    d2[t] = rf4_t{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (BF) {
      d1[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(rb8_t, a[t]), __builtin_bit_cast(rb8_t, b1), d1[t], 0, 0, 0);
      d2[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(rb8_t, a[t]), __builtin_bit_cast(rb8_t, b2), d2[t], 0, 0, 0);
    } else {
      d1[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(rh8_t, a[t]), __builtin_bit_cast(rh8_t, b1), d1[t], 0, 0, 0);
      d2[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(rh8_t, a[t]), __builtin_bit_cast(rh8_t, b2), d2[t], 0, 0, 0);
    }
  }
  uint32_t packed[XC][4];
  float bsc[XC];
  // lane (j, g) holds sub-blocks 4 g + r (r = 0..3) of 128-block g of the chunk; H_4 across
  // them (Sylvester order: r = the high index bits of the 128-block), then the block's
  // power-of-two scale (max |x| -> [2^14, 2^15)) and the fp16 pairs.  One branch on the
  // rotation outside the chunk loop keeps the XC chains in one block, free to interleave.
  auto finish = [&](auto had_t) __attribute__((always_inline)) {
    constexpr bool HAD = decltype(had_t)::value;
    float lo[XC][4], hi[XC][4];
    uint32_t mx[XC];
#pragma unroll
    for (int t = 0; t < XC; ++t) {
      if constexpr (HAD) {
        const float s0 = d1[t][0] + d1[t][1], s1 = d1[t][0] - d1[t][1], s2 = d1[t][2] + d1[t][3], s3 = d1[t][2] - d1[t][3];
        lo[t][0] = s0 + s2; lo[t][1] = s1 + s3; lo[t][2] = s0 - s2; lo[t][3] = s1 - s3;
        const float t0 = d2[t][0] + d2[t][1], t1 = d2[t][0] - d2[t][1], t2 = d2[t][2] + d2[t][3], t3 = d2[t][2] - d2[t][3];
        hi[t][0] = t0 + t2; hi[t][1] = t1 + t3; hi[t][2] = t0 - t2; hi[t][3] = t1 - t3;
      } else {
        // the MFMA results go straight into the inline asm below, whose reads the compiler's
        // hazard padding does not cover (a VALU read of an MFMA result needs wait states the
        // hardware does not insert): 16 wait states, tied to the results so that they sit
        // between the MFMAs and the asm
        asm volatile("s_nop 7\n\ts_nop 7" : "+v"(d1[t]), "+v"(d2[t]));
#pragma unroll
        for (int q = 0; q < 4; ++q) { lo[t][q] = d1[t][q]; hi[t][q] = d2[t][q]; }
      }
      // max |value| (v_max3_f32 with |.| source modifiers: a NaN input yields a NaN maximum,
      // whose exponent field (all ones) then gives the smallest scale, as an infinity does)
      float m0, m1;
      asm("v_max3_f32 %0, |%1|, |%2|, |%3|" : "=v"(m0) : "v"(lo[t][0]), "v"(lo[t][1]), "v"(lo[t][2]));
      asm("v_max3_f32 %0, %1, |%2|, |%3|" : "=v"(m0) : "v"(m0), "v"(lo[t][3]), "v"(hi[t][0]));
      asm("v_max3_f32 %0, |%1|, |%2|, |%3|" : "=v"(m1) : "v"(hi[t][1]), "v"(hi[t][2]), "v"(hi[t][3]));
      asm("v_max_f32 %0, %1, %2" : "=v"(m0) : "v"(m0), "v"(m1));
      mx[t] = __builtin_bit_cast(uint32_t, m0);
    }
    // max over each 16-lane row (quad permutes, half-row mirror, row mirror) as integer maxima
    // of the non-negative bit patterns, one v_max_u32_dpp per chunk and step, the XC chunks
    // interleaved behind one wait state pair
#define SPECTRA_ROWMAX_STEP(CTRL)                                                                     \
    _Pragma("unroll") for (int t = 0; t < XC; ++t) {                                                    \
      if (t == 0) asm volatile("s_nop 1" ::: );                                                         \
      asm volatile("v_max_u32_dpp %0, %0, %0 " CTRL " row_mask:0xf bank_mask:0xf" : "+v"(mx[t]));       \
    }
    SPECTRA_ROWMAX_STEP("quad_perm:[1,0,3,2]")
    SPECTRA_ROWMAX_STEP("quad_perm:[2,3,0,1]")
    SPECTRA_ROWMAX_STEP("row_half_mirror")
    SPECTRA_ROWMAX_STEP("row_mirror")
#undef SPECTRA_ROWMAX_STEP
#pragma unroll
    for (int t = 0; t < XC; ++t) {
      // 2^F with F = 14 - floor(log2 max) (max * 2^F in [2^14, 2^15)), clamped to F <= 126
      // (exponent field >= 15); 1 for an all-zero block.  The scale and its inverse are
      // built directly as float bit patterns.
      const int eb = max((int)(mx[t] >> 23), 15);
      const bool zero = mx[t] == 0u;
      const float f = __builtin_bit_cast(float, zero ? 0x3f800000u : (uint32_t)(268 - eb) << 23);
#pragma unroll
      for (int q = 0; q < 4; ++q) packed[t][q] = pack_scaled(lo[t][q], hi[t][q], f);
      bsc[t] = __builtin_bit_cast(float, zero ? 0x3f800000u : (uint32_t)(eb - 14) << 23);
    }
  };
  if (p.had) finish(std::true_type{});
  else finish(std::false_type{});

#pragma unroll
  for (int t = 0; t < XC; ++t) {
    const int ch = RM ? pw : pw + np * t;
    uint32_t* xpt = RM ? xpd + t * (p.xp_row >> 2) : xpd;
    float* xst = RM ? xsc + t * (p.xsc_row >> 2) : xsc;
    if (ch < p.nchunk) {  // wave-uniform
      const int blk = 4 * ch + g;  // global 128-block
#pragma unroll
      for (int q = 0; q < 4; ++q) xpt[((jj >> 2) * Q + 4 * blk + q) * 4 + (jj & 3)] = packed[t][q];
      if (jj == 0) xst[blk] = bsc[t];
    }
  }
  if (m != 0) return;
  if constexpr (PRO == kProRms) {  // per-producer sums of h^2, fixed order
    ssq = wave_sum(ssq);
    if (lane == 0) ((float*)(smem + p.off_ss))[pw] = ssq;
  }
  // block scales (fp32) [R][K / block], bias and residual
  if (ptid < p.R * p.cpr) {
    float* scf = (float*)(smem + p.off_sc);
    const uint32_t sv[4] = {r.scv.x, r.scv.y, r.scv.z, r.scv.w};
    float4* d = (float4*)(scf + ptid * 8);
    d[0] = make_float4(h2f((uint16_t)sv[0]), h2f((uint16_t)(sv[0] >> 16)), h2f((uint16_t)sv[1]), h2f((uint16_t)(sv[1] >> 16)));
    d[1] = make_float4(h2f((uint16_t)sv[2]), h2f((uint16_t)(sv[2] >> 16)), h2f((uint16_t)sv[3]), h2f((uint16_t)(sv[3] >> 16)));
  }
  if (p.bias != nullptr && ptid < c.Rw)
    ((float*)(smem + p.off_bias))[ptid] =
        p.bias_dt == SPECTRA_F32 ? __builtin_bit_cast(float, r.bias_raw) : to_f32_16((uint16_t)r.bias_raw, p.bias_dt);
  if (p.res != nullptr && ptid < c.Rw) ((uint16_t*)(smem + p.off_res))[ptid] = r.res_raw;
}

// row-wave loads: the weight runs of every slot, then the CSR entries of the group's rows
// (lane li stages entry e0 + li of each row; lanes past the row's entries, and arrays
// without entries, read a dummy word: entry 0, or the workgroup's first weight word).  The
// entries' addresses wait for the row pointers' scalar loads, which are issued after the
// start barrier; the weight runs, which wait for nothing, go first.
template <int G, int SPR, int RPG>
struct RowRegs {
  uint4 wq[SPR * RPG];
  int ocol[RPG], e0r[RPG], cntr[RPG];
  uint32_t oval[RPG];
};

template <int G, int SPR, int RPG>
__device__ __forceinline__ void rows_row_loads(const RowsParams& p, const RowsCtx& c, const int* sx,
                                               RowRegs<G, SPR, RPG>& r) {
  constexpr int NS = SPR * RPG;
  const uint8_t* wbase = p.packed + (int64_t)c.r0 * p.ldp;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int j = s / SPR, ch = s % SPR;
    const int row = c.grow0 + j;
    const uint32_t o = row < c.Rw ? (uint32_t)(row * p.ldp) + (uint32_t)(ch * G + c.li) * 16u : 0u;  // dummy: one line
    r.wq[s] = load_nt_u4(wbase + o);
  }
  asm volatile("" ::: "memory");  // the CSR entries (which wait for the row pointers) behind the weight runs
#pragma unroll
  for (int j = 0; j < RPG; ++j) {
    const int a = G == 32 ? ((c.lane >> 5) ? sx[RPG + j] : sx[j]) : sx[j];
    const int b = G == 32 ? ((c.lane >> 5) ? sx[RPG + j + 1] : sx[j + 1]) : sx[j + 1];
    r.e0r[j] = a;
    r.cntr[j] = c.grow0 + j < c.Rw ? b - a : 0;
    const bool ok = p.csr && c.li < r.cntr[j];
    const void* cb = p.csr ? (const void*)p.ccol : (const void*)wbase;
    const void* vb = p.csr ? (const void*)p.cval : (const void*)wbase;
    const uint32_t e = ok ? (uint32_t)(a + c.li) : 0u;
    r.ocol[j] = load_at<int>(cb, 4u * e);
    r.oval[j] = load_at<uint16_t>(vb, 2u * e);
  }
}

// decode one slot's 16 packed bytes into fp16 code pairs through the LUT (lane-replicated,
// at LDS address 0: the kernel has no static LDS, the host checks)
__device__ __forceinline__ void rows_decode(const uint4& w, uint32_t lanebits, uint32_t (&dec)[16]) {
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int b = 0; b < 16; ++b) {
    const uint32_t addr = __builtin_amdgcn_perm(wd[b >> 2], lanebits, 0x0c0c0000u | ((4u + (b & 3)) << 8));
    dec[b] = *(const __attribute__((address_space(3))) uint32_t*)(uintptr_t)addr;
  }
}

// the rotated activations of one run (lane li of chunk-slot c: run c * G + li): 16 dwords of
// fp16 pairs and the run's 128-block scale, read once and shared by the group's RPG rows
struct XRun {
  uint32_t xpair[16];
  float xs;
  int q;
};

template <int G>
__device__ __forceinline__ XRun rows_xrun(const RowsParams& p, const RowsCtx& c, const uint8_t* smem, int ch,
                                          int m = 0) {
  const int Q = c.Q;
  const uint4* xp4 = (const uint4*)(smem + p.off_xp + (uint32_t)m * p.xp_row);
  const float* xsc = (const float*)(smem + p.off_xsc + (uint32_t)m * p.xsc_row);
  XRun r;
  r.q = ch * G + c.li;
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) {
    const uint4 a = xp4[cc * Q + r.q];
    r.xpair[4 * cc] = a.x; r.xpair[4 * cc + 1] = a.y; r.xpair[4 * cc + 2] = a.z; r.xpair[4 * cc + 3] = a.w;
  }
  r.xs = xsc[r.q >> 2];
  return r;
}

// one slot's dot product with the rotated activations of its run, scaled into the row's sum
__device__ __forceinline__ float rows_dot(const RowsParams& p, const RowsCtx& c, const uint8_t* smem, const XRun& x,
                                          int j, const uint32_t (&dec)[16]) {
  const float* scf = (const float*)(smem + p.off_sc);
  const int rowc = min(c.grow0 + j, c.Rw - 1);
  const float am = scf[rowc * (c.K >> p.gshift) + (x.q >> (p.gshift - 5))];
  float d = 0.0f;
#pragma unroll
  for (int b = 0; b < 16; ++b)
    d = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, dec[b]), __builtin_bit_cast(f16x2_t, x.xpair[b]), d, false);
  return d * (am * x.xs);
}

// the same product without the block scale (several activation rows share it)
__device__ __forceinline__ float rows_dot_raw(const XRun& x, const uint32_t (&dec)[16]) {
  float d = 0.0f;
#pragma unroll
  for (int b = 0; b < 16; ++b)
    d = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, dec[b]), __builtin_bit_cast(f16x2_t, x.xpair[b]), d, false);
  return d;
}

// the row waves' work once the weights are issued: the first NP slots are decoded as they
// land, before the activations are ready (wait_lut / wait_x(m): the producers' counters,
// the LUT and activation row m; both no-ops when the caller already synchronised), then
// the dot products, the outlier products and the row totals.  Several activation rows with
// every slot decoded up front: the rows are taken one by one as the producers finish them.
template <int G, int SPR, int RPG, int NP, bool BF, int PRO, int MR, typename WL, typename WX>
__device__ __forceinline__ void rows_stream(const RowsParams& p, const RowsCtx& c, uint8_t* smem, int np,
                                            RowRegs<G, SPR, RPG>& r, WL wait_lut, WX wait_x, const bool* late) {
  constexpr int NS = SPR * RPG;
  const int Q = c.Q, lane = c.lane, li = c.li;
  const uint32_t* xpd = (const uint32_t*)(smem + p.off_xp);
  const float* xsc = (const float*)(smem + p.off_xsc);
  const uint32_t lanebits = (uint32_t)(lane & 31) << 2;  // this lane's LUT copy: conflict-free reads
  float acc[RPG][MR];
#pragma unroll
  for (int j = 0; j < RPG; ++j)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[j][m] = 0.0f;
  // several rows: the residual values of the group's rows, loaded here and used at the
  // end (issued by every lane of the path, from a valid dummy address without a residual)
  uint16_t rsv[MR > 1 ? RPG : 1][MR];
  if constexpr (MR > 1) {
    const bool hr = p.res != nullptr;
    const void* rb = hr ? p.res : (const void*)p.absmax;
#pragma unroll
    for (int j = 0; j < RPG; ++j)
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const int row = min(c.grow0 + j, c.Rw - 1);
        rsv[j][m] = load_at<uint16_t>(rb, hr ? (uint32_t)(((int64_t)m * p.ldr + c.r0 + row) * 2) : 0u);
      }
  }
  uint32_t pre[NP > 0 ? NP : 1][16];
  wait_lut();
#pragma unroll
  for (int s = 0; s < NP; ++s) rows_decode(r.wq[s], lanebits, pre[s]);
  if constexpr (MR > 1 && NP == NS) {
    const float* scf = (const float*)(smem + p.off_sc);
    float am[NS];  // the slots' block scales, shared by the rows
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      wait_x(m);
      if (m == 0) {  // the block scales are staged with row 0
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const int rowc = min(c.grow0 + s / SPR, c.Rw - 1);
          am[s] = scf[rowc * (c.K >> p.gshift) + (((s % SPR) * G + li) >> (p.gshift - 5))];
        }
      }
#pragma unroll
      for (int ch = 0; ch < SPR; ++ch) {
        const XRun xr = rows_xrun<G>(p, c, smem, ch, m);
#pragma unroll
        for (int j = 0; j < RPG; ++j) {
          const int s = j * SPR + ch;
          acc[j][m] += rows_dot_raw(xr, pre[s < NP ? s : 0]) * (am[s] * xr.xs);
        }
      }
      // row m's products complete before the wait for row m + 1 (none is deferred past it
      // with its activations held in registers)
#pragma unroll
      for (int j = 0; j < RPG; ++j) asm volatile("" : "+v"(acc[j][m]));
    }
  } else {
#pragma unroll
  for (int m = 0; m < MR; ++m) wait_x(m);
  // chunk-slot major: each run's activations are read once for the group's RPG rows (slot
  // s = j * SPR + ch); every row still sums its chunk-slots in order
#pragma unroll
  for (int ch = 0; ch < SPR; ++ch) {
    if constexpr (MR == 1) {
      const XRun xr = rows_xrun<G>(p, c, smem, ch);
#pragma unroll
      for (int j = 0; j < RPG; ++j) {
        const int s = j * SPR + ch;
        if (s < NP) {
          acc[j][0] += rows_dot(p, c, smem, xr, j, pre[s < NP ? s : 0]);
        } else {
          uint32_t dec[16];
          rows_decode(r.wq[s], lanebits, dec);
          acc[j][0] += rows_dot(p, c, smem, xr, j, dec);
        }
      }
    } else {  // several activation rows: each slot decoded once, its block scale read once;
              // each row's activations read just before its product (registers)
      const float* scf = (const float*)(smem + p.off_sc);
      const int q = ch * G + li;
#pragma unroll
      for (int j = 0; j < RPG; ++j) {
        const int s = j * SPR + ch;
        uint32_t dec[16];
        rows_decode(r.wq[s], lanebits, dec);
        const int rowc = min(c.grow0 + j, c.Rw - 1);
        const float am = scf[rowc * (c.K >> p.gshift) + (q >> (p.gshift - 5))];
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const XRun xr = rows_xrun<G>(p, c, smem, ch, m);
          acc[j][m] += rows_dot_raw(xr, dec) * (am * xr.xs);
          asm volatile("" : "+v"(acc[j][m]));  // one row's activations in registers at a time
        }
      }
    }
  }
  }
  // outliers: entry value x rotated activation, into the row's lanes
  if (MR == 1 && p.csr) {
    const uint16_t* xp16 = (const uint16_t*)xpd;
#pragma unroll
    for (int j = 0; j < RPG; ++j) {
      const int cnt = r.cntr[j];
      int col = r.ocol[j];
      uint32_t ov = r.oval[j];
      asm volatile("" : "+v"(col), "+v"(ov)::"memory");  // consumed here, after the stream
      if (li < cnt) acc[j][0] += h2f((uint16_t)ov) * (h2f(xp16[xs_pos(col, p.marlin, Q)]) * xsc[col >> 7]);
      // entries beyond one per lane (rare): read from the side tensor
      for (int el = G + li; el < cnt; el += G) {
        const int cl = p.ccol[r.e0r[j] + el];
        acc[j][0] += h2f(p.cval[r.e0r[j] + el]) * (h2f(xp16[xs_pos(cl, p.marlin, Q)]) * xsc[cl >> 7]);
      }
    }
  } else if (MR > 1 && p.csr) {
#pragma unroll
    for (int j = 0; j < RPG; ++j) {
      const int cnt = r.cntr[j];
      int col = r.ocol[j];
      uint32_t ov = r.oval[j];
      asm volatile("" : "+v"(col), "+v"(ov)::"memory");  // consumed here, after the stream
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        const uint16_t* xp16 = (const uint16_t*)((const uint8_t*)xpd + (uint32_t)m * p.xp_row);
        const float* xs = (const float*)((const uint8_t*)xsc + (uint32_t)m * p.xsc_row);
        if (li < cnt) acc[j][m] += h2f((uint16_t)ov) * (h2f(xp16[xs_pos(col, p.marlin, Q)]) * xs[col >> 7]);
        // entries beyond one per lane (rare): read from the side tensor
        for (int el = G + li; el < cnt; el += G) {
          const int cl = p.ccol[r.e0r[j] + el];
          acc[j][m] += h2f(p.cval[r.e0r[j] + el]) * (h2f(xp16[xs_pos(cl, p.marlin, Q)]) * xs[cl >> 7]);
        }
      }
    }
  }
  // row totals: one butterfly sum per row, lane 0 of the group stores
  float inv = 1.0f;  // kProRms: rsqrt(mean(h^2) + eps)
  if constexpr (PRO == kProRms) {
    const float* ss = (const float*)(smem + p.off_ss);
    float t = 0.0f;
    for (int w = 0; w < np; ++w) t += ss[w];
    inv = 1.0f / sqrtf(t / (float)c.K + p.eps);
  }
  constexpr int odt = BF ? SPECTRA_BF16 : SPECTRA_F16;
  const float* bl = (const float*)(smem + p.off_bias);
  const uint16_t* rsl = (const uint16_t*)(smem + p.off_res);
#pragma unroll
  for (int j = 0; j < RPG; ++j) {
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const float v = group_sum<G>(acc[j][m], lane);
      const int row = c.grow0 + j;
      if (li == 0 && row < c.Rw) {
        float y = v * p.out_scale;
        if constexpr (PRO == kProRms) y *= inv;
        if (p.bias != nullptr) y += bl[row];
        if (p.res != nullptr)
          y = to_f32_16(from_f32_16(y, odt), odt) + to_f32_16(MR == 1 ? rsl[row] : rsv[j][m], odt);
        if (late != nullptr && *late) y = __builtin_nanf("");
        if constexpr (MR == 1) ((uint16_t*)p.out)[c.r0 + row] = from_f32_16(y, odt);
        else ((uint16_t*)p.out)[(int64_t)m * p.ldo + c.r0 + row] = from_f32_16(y, odt);
      }
    }
  }
}

// MR > 1: MR activation rows (x rows ldx apart, out rows ldo apart), no prologue; the row
// waves decode each slot once for the MR dot products.  Without producer waves (the form
// the plan picks) every wave rotates its chunk of all rows as interleaved chains; with
// them (SPLIT, not instantiated for several rows) the producers rotate the rows one after
// another, the next row's chunks loading while a row rotates, and count each row
template <int G, int SPR, int RPG, int XC, bool BF, int PRO, bool SPLIT, int MR = 1>
__global__ void __launch_bounds__(1024, 1) gemv_rows_kernel(const RowsParams p) {
  static_assert(MR == 1 || PRO == kProNone, "several activation rows: no prologue");
  extern __shared__ __align__(16) uint8_t smem[];
  constexpr int RW = RPG * (64 / G);  // rows per wave
  constexpr int NS = SPR * RPG;
  // slots decoded before the activations are ready (one row: the registers allow it)
  // (several rows: all of them or none, the rows then taken one by one or together)
  constexpr int NP = NS <= 4 ? NS : MR > 1 ? 0 : NS <= 8 ? 2 : 0;
  const int tid = threadIdx.x;
  const int W = p.W;  // == blockDim.x / 64; blockDim would pull in the 256-byte implicit-argument block
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int np = SPLIT ? W - p.wr : W;  // producer waves
  // producers are waves 0 .. np - 1 (dispatched first), row waves np .. W - 1
  const int rtid = SPLIT ? tid - 64 * np : tid;  // thread index among the row waves
  RowsCtx c;
  c.tid = tid;
  c.lane = tid & 63;
  c.wave = wave;
  c.W = W;
  c.K = p.k;
  c.Q = p.k >> 5;
  c.r0 = blockIdx.x * p.R;
  c.Rw = min(p.R, p.n - c.r0);
  c.gi = rtid / G;
  c.li = rtid % G;
  c.grow0 = c.gi * RPG;  // this group's first row inside the workgroup
  // every argument the issue phase needs, fetched in one round trip before the first load
  asm volatile("" ::"s"(p.x), "s"(p.packed), "s"(p.ldp), "s"(p.absmax), "s"(p.lda), "s"(p.csr), "s"(p.rowptr),
               "s"(p.bias), "s"(p.res), "s"(p.bias_dt), "s"(p.nchunk), "s"(p.cpr), "s"(p.cmagic), "s"(p.wr), "s"(p.W));
  // [0]: LUT rows built, [1 + m]: activation row m rotated (the block scales, bias and
  // residual staged with row 0)
  uint32_t* counter = (uint32_t*)(smem + kRowsCounterOff);
  const int rwave = SPLIT ? wave - np : wave;  // row-wave index

  if constexpr (SPLIT) {
    if (wave < np) {
      // ---------------- producer waves ----------------
      if (tid == 0) {
#pragma unroll
        for (int i = 0; i <= MR; ++i) counter[i] = 0u;
      }
      // several rows: two register sets, the next row's activations loading while a row rotates
      ProducerRegs<XC, PRO> pr[MR == 1 ? 1 : 2];
      rows_producer_xloads<XC, PRO>(p, c, p.x, wave, np, pr[0]);
      rows_producer_sloads<XC, PRO>(p, c, wave, tid, pr[0]);
      // --- start barrier: counters zeroed (this wave waits for its LDS writes); the
      //     activation requests precede the weight runs
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      __builtin_amdgcn_s_setprio(3);  // the producers are the critical path of the workgroup
      build_pair_lut32<SPECTRA_FMT_NF4>(smem, wave, np, c.lane);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // LDS operations of a wave complete in order
      if (c.lane == 0) __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
#pragma unroll
      for (int m = 0; m < MR; ++m) {
        if (m + 1 < MR)
          rows_producer_xloads<XC, PRO>(p, c, (const uint16_t*)p.x + (int64_t)(m + 1) * p.ldx, wave, np,
                                        pr[(m + 1) & 1]);
        rows_rotate<XC, BF, PRO>(p, c, smem, wave, np, tid, pr[m & 1], m);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (c.lane == 0) __hip_atomic_fetch_add(counter + 1 + m, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
      return;
    }
    // ---------------- row waves ----------------
    // --- start barrier, with no wait: a row wave publishes nothing before it
    asm volatile("s_barrier" ::: "memory");
    int sx[RW + 1];  // CSR extents of the wave's rows: scalar loads, in flight while the weights issue
    if (p.csr) {
      const __attribute__((address_space(4))) int32_t* rpc = (const __attribute__((address_space(4))) int32_t*)p.rowptr;
#pragma unroll
      for (int j = 0; j <= RW; ++j) sx[j] = rpc[min(c.r0 + rwave * RW + j, p.n)];
    } else {
#pragma unroll
      for (int j = 0; j <= RW; ++j) sx[j] = 0;
    }
    RowRegs<G, SPR, RPG> rr;
    rows_row_loads<G, SPR, RPG>(p, c, sx, rr);
    // waits on the producers' counters.  The producers are co-resident waves of this
    // workgroup that wait for nothing but their own loads, so the count always completes;
    // the wait is still bounded, and a wave whose wait ran out stores NaN for its rows
    // rather than a value from incomplete activations.
    bool late = false;
    auto wait_for = [&](int which) {
      int it = 0;
      for (; it < kRowsSpinLimit; ++it) {
        if (__hip_atomic_load(counter + which, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= (uint32_t)np) break;
        __builtin_amdgcn_s_sleep(1);
      }
      late = late || it == kRowsSpinLimit;
      asm volatile("" ::: "memory");
    };
    rows_stream<G, SPR, RPG, NP, BF, PRO, MR>(p, c, smem, np, rr, [&] { wait_for(0); }, [&](int m) { wait_for(1 + m); },
                                              &late);
  } else {
    // every wave loads and produces, then streams its rows
    int sx[RW + 1];
    if (p.csr) {
      const __attribute__((address_space(4))) int32_t* rpc = (const __attribute__((address_space(4))) int32_t*)p.rowptr;
#pragma unroll
      for (int j = 0; j <= RW; ++j) sx[j] = rpc[min(c.r0 + wave * RW + j, p.n)];
    } else {
#pragma unroll
      for (int j = 0; j <= RW; ++j) sx[j] = 0;
    }
    RowRegs<G, SPR, RPG> rr;
    if constexpr (MR > 1) {
      // several rows (one chunk per wave: the plan gives every wave at most one): each
      // wave's chunk of every row loaded up front, the rows rotated as interleaved chains
      static_assert(MR == 1 || XC == 1, "several rows without producer waves: one chunk per wave");
      ProducerRegs<MR, PRO> pm;
      const uint32_t o = (wave < p.nchunk ? (uint32_t)wave * 1024u : 0u) + 64u * (uint32_t)(c.lane & 15) +
                         16u * (uint32_t)(c.lane >> 4);
#pragma unroll
      for (int m = 0; m < MR; ++m) pm.xr[m] = load_at<uint4>((const uint16_t*)p.x + (int64_t)m * p.ldx, o);
      rows_producer_sloads<MR, PRO>(p, c, wave, tid, pm);
      rows_row_loads<G, SPR, RPG>(p, c, sx, rr);
      build_pair_lut32<SPECTRA_FMT_NF4>(smem, wave, W, c.lane);
      rows_rotate<MR, BF, PRO, true>(p, c, smem, wave, W, tid, pm, 0);
    } else {
      ProducerRegs<XC, PRO> pr;
      rows_producer_loads<XC, PRO>(p, c, wave, W, tid, pr);
      rows_row_loads<G, SPR, RPG>(p, c, sx, rr);
      build_pair_lut32<SPECTRA_FMT_NF4>(smem, wave, W, c.lane);
      rows_rotate<XC, BF, PRO>(p, c, smem, wave, W, tid, pr);
    }
    // --- LUT, activation pairs, scales: this wave's LDS writes complete, then the barrier.
    //     (__syncthreads would also wait for every outstanding global load, the weight
    //     runs included, and so hold the decode back until the whole stream has landed.)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (wave * RW >= c.Rw) {  // a wave without rows (it only helped with the activations)
      __builtin_amdgcn_s_waitcnt(0);  // its dummy loads land before it ends
      return;
    }
    rows_stream<G, SPR, RPG, 0, BF, PRO, MR>(p, c, smem, W, rr, [] {}, [](int) {}, nullptr);
  }
}

typedef void (*gemv_rows_fn)(const RowsParams);

}  // namespace spectra
