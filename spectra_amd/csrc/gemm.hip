// Batched / prefill GEMM family for gfx950 (replaces kernels.py:187-389):
//   out = FWHT(a) . W_eff^T + bias
//
// 1. gemm_prep_kernel (one workgroup per activation row): blockwise FWHT in fp32 (the
//    reference's butterfly order), division by sqrt(block), a power-of-two row scale and
//    fp16 rounding.  The row is stored in packed-byte pair order: position 2 b + h holds
//    the element that nibble h of packed byte b multiplies, so a decoded byte (an fp16
//    code pair) and the activations it meets sit at the same positions.
// 2. gemm_outlier_lists_kernel (when the weight has outliers): each group of 16 weight rows'
//    CSR entries / outlier columns bucketed by K-step, with each entry's position in the
//    decoded LDS tile precomputed.
// 3. gemm_kernel<FMT, BN>: a 256 x BN output tile per workgroup, K step 32, 8 waves of
//    128 x BN/4 (v_mfma_f32_32x32x16_f16, fp32 accumulators, two waves per SIMD).  Each step
//    one thread decodes half (BN = 256) or a quarter (BN = 128) of one weight row's 16-byte
//    run through the lane-replicated nibble-pair LUT, applies the block scale (Format A:
//    (q - z) * s) with one fp16 rounding, and writes the row into LDS; the lanes holding one
//    of the step's outlier entries then write its value over its position (the quantized
//    code there is exactly 0).  Activation and weight tiles are double-buffered in LDS with
//    one barrier per step; global loads (tiles, outlier entries) run two steps ahead, and
//    each half-step interleaves the MFMAs of one step with the decode, tile writes and
//    loads of the next (scheduling groups), so the matrix pipe is fed while the wave
//    decodes.  The epilogue undoes the row scale, adds the bias in fp32 and rounds once.
#include <cmath>

#include "common.h"

namespace spectra {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f16v_t __attribute__((ext_vector_type(16)));
typedef _Float16 f16x2g_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBM = 256, kBK = 32;
constexpr int kGemmWaves = 8;  // two per SIMD (four waves of 128 x 128 measured slower)
constexpr int kRowH = 32;         // fp16 per LDS tile row (64 bytes, four 16-byte chunks, swizzled)
constexpr int kPrepThreads = 256;
constexpr int kGLut = 65536;      // lane-replicated nibble-pair LUT at LDS address 0
constexpr int kOGroup = 16;       // weight rows per outlier step list
constexpr int kOListThreads = 256;

// 16-byte chunk c of tile row r sits at chunk c ^ tile_swz(r): with 64-byte rows, every
// 8-lane (32 banks) or 16-lane (64 banks) phase of the tile stores (two or four lanes per
// row) and of the MFMA fragment reads (one lane per row, 32 consecutive rows) touches
// distinct banks.  The mask takes rows' bits 1..3 only, so rows 32 apart share it.
__device__ __forceinline__ int tile_swz(int r) {
  return (((r >> 1) ^ (r >> 2)) & 1) | ((((r >> 1) ^ (r >> 3)) & 1) << 1);
}

// ---------------------------------------------------------------------------
// activation pre-pass
// ---------------------------------------------------------------------------
// One workgroup of 256 threads per activation row.  The row's 8-element chunks are spread
// over the threads (chunk c = tid + 256 u, up to 16 per thread), so a Hadamard block of b
// <= 512 elements lies in b / 8 consecutive lanes of one wave: stages h = 1, 2, 4 run on
// register bits and h = 8 .. 256 across lanes (each stage one fp32 add or subtract, the
// reference's order and rounding); blocks of 1024 finish their last stage through LDS.
// The row is scaled by a power of two (max |x_rot| -> [2^14, 2^15)), rounded to fp16 and
// written in packed-byte pair order.
constexpr int kPrepMaxU = 16;  // K <= 256 * 8 * 16 = 32768

// raw_dt >= 0 (the library-GEMM path): no scale (F = 0), the rotated row rounded to raw_dt
// (SPECTRA_F16 or SPECTRA_BF16), the compute dtype of the reference's GEMM; marlin must be 0.
// With no row-wide scale to find, blockIdx.y then picks a segment of kPrepThreads * 8 * kPrepU
// elements of the row (a multiple of every Hadamard block size), so a long row spreads over
// several workgroups; the scaled mode runs with gridDim.y = 1 (the whole row).
template <int kPrepU>
__global__ void __launch_bounds__(kPrepThreads) gemm_prep_kernel(const void* __restrict__ a, int64_t lda, int dt,
                                                                  int k, int log_had, float div, int marlin, int vec,
                                                                  uint16_t* __restrict__ a16,
                                                                  int32_t* __restrict__ fexp, int raw_dt) {
  extern __shared__ float fs[];  // [k] fp32 (the 1024-block stage), then [k] fp16 (pair-order write)
  __shared__ float wmax[kPrepThreads / 64];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t seg0 = (int64_t)blockIdx.y * (kPrepThreads * 8 * kPrepU);  // first element
  const int n8 = (int)min((int64_t)k - seg0, (int64_t)kPrepThreads * 8 * kPrepU) >> 3;
  float v[kPrepU][8];
#pragma unroll
  for (int u = 0; u < kPrepU; ++u) {
    const int c = tid + u * kPrepThreads;
    if (c < n8) {
      if (vec) {
        const uint4 q = ((const uint4*)((const uint16_t*)a + row * lda + seg0))[c];
        const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[u][2 * e] = to_f32_16((uint16_t)(w4[e] & 0xffffu), dt);
          v[u][2 * e + 1] = to_f32_16((uint16_t)(w4[e] >> 16), dt);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[u][e] = load_elem(a, row * lda + seg0 + 8 * c + e, dt);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[u][e] = 0.0f;
    }
  }
  // compressor.py:34-39: stages h = 1, 2, 4, ...: (u, v) -> (u + v, u - v) in fp32
  // (stage loops unrolled with compile-time strides: the register array stays in registers)
#pragma unroll
  for (int lh = 0; lh < 3; ++lh) {
    if (lh < log_had) {
      const int h = 1 << lh;
#pragma unroll
      for (int u = 0; u < kPrepU; ++u)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if ((e & h) == 0) {
            const float x0 = v[u][e], x1 = v[u][e | h];
            v[u][e] = x0 + x1;
            v[u][e | h] = x0 - x1;
          }
    }
  }
  // stages h = 8 .. 256 across the lanes of a block (lane bit lh - 3)
  const int lane = tid & 63;
  float sgn = 1.0f;
  auto side = [&](int lb) { const bool hi = (tid & lb) != 0; if (hi) sgn = -sgn; return hi ? -1.0f : 1.0f; };
  if (log_had > 3) prep_fly<1>(v, side(1), lane);
  if (log_had > 4) prep_fly<2>(v, side(2), lane);
  if (log_had > 5) prep_fly<4>(v, side(4), lane);
  if (log_had > 6) prep_fly<8>(v, side(8), lane);
  if (log_had > 7) prep_fly<16>(v, side(16), lane);
  if (log_had > 8) prep_fly<32>(v, side(32), lane);
  if (log_had > 9) {  // 1024-blocks: the stage across waves through LDS
#pragma unroll
    for (int u = 0; u < kPrepU; ++u)
      if (tid + u * kPrepThreads < n8)
#pragma unroll
        for (int e = 0; e < 8; ++e) fs[8 * (tid + u * kPrepThreads) + e] = v[u][e];
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kPrepU; ++u) {
      const int c = tid + u * kPrepThreads;
      if (c < n8) {
        const float cc = (c & 64) != 0 ? -1.0f : 1.0f;  // element bit 9 = chunk bit 6 (same for every u)
#pragma unroll
        for (int e = 0; e < 8; ++e) v[u][e] = __builtin_fmaf(fs[8 * (c ^ 64) + e], cc, v[u][e]);
      }
    }
    __syncthreads();
    if (tid & 64) sgn = -sgn;  // every chunk of this thread has the same bit 6 (256 | 64)
  }
  // the normalisation by sqrt(block) (compressor.py:40-41) rides on the output scale below
  float mx = 0.0f;
#pragma unroll
  for (int u = 0; u < kPrepU; ++u)
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[u][e]));
  mx = wave_max(mx);
  if ((tid & 63) == 0) wmax[tid >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  if (log_had > 0) mx = mx / div;  // the normalised row's max |x_rot|
  const uint32_t bits = __builtin_bit_cast(uint32_t, mx);
  const int eb = (int)(bits >> 23);
  const int E = eb == 0 ? -126 : eb - 127;
  int F = bits == 0 ? 0 : 14 - E;  // max |x_rot| * 2^F in [2^14, 2^15): exact scaling, no overflow
  F = F < -126 ? -126 : (F > 126 ? 126 : F);
  if (raw_dt >= 0) F = 0;
  const float f2 = __builtin_bit_cast(float, (uint32_t)(F + 127) << 23);
  // output scale: 2^F / sqrt(block) (one rounding), with the lane's butterfly sign
  const float f = sgn * (log_had > 0 ? f2 / div : f2);
  uint16_t* xs = (uint16_t*)fs;
  if (marlin) {  // natural order into LDS, then pairs (k, k + 16) of each 32-run
#pragma unroll
    for (int u = 0; u < kPrepU; ++u) {
      const int c = tid + u * kPrepThreads;
      if (c < n8) {
        uint32_t d[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          d[e] = (uint32_t)f2h(v[u][2 * e] * f) | ((uint32_t)f2h(v[u][2 * e + 1] * f) << 16);
        *(uint4*)(xs + 8 * c) = make_uint4(d[0], d[1], d[2], d[3]);
      }
    }
    __syncthreads();
    // output chunk c (positions 8 c .. 8 c + 7) = bytes 4 c .. 4 c + 3: run c / 4, j = 4 (c % 4) + i
#pragma unroll
    for (int u = 0; u < kPrepU; ++u) {
      const int c = tid + u * kPrepThreads;
      if (c < n8) {
        const uint16_t* run = xs + 32 * (c >> 2);
        const int j0 = 4 * (c & 3);
        uint32_t d[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) d[i] = (uint32_t)run[j0 + i] | ((uint32_t)run[j0 + i + 16] << 16);
        *(uint4*)(a16 + row * k + seg0 + 8 * c) = make_uint4(d[0], d[1], d[2], d[3]);
      }
    }
  } else {  // byte j = (k 2j, k 2j + 1): pair order is the natural order
#pragma unroll
    for (int u = 0; u < kPrepU; ++u) {
      const int c = tid + u * kPrepThreads;
      if (c < n8) {
        uint32_t d[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          d[e] = raw_dt >= 0 ? (uint32_t)from_f32_16(v[u][2 * e] * f, raw_dt) |
                                   ((uint32_t)from_f32_16(v[u][2 * e + 1] * f, raw_dt) << 16)
                             : (uint32_t)f2h(v[u][2 * e] * f) | ((uint32_t)f2h(v[u][2 * e + 1] * f) << 16);
        *(uint4*)(a16 + row * k + seg0 + 8 * c) = make_uint4(d[0], d[1], d[2], d[3]);
      }
    }
  }
  if (tid == 0) fexp[row] = F;
}

// the activation prep of the library-GEMM path: every row rotated (natural order) and
// rounded to the activation dtype dt, unscaled
int gemm_prep_rotate(const void* a, int64_t lda, int64_t m, int dt, int k, int had, uint16_t* a16, int32_t* fexp,
                     hipStream_t s) {
  int log_had = 0;
  while (had > 1 && (1 << log_had) < had) ++log_had;
  const float div = had > 1 ? (float)std::sqrt((double)had) : 1.0f;
  // segments of kPrepThreads * 8 * 2 = 4096 elements (two chunks of 8 per thread)
  const void* prep = (const void*)gemm_prep_kernel<2>;
  int st = ensure_lds_limit(prep);
  if (st != SPECTRA_OK) return st;
  const int vec = (reinterpret_cast<uintptr_t>(a) % 16) == 0 && lda % 8 == 0;
  const int marl = 0, raw_dt = dt;
  const int seg = kPrepThreads * 8 * 2, nseg = (k + seg - 1) / seg;
  const size_t prep_lds = (size_t)seg * (had > 512 ? 4 : 2);
  void* pargs[] = {(void*)&a, (void*)&lda, (void*)&dt, (void*)&k, (void*)&log_had, (void*)&div, (void*)&marl,
                   (void*)&vec, (void*)&a16, (void*)&fexp, (void*)&raw_dt};
  SPECTRA_HIP_CHECK(hipLaunchKernel(prep, dim3((unsigned)m, (unsigned)nseg), dim3(kPrepThreads), pargs, prep_lds, s));
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

// ---------------------------------------------------------------------------
// MFMA GEMM
// ---------------------------------------------------------------------------
struct GemmParams {
  const uint16_t* a16;  // [M, K] fp16 in pair order, row stride K
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
  int ksplit, ksteps;  // K splits (blockIdx.z) and kBK-steps per split
  float* part;         // ksplit > 1: fp32 partials [ksplit][m][n]
  // outlier step lists (gemm_outlier_lists_kernel): ostart[g][s] = first entry of row
  // group g in K-step s (s = 0 .. K / kBK, the last = the group's end); oent = entries
  const int32_t* ostart;
  const uint32_t* oent;
  int ogroups;
};

template <int FMT, int BN, int NW>
__global__ void __launch_bounds__(64 * NW) gemm_kernel(const GemmParams p) {
  constexpr int NTHR = 64 * NW;
  constexpr int WNW = NW / 2;         // waves along N (two along M)
  constexpr int WN = BN / WNW;        // wave tile: 128 x WN
  constexpr int NT = WN / 32;         // 32-column MFMA tiles per wave
  constexpr int BPT = 16 * BN / NTHR; // packed bytes one thread decodes per step
  constexpr int AU = 4096 / NTHR / 4; // 16-byte activation chunks one thread copies per step
  constexpr int TPR = 16 / BPT;       // threads per weight row
  extern __shared__ __align__(16) uint8_t smem[];
  uint16_t* As = (uint16_t*)(smem + kGLut);       // [2][256][kRowH]
  uint16_t* Ws = As + 2 * kBM * kRowH;            // [2][BN][kRowH]
  int32_t* fx = (int32_t*)(Ws + 2 * BN * kRowH);  // [256] row exponents
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * kBM;
  const int wm = wave / WNW, wn = wave % WNW;
  const int K = p.k;
  // this workgroup's K range: steps [ks, ks + nk) of kBK
  const int ks = blockIdx.z * p.ksteps;
  const int nk = min(p.ksteps, K / kBK - ks);
  asm volatile("" ::"s"(p.a16), "s"(p.packed), "s"(p.ldp), "s"(p.scales), "s"(p.lds), "s"(p.m), "s"(p.n),
               "s"(p.k), "s"(p.gshift), "s"(p.marlin), "s"(p.okind), "s"(p.rowptr), "s"(p.fexp));

  // ---- operand assignment: A row tid / 2, 32 of its 64 bytes a step; weight row
  //      tid / TPR, bytes [(tid % TPR) * BPT, + BPT) of the row's 16-byte run ----
  const int ar = tid / (4 / AU), ah = tid % (4 / AU);  // row, and which AU-chunk part of its 64 bytes
  const uint16_t* asrc = p.a16 + (int64_t)min(m0 + ar, p.m - 1) * K + 8 * AU * ah + ks * kBK;
  const int wr = tid / TPR, wb0 = (tid % TPR) * BPT;
  const int wrow = min(n0 + wr, p.n - 1);
  const uint8_t* wsrc = p.packed + (int64_t)wrow * p.ldp + wb0 + ks * 16;
  const uint16_t* ssrc = p.scales + (int64_t)wrow * p.lds;
  const uint8_t* zsrc = FMT == SPECTRA_FMT_ASYM_G32 ? p.zeros + (int64_t)wrow * p.ldz : nullptr;

  // ---- outlier step lists: this wave decodes tile rows [wlo, wlo + 64 / TPR), one (TPR = 4)
  //      or two (TPR = 2) groups of kOGroup; the lanes of half h of a two-group wave serve
  //      group h.  Each step a lane reads one entry of its group's list for the step (two
  //      steps ahead, like the tiles), and after the decode the lanes holding an entry
  //      write its value over the decoded position (the code there is exactly 0).  The
  //      group's start offsets are read one stage earlier still. ----
  constexpr int OGW = 64 / TPR / kOGroup;  // groups per wave: 2 or 1
  constexpr int OCAP = 64 / OGW;           // entries of a group one read covers: 32 or 64
  const bool has_o = p.okind != SPECTRA_OUTLIERS_NONE;
  const int wlo = 64 * wave / TPR;          // first tile row this wave decodes (wave-uniform)
  const int oh = OGW == 2 ? lane >> 5 : 0;  // this lane's group inside the wave
  const int oln = lane & (OCAP - 1);        // this lane's slot in the group's list
  // (groups past the last row are clamped: those tile rows are never stored)
  const int og = min((n0 + wlo) / kOGroup + oh, p.ogroups - 1);
  const int KS = K / kBK;
  const int32_t* ost = p.ostart + (has_o ? (int64_t)og * (KS + 1) : 0);
  int oo0x = 0, oo0y = 0, oo1x = 0, oo1y = 0;  // (first, end) entry of the step a stage loads next
  int oc0x = 0, oc0y = 0, oc1x = 0, oc1y = 0;  // ... of the step a stage holds
  uint32_t oe0 = 0, oe1 = 0;                   // this lane's entry of that step
  // (unconditional reads: without outliers the host points both arrays at a readable
  // dummy and index 0 is read; past the split's end the index stays in bounds, unused)
  auto ooffs = [&](int& ox, int& oy, int step) __attribute__((always_inline)) {
    const int gi = has_o ? min(ks + step, KS - 1) : 0;
    ox = ost[gi];
    oy = ost[gi + 1];
  };
  // the stage's entry for `step` (offsets read a stage earlier), then the offsets of step + 2
  auto oload = [&](int& oox, int& ooy, int& ocx, int& ocy, uint32_t& oe, int step) __attribute__((always_inline)) {
    ocx = oox;
    ocy = ooy;
    const int e = oox + oln;
    oe = p.oent[has_o && e < ooy ? e : 0];
    ooffs(oox, ooy, step + 2);
  };

  // ---- global -> register staging, two steps ahead ----
  // (two named register stages; an array of them would be placed in scratch memory)
  u32x4_t sa0a, sa0b, sa0c, sa0d, sa1a, sa1b, sa1c, sa1d;
  u32x4_t sw0, sw1;  // BPT packed bytes in the low BPT / 4 lanes
  uint16_t ss0 = 0, ss1 = 0;
  uint8_t sz0 = 0, sz1 = 0;
  auto load = [&](u32x4_t& ga, u32x4_t& gb, u32x4_t& gc, u32x4_t& gd, u32x4_t& gw, uint16_t& gs, uint8_t& gz,
                  int step) __attribute__((always_inline)) {
    const u32x4_t* ap = (const u32x4_t*)(asrc + step * kBK);
    ga = ap[0];
    gb = ap[1];
    if constexpr (AU == 4) {
      gc = ap[2];
      gd = ap[3];
    }
    if constexpr (BPT == 16) {
      gw = *(const u32x4_t*)(wsrc + step * 16);
    } else if constexpr (BPT == 8) {
      const uint2 v = *(const uint2*)(wsrc + step * 16);
      gw.x = v.x;
      gw.y = v.y;
    } else {
      gw.x = *(const uint32_t*)(wsrc + step * 16);
    }
    gs = ssrc[((ks + step) * kBK) >> p.gshift];
    if constexpr (FMT == SPECTRA_FMT_ASYM_G32) gz = zsrc[ks + step];
  };

  // ---- nibble-pair LUT (from registers, no LDS reads) ----
  build_pair_lut<FMT>(smem, wave, NW, lane);
  for (int r = tid; r < kBM; r += NTHR) fx[r] = p.fexp[min(m0 + r, p.m - 1)];
  const uint32_t lanebits = (uint32_t)lane << 2;

  auto outl = [&](int buf, int ocx, int ocy, uint32_t oe) __attribute__((always_inline)) {
    // outliers of the step: every decode write of the wave precedes these (program order)
    if (has_o) {
      // the entry carries its fp16 index inside the group's tile rows (swizzle included)
      uint16_t* grp_l = Ws + (buf * BN + wlo + kOGroup * oh) * kRowH;
      auto put = [&](uint32_t v) __attribute__((always_inline)) { grp_l[v >> 16] = (uint16_t)v; };
      if (ocx + oln < ocy) put(oe);
      // a group with more entries in the step than one read covers (far beyond the
      // format's ratios): the rest read directly, and no read left in flight after
      if (__builtin_amdgcn_ballot_w64(ocy - ocx > OCAP) != 0) {
        for (int e = ocx + OCAP + oln; e < ocy; e += OCAP) put(p.oent[e]);
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
      }
    }
  };

  // ---- register stage -> LDS buffer: activations as loaded, weights decoded ----
  auto store = [&](u32x4_t ga, u32x4_t gb, u32x4_t gc, u32x4_t gd, u32x4_t gw, uint16_t gs, uint8_t gz, int buf,
                   int ocx, int ocy, uint32_t oe) __attribute__((always_inline)) {
    uint16_t* arow_l = As + (buf * kBM + ar) * kRowH;
    const int asw = tile_swz(ar);
    *(u32x4_t*)(arow_l + 8 * ((AU * ah) ^ asw)) = ga;
    *(u32x4_t*)(arow_l + 8 * ((AU * ah + 1) ^ asw)) = gb;
    if constexpr (AU == 4) {
      *(u32x4_t*)(arow_l + 8 * ((AU * ah + 2) ^ asw)) = gc;
      *(u32x4_t*)(arow_l + 8 * ((AU * ah + 3) ^ asw)) = gd;
    }
    const _Float16 sh = __builtin_bit_cast(_Float16, gs);
    const f16x2g_t s2 = {sh, sh};
    uint32_t d[BPT];
#pragma unroll
    for (int b = 0; b < BPT; ++b) {
      const uint32_t addr = __builtin_amdgcn_perm(gw[b >> 2], lanebits, 0x0c0c0000u | ((4u + (b & 3)) << 8));
      f16x2g_t c = __builtin_bit_cast(f16x2g_t, *(const __attribute__((address_space(3))) uint32_t*)(uintptr_t)addr);
      if constexpr (FMT == SPECTRA_FMT_ASYM_G32) {
        const _Float16 zh = (_Float16)(-(float)gz);
        const f16x2g_t z2 = {zh, zh};
        c = c + z2;  // q - z: exact in fp16
      }
      c = c * s2;  // one fp16 rounding
      d[b] = __builtin_bit_cast(uint32_t, c);
    }
    uint16_t* wrow_l = Ws + (buf * BN + wr) * kRowH;
    const int wsw = tile_swz(wr);
    const int wc0 = wb0 / 4;  // first 16-byte chunk (8 fp16) of this thread's decoded run
#pragma unroll
    for (int u = 0; u < BPT / 4; ++u)
      *(uint4*)(wrow_l + 8 * ((wc0 + u) ^ wsw)) = make_uint4(d[4 * u], d[4 * u + 1], d[4 * u + 2], d[4 * u + 3]);
    outl(buf, ocx, ocy, oe);
  };

  f16v_t acc[4][NT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // Every load is issued unconditionally (steps past the split re-read its last one), so
  // the loads in flight are the same on every path and each wait covers exactly its stage.
  auto load0 = [&](int step) __attribute__((always_inline)) {
    load(sa0a, sa0b, sa0c, sa0d, sw0, ss0, sz0, min(step, nk - 1));
    oload(oo0x, oo0y, oc0x, oc0y, oe0, step);
  };
  auto load1 = [&](int step) __attribute__((always_inline)) {
    load(sa1a, sa1b, sa1c, sa1d, sw1, ss1, sz1, min(step, nk - 1));
    oload(oo1x, oo1y, oc1x, oc1y, oe1, step);
  };
  ooffs(oo0x, oo0y, 0);
  ooffs(oo1x, oo1y, 1);
  load0(0);
  load1(1);
  __syncthreads();  // LUT
  store(sa0a, sa0b, sa0c, sa0d, sw0, ss0, sz0, 0, oc0x, oc0y, oe0);
  load0(2);
  __syncthreads();

  const int arow = wm * 128 + (lane & 31), brow = wn * WN + (lane & 31), kq = 8 * (lane >> 5);
  const int aswz = tile_swz(arow), bswz = tile_swz(brow);  // rows 32 apart share the mask
  auto mfma_step = [&](int buf) {
#pragma unroll
    for (int s16 = 0; s16 < kBK; s16 += 16) {
      h8_t af[4], bf[NT];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *(const h8_t*)(As + (buf * kBM + arow + 32 * i) * kRowH + 8 * (((s16 + kq) >> 3) ^ aswz));
#pragma unroll
      for (int j = 0; j < NT; ++j)
        bf[j] = *(const h8_t*)(Ws + (buf * BN + brow + 32 * j) * kRowH + 8 * (((s16 + kq) >> 3) ^ bswz));
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };

  // One half-step: the MFMAs of the step in buffer mbuf, interleaved with the decode and
  // tile writes of the next step (into the other buffer) and the loads of the stage.
  auto half = [&](int mbuf, u32x4_t ga, u32x4_t gb, u32x4_t gc, u32x4_t gd, u32x4_t gw, uint16_t gs, uint8_t gz,
                  int ocx, int ocy, uint32_t oe, int lstage, int lstep) __attribute__((always_inline)) {
    const int buf = 1 - mbuf;
    h8_t af[2][4], bf[2][NT];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[s2][i] = *(const h8_t*)(As + (mbuf * kBM + arow + 32 * i) * kRowH + 8 * (((16 * s2 + kq) >> 3) ^ aswz));
#pragma unroll
      for (int j = 0; j < NT; ++j)
        bf[s2][j] = *(const h8_t*)(Ws + (mbuf * BN + brow + 32 * j) * kRowH + 8 * (((16 * s2 + kq) >> 3) ^ bswz));
    }
    // decode of the next step
    const _Float16 sh = __builtin_bit_cast(_Float16, gs);
    const f16x2g_t sc2 = {sh, sh};
    uint32_t d[BPT];
#pragma unroll
    for (int b = 0; b < BPT; ++b) {
      const uint32_t addr = __builtin_amdgcn_perm(gw[b >> 2], lanebits, 0x0c0c0000u | ((4u + (b & 3)) << 8));
      f16x2g_t c = __builtin_bit_cast(f16x2g_t, *(const __attribute__((address_space(3))) uint32_t*)(uintptr_t)addr);
      if constexpr (FMT == SPECTRA_FMT_ASYM_G32) {
        const _Float16 zh = (_Float16)(-(float)gz);
        const f16x2g_t z2 = {zh, zh};
        c = c + z2;
      }
      c = c * sc2;
      d[b] = __builtin_bit_cast(uint32_t, c);
    }
    uint16_t* arow_l = As + (buf * kBM + ar) * kRowH;
    const int asw = tile_swz(ar);
    *(u32x4_t*)(arow_l + 8 * ((AU * ah) ^ asw)) = ga;
    *(u32x4_t*)(arow_l + 8 * ((AU * ah + 1) ^ asw)) = gb;
    if constexpr (AU == 4) {
      *(u32x4_t*)(arow_l + 8 * ((AU * ah + 2) ^ asw)) = gc;
      *(u32x4_t*)(arow_l + 8 * ((AU * ah + 3) ^ asw)) = gd;
    }
    uint16_t* wrow_l = Ws + (buf * BN + wr) * kRowH;
    const int wsw = tile_swz(wr);
    const int wc0 = wb0 / 4;
#pragma unroll
    for (int u = 0; u < BPT / 4; ++u)
      *(uint4*)(wrow_l + 8 * ((wc0 + u) ^ wsw)) = make_uint4(d[4 * u], d[4 * u + 1], d[4 * u + 2], d[4 * u + 3]);
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[s2][i], bf[s2][j], acc[i][j], 0, 0, 0);
    if (lstage == 0) load0(lstep);
    else load1(lstep);
    // Interleave: the first k16's fragments, then per MFMA one LDS op (fragment / LUT read
    // or tile write), two VALU (decode) and one global load, so the MFMA pipe is fed while
    // this wave's decode and copies run (measured best of the patterns tried).
    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);  // LDS reads
#pragma unroll
    for (int q = 0; q < 2 * 4 * NT; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x080, 1, 0);  // LDS
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
    }
    outl(buf, ocx, ocy, oe);
  };

  // two steps per iteration so the register stages have static indices
  int kt = 0;
  for (; kt + 1 < nk; kt += 2) {
    // MFMAs of step kt (buffer 0) with step kt+1 -> buffer 1; then step kt+1 with kt+2 ->
    // buffer 0 (past the end: unread)
    half(0, sa1a, sa1b, sa1c, sa1d, sw1, ss1, sz1, oc1x, oc1y, oe1, 1, kt + 3);
    __syncthreads();
    half(1, sa0a, sa0b, sa0c, sa0d, sw0, ss0, sz0, oc0x, oc0y, oe0, 0, kt + 4);
    __syncthreads();
  }
  if (kt < nk) mfma_step(0);  // odd step count: the last step sits in buffer 0

  // ---- epilogue: D[row][col], row = 8 (r / 4) + 4 (lane / 32) + r % 4, col = lane % 32 ----
  if (p.ksplit > 1) {  // fp32 partials of this split (row exponent applied, no bias)
    float* part = p.part + (int64_t)blockIdx.z * p.m * p.n;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int col = n0 + wn * WN + j * 32 + (lane & 31);
      if (col >= p.n) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rl = wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
          if (m0 + rl < p.m)
            part[(int64_t)(m0 + rl) * p.n + col] = acc[i][j][r] * __builtin_bit_cast(float, (uint32_t)(127 - fx[rl]) << 23);
        }
      }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int col = n0 + wn * WN + j * 32 + (lane & 31);
    if (col >= p.n) continue;
    const float bv = p.bias ? load_elem(p.bias, col, p.bias_dt) : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rl = wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (m0 + rl < p.m) {
          const float y = acc[i][j][r] * __builtin_bit_cast(float, (uint32_t)(127 - fx[rl]) << 23) + bv;
          ((uint16_t*)p.out)[(int64_t)(m0 + rl) * p.ldo + col] = from_f32_16(y, p.act_dt);
        }
      }
    }
  }
}

// out[r, c] = act(sum over splits of part[z][r][c] + bias[c]), splits summed in order
constexpr int kRedThreads = 256;
__global__ void __launch_bounds__(kRedThreads) splitk_reduce_kernel(const float* __restrict__ part, int ksplit, int m,
                                                                     int n, const void* bias, int bias_dt, void* out,
                                                                     int64_t ldo, int act_dt) {
  const int64_t i = (int64_t)blockIdx.x * kRedThreads + threadIdx.x;  // 4 consecutive columns
  const int64_t n4 = n >> 2;
  if (i >= (int64_t)m * n4) return;
  const int64_t r = i / n4, c = (i - r * n4) * 4;
  const int64_t mn = (int64_t)m * n;
  float4 a = *(const float4*)(part + r * n + c);
  for (int z = 1; z < ksplit; ++z) {
    const float4 b = *(const float4*)(part + z * mn + r * n + c);
    a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
  }
  float v[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (bias) v[e] += load_elem(bias, c + e, bias_dt);
    ((uint16_t*)out)[r * ldo + c + e] = from_f32_16(v[e], act_dt);
  }
}

// Outlier step lists for the GEMM, one workgroup per group of kOGroup weight rows: the
// group's entries (CSR, or the outlier columns of every row) bucketed by K-step with a
// counting sort in LDS.  ostart[g][s] = first entry of step s (s = 0 .. KS, the last = the
// group's end), oent[e] = (fp16 index inside the group's 16 LDS tile rows, swizzle applied)
// << 16 | fp16 value bits -- the tile rows of a group share their swizzle pattern modulo 16,
// so the position is known here.  The order inside a step is arbitrary: each entry owns its
// position in the tile.
__global__ void __launch_bounds__(kOListThreads) gemm_outlier_lists_kernel(
    int okind, const int32_t* __restrict__ rowptr, const int32_t* __restrict__ ccol,
    const uint16_t* __restrict__ cval, const int64_t* __restrict__ oidx, const void* __restrict__ ow,
    int64_t ldow, int ow_dt, int n_out, int n, int KS, int marlin, int32_t* __restrict__ ostart,
    uint32_t* __restrict__ oent) {
  extern __shared__ int32_t cnt[];  // [KS + 1]: counts, then cursors
  __shared__ int32_t rp[kOGroup + 1];
  __shared__ int32_t wtot[kOListThreads / 64];
  const int g = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const bool csr = okind == SPECTRA_OUTLIERS_CSR;
  const int r0 = g * kOGroup, nr = min(kOGroup, n - r0);
  // the group's entries are [rp[0], rp[nr]), row r's [rp[r], rp[r + 1]) (the outlier columns
  // of every row for Format A: n_out per row)
  if (tid <= nr) rp[tid] = csr ? rowptr[r0 + tid] : (r0 + tid) * n_out;
  for (int t = tid; t <= KS; t += kOListThreads) cnt[t] = 0;
  __syncthreads();
  const int base = rp[0], total = rp[nr] - base;
  // entry el of the group: its row, column and fp16 value (entries in parallel, no per-row chain)
  auto entry = [&](int el, int& r, int& c, uint32_t& v) __attribute__((always_inline)) {
    if (csr) {
      const int e = base + el;
      r = 0;
#pragma unroll
      for (int q = 1; q < kOGroup; ++q) r += (q < nr && rp[q] <= e) ? 1 : 0;
      c = ccol[e];
      v = cval[e];
    } else {
      r = el / n_out;
      const int jj = el - r * n_out;
      c = (int)oidx[jj];
      v = f2h(load_elem(ow, (int64_t)(r0 + r) * ldow + jj, ow_dt));
    }
  };
  for (int el = tid; el < total; el += kOListThreads) {
    int r, c;
    uint32_t v;
    entry(el, r, c, v);
    if ((unsigned)c < (unsigned)(KS * kBK)) atomicAdd(&cnt[c / kBK], 1);  // (columns outside K: dropped)
  }
  __syncthreads();
  // exclusive scan of cnt[0, KS): thread t owns a run of `per` consecutive steps
  const int per = (KS + kOListThreads - 1) / kOListThreads;
  const int lo = min(tid * per, KS), hi = min(lo + per, KS);
  int run = 0;
  for (int t = lo; t < hi; ++t) run += cnt[t];
  int inc = run;  // inclusive scan over the wave
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(inc, o, 64);
    if (lane >= o) inc += v;
  }
  if (lane == 63) wtot[wv] = inc;
  __syncthreads();
  int pre = inc - run;
  for (int w = 0; w < wv; ++w) pre += wtot[w];
  int32_t* og = ostart + (int64_t)g * (KS + 1);
  for (int t = lo; t < hi; ++t) {
    const int c = cnt[t];
    cnt[t] = pre;  // cursor
    og[t] = base + pre;
    pre += c;
  }
  if (tid == kOListThreads - 1) og[KS] = base + pre;  // the last thread's runs end at KS
  __syncthreads();
  for (int el = tid; el < total; el += kOListThreads) {
    int r, c;
    uint32_t v;
    entry(el, r, c, v);
    if ((unsigned)c >= (unsigned)(KS * kBK)) continue;
    const int pos = atomicAdd(&cnt[c / kBK], 1);
    const int cs = c % kBK;
    const int jb = marlin ? (cs & 15) : (cs >> 1), h = marlin ? (cs >> 4) : (cs & 1);
    const int e2 = 2 * jb + h;  // fp16 index in the step's decoded row (packed-byte pair order)
    const int off = r * kRowH + 8 * ((e2 >> 3) ^ tile_swz(r)) + (e2 & 7);
    oent[base + pos] = ((uint32_t)off << 16) | v;
  }
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// tile plan: 256 x 256 tiles once there are at least 64 of them (twice the MFMA work per
// step of the 128-wide tile, whose fixed per-step work weighs double), 256 x 128 below that,
// and K splits while the tiles fill fewer than 256 CUs (each split >= 8 steps of 32; fp32
// partials, a fixed-order reduce)
struct GemmPlan {
  int BN, mt, nt, ksplit, ksteps;
};
static GemmPlan plan_gemm(int64_t m, int64_t n, int64_t k) {
  GemmPlan g;
  g.mt = (int)((m + kBM - 1) / kBM);
  const bool wide = (int64_t)g.mt * ((n + 255) / 256) >= 64;
  g.BN = wide ? 256 : 128;
  g.nt = (int)((n + g.BN - 1) / g.BN);
  const int tiles = g.mt * g.nt;
  const int steps = (int)(k / kBK);
  const int ncu = device_cu_count();  // K splits while the tiles fill fewer workgroups than CUs
  int ks = tiles < ncu && n % 4 == 0 ? ncu / tiles : 1;
  ks = ks > 8 ? 8 : ks;
  while (ks > 1 && steps / ks < 8) --ks;
  g.ksteps = (steps + ks - 1) / ks;
  g.ksplit = (steps + g.ksteps - 1) / g.ksteps;
  return g;
}

// entries the outlier step lists hold (0: none)
static int64_t outlier_entries(const spectra_qweight_t* w) {
  if (w->outlier_kind == SPECTRA_OUTLIERS_CSR && w->csr_nnz > 0) return w->csr_nnz;
  if (w->outlier_kind == SPECTRA_OUTLIERS_COLUMNS && w->num_outliers > 0) return w->n * (int64_t)w->num_outliers;
  return 0;
}

// prefill.hip: the library GEMM path (m >= 512)
constexpr int64_t kLibraryMinM = 512;
size_t prefill_workspace(const spectra_qweight_t* w, int64_t m, int act_dtype);
int prefill_launch(const spectra_qweight_t* w, const void* a, int64_t lda, int64_t m, int act_dtype, void* out,
                   int64_t ldo, void* workspace, size_t workspace_bytes, hipStream_t s);

// skinny.hip: the small-batch MFMA family (2 <= m <= 16)
size_t skinny_workspace(const spectra_qweight_t* w, int64_t m);
int skinny_launch(const spectra_qweight_t* w, const void* x, int64_t ldx, int64_t m, int act_dtype, void* out,
                  int64_t ldo, void* workspace, size_t workspace_bytes, hipStream_t stream);

}  // namespace spectra

using namespace spectra;

namespace spectra {
// the MFMA families' own buffers: every call of the GEMM entry runs with this much (the
// library path of m >= kLibraryMinM needs more and runs only when the workspace holds it)
size_t gemm_workspace_min(const spectra_qweight_t* w, int64_t m) {
  if (w == nullptr || m <= 0) return 0;
  const GemmPlan g = plan_gemm(m, w->n, w->k);
  size_t gemm = align256((size_t)m * (size_t)w->k * 2) + align256((size_t)m * 4) +
                (g.ksplit > 1 ? align256((size_t)g.ksplit * m * w->n * 4) : 0);
  const int64_t nent = outlier_entries(w);
  if (nent > 0)  // outlier step lists
    gemm += align256((size_t)((w->n + kOGroup - 1) / kOGroup) * (size_t)(w->k / kBK + 1) * 4) +
            align256((size_t)nent * 4);
  const size_t small = skinny_workspace(w, m);
  return gemm > small ? gemm : small;
}
}  // namespace spectra

extern "C" size_t spectra_w4a16_gemm_workspace(const spectra_qweight_t* w, int64_t m, int32_t act_dtype) {
  if (w == nullptr || m <= 0) return 0;
  const size_t need = gemm_workspace_min(w, m), lib = prefill_workspace(w, m, act_dtype);
  return need > lib ? need : lib;
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
  if (w->k % 64 != 0) return fail(SPECTRA_ERR_UNSUPPORTED, "the GEMM family needs K % 64 == 0");
  if (w->k > 32768) return fail(SPECTRA_ERR_UNSUPPORTED, "the GEMM family serves K <= 32768");
  if (w->format == SPECTRA_FMT_NF4 && w->group_size < 32)
    return fail(SPECTRA_ERR_UNSUPPORTED, "the GEMM family needs an NF4 block of at least 32");
  if (w->hadamard_block > 1024) return fail(SPECTRA_ERR_UNSUPPORTED, "the GEMM family serves hadamard_block <= 1024");
  SPECTRA_REQUIRE((reinterpret_cast<uintptr_t>(w->packed) % 16) == 0 && w->packed_stride % 16 == 0,
                  "packed weights must be 16-byte aligned with a row stride multiple of 16");
  const size_t need = gemm_workspace_min(w, m);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(SPECTRA_ERR_WORKSPACE, "workspace missing or smaller than the GEMM family needs "
                                       "(spectra_w4a16_gemm_workspace() bytes serve every family)");
  SPECTRA_REQUIRE((reinterpret_cast<uintptr_t>(workspace) % 256) == 0, "workspace must be 256-byte aligned");
  const hipStream_t s = (hipStream_t)stream;
  if (m >= 2 && m <= 16) {  // HBM-bound small batches: the MFMA stream family when it serves the operands
    const int sst = skinny_launch(w, a, lda, m, act_dtype, out, ldo, workspace, workspace_bytes, s);
    if (sst != SPECTRA_ERR_UNSUPPORTED) return sst;
  }
  if (m >= kLibraryMinM) {  // prompt sizes: dequantized weights on the matrix-core library GEMM
    const int pst = prefill_launch(w, a, lda, m, act_dtype, out, ldo, workspace, workspace_bytes, s);
    if (pst != SPECTRA_ERR_UNSUPPORTED) return pst;
  }
  uint16_t* a16 = (uint16_t*)workspace;
  int32_t* fexp = (int32_t*)((uint8_t*)workspace + align256((size_t)m * w->k * 2));
  const int had = w->hadamard_block;
  int log_had = 0;
  while (had > 1 && (1 << log_had) < had) ++log_had;
  const float div = had > 1 ? (float)std::sqrt((double)had) : 1.0f;
  // chunks of 8 activations per prep thread, rounded up to a power of two
  const int64_t n8 = w->k / 8;
  const int pu = n8 <= 256 ? 1 : n8 <= 512 ? 2 : n8 <= 1024 ? 4 : n8 <= 2048 ? 8 : 16;
  const void* prep = pu == 1 ? (const void*)gemm_prep_kernel<1> : pu == 2 ? (const void*)gemm_prep_kernel<2>
                   : pu == 4 ? (const void*)gemm_prep_kernel<4> : pu == 8 ? (const void*)gemm_prep_kernel<8>
                             : (const void*)gemm_prep_kernel<16>;
  int st2 = ensure_lds_limit(prep);
  if (st2 != SPECTRA_OK) return st2;
  const int vec = (reinterpret_cast<uintptr_t>(a) % 16) == 0 && lda % 8 == 0;
  const int kk32 = (int)w->k, marl = w->marlin_layout ? 1 : 0;
  const size_t prep_lds = (size_t)w->k * (had > 512 ? 4 : 2);
  const int scaled = -1;  // per-row power-of-two scale, fp16
  void* pargs[] = {(void*)&a, (void*)&lda, (void*)&act_dtype, (void*)&kk32, (void*)&log_had, (void*)&div,
                   (void*)&marl, (void*)&vec, (void*)&a16, (void*)&fexp, (void*)&scaled};
  SPECTRA_HIP_CHECK(hipLaunchKernel(prep, dim3((unsigned)m), dim3(kPrepThreads), pargs, prep_lds, s));
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
  const GemmPlan g = plan_gemm(m, w->n, w->k);
  const bool wide = g.BN == 256;
  const int BN = g.BN;
  p.ksplit = g.ksplit;
  p.ksteps = g.ksteps;
  p.part = g.ksplit > 1 ? (float*)((uint8_t*)fexp + align256((size_t)m * 4)) : nullptr;
  // outlier step lists (after the partials in the workspace), built for this call
  const int64_t nent = outlier_entries(w);
  const int KS = (int)(w->k / kBK);
  p.ogroups = (int)((w->n + kOGroup - 1) / kOGroup);
  if (nent > 0) {
    if (nent >= (int64_t(1) << 31)) return fail(SPECTRA_ERR_UNSUPPORTED, "the GEMM family serves < 2^31 outlier entries");
    uint8_t* lists = (uint8_t*)fexp + align256((size_t)m * 4) +
                     (g.ksplit > 1 ? align256((size_t)g.ksplit * m * w->n * 4) : 0);
    int32_t* ostart = (int32_t*)lists;
    uint32_t* oent = (uint32_t*)(lists + align256((size_t)p.ogroups * (size_t)(KS + 1) * 4));
    p.ostart = ostart;
    p.oent = oent;
    hipLaunchKernelGGL(gemm_outlier_lists_kernel, dim3((unsigned)p.ogroups), dim3(kOListThreads),
                       (size_t)(KS + 1) * 4, s, p.okind, w->csr_rowptr, w->csr_col, w->csr_val, w->outlier_idx,
                       w->outlier_w, w->outlier_w_stride, w->outlier_w_dtype, (int)w->num_outliers, (int)w->n, KS,
                       p.marlin, ostart, oent);
    SPECTRA_HIP_CHECK(hipGetLastError());
  } else {
    p.okind = SPECTRA_OUTLIERS_NONE;
    p.ostart = (const int32_t*)a16;  // readable dummies: the kernel reads index 0 and 1 only
    p.oent = (const uint32_t*)a16;
  }
  const size_t lds = (size_t)kGLut + (size_t)2 * (kBM + BN) * kRowH * 2 + kBM * 4;
  dim3 grid((unsigned)g.nt, (unsigned)g.mt, (unsigned)g.ksplit);
  const void* kern;
  if (w->format == SPECTRA_FMT_NF4)
    kern = wide ? (const void*)gemm_kernel<SPECTRA_FMT_NF4, 256, kGemmWaves>
                : (const void*)gemm_kernel<SPECTRA_FMT_NF4, 128, kGemmWaves>;
  else
    kern = wide ? (const void*)gemm_kernel<SPECTRA_FMT_ASYM_G32, 256, kGemmWaves>
                : (const void*)gemm_kernel<SPECTRA_FMT_ASYM_G32, 128, kGemmWaves>;
  st2 = ensure_lds_limit(kern, true);
  if (st2 != SPECTRA_OK) return st2;
  void* kargs[] = {(void*)&p};
  SPECTRA_HIP_CHECK(hipLaunchKernel(kern, grid, dim3(64 * kGemmWaves), kargs, lds, s));
  SPECTRA_HIP_CHECK(hipGetLastError());
  if (g.ksplit > 1) {
    const int64_t work = m * (w->n / 4);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((work + kRedThreads - 1) / kRedThreads)),
                       dim3(kRedThreads), 0, s, (const float*)p.part, g.ksplit, (int)m, (int)w->n, w->bias,
                       w->bias_dtype, out, ldo, act_dtype);
    SPECTRA_HIP_CHECK(hipGetLastError());
  }
  return SPECTRA_OK;
}
