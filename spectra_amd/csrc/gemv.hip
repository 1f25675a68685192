// Host side of the decode GEMV family: decomposition, LDS layout, argument checks and
// launch.  The kernels live in gemv_kernel.h, instantiated per activation dtype in
// gemv_f16.hip and gemv_bf16.hip.
#include <algorithm>
#include <cmath>

#include "gemv_kernel.h"
#include "gemv_rows_inst.h"
#include "gemv_rows_lm.h"
#include "gemv_stream.h"

namespace spectra {

static uint32_t align16(uint32_t v) { return (v + 15u) & ~15u; }

struct GemvPlan {
  int mt, S, G, rpw, R, BD, grid, ocap;
  bool wide;  // 16 waves per workgroup
  uint32_t off_xp, off_xsc, off_part, off_rp, off_bias, off_ss, off_res, off_oprod, lds_bytes;
};

// returns false when the shape does not fit this kernel family
static bool plan_gemv(int64_t n, int64_t k, int m, bool outliers, bool csr, GemvPlan* pl, int rpw2) {
  const int mt = m <= 1 ? 1 : (m <= 2 ? 2 : 4);
  if (m > 4 || k > 16384 || k % 32) return false;
  const int S = (int)((k + 2047) / 2048);
  // 8 waves per workgroup (two per SIMD): the setup work is per element, the stream per wave
  int G = 8 / S;
  const int ncu = device_cu_count();
  const int64_t want = (n + ncu - 1) / ncu;  // rows per workgroup for ~one workgroup per CU
  if (G > want) G = (int)want;
  if (G < 1) G = 1;
  int rpw = (int)((want + G - 1) / G);
  const int rpw_max = mt == 4 ? 8 : kRpwMax;
  bool wide = false;
  const bool two = rpw > rpw_max && mt == 1;
  if (two) {
    // more rows than one resident workgroup per CU holds: size for two per CU (LDS <= 80 KB
    // below, at most rpw2 rows per wave: the kernels built for 128 VGPRs), so that one
    // workgroup's set-up overlaps the other's stream
    const int64_t want2 = (n + 511) / 512;
    rpw = (int)((want2 + G - 1) / G);
    if (rpw > rpw2) rpw = rpw2;
  } else if (mt == 1) {
    // one workgroup per CU: 16 waves (four per SIMD) hide the phases' latencies better
    // (measured: down_proj 7.84 -> 7.35 us); with two per CU the 8-wave plan stays ahead
    int G16 = 16 / S;
    if (G16 > want) G16 = (int)want;
    if (G16 < 1) G16 = 1;
    const int rpw16 = (int)((want + G16 - 1) / G16);
    if (S * G16 > 8 && rpw16 <= kRpwWide) {
      G = G16;
      rpw = rpw16;
      wide = true;
    }
  }
  rpw = rpw < 1 ? 1 : (rpw > rpw_max ? rpw_max : rpw);
  // exactly the rows that spread N over the CUs (one workgroup per CU, or two in the large-N
  // plan): the last row of some waves then stays empty, and every CU streams
  const int64_t per_wg = two ? (n + 511) / 512 : want;
  const int R = (int64_t)G * rpw > per_wg ? (int)per_wg : G * rpw;
  const int BD = 64 * S * G;
  // each thread stages at most mt 32-element activation runs
  const int64_t runs = (int64_t)mt * (k / 32);
  if (runs > (int64_t)BD * mt) return false;
  if (R + 1 > BD || R > 4096) return false;
  pl->mt = mt; pl->S = S; pl->G = G; pl->rpw = rpw; pl->R = R; pl->BD = BD; pl->wide = wide;
  pl->grid = (int)((n + R - 1) / R);
  uint32_t off = kLutBytes;
  pl->off_xp = off;
  off = align16(off + (uint32_t)(mt * S * 2048 * 2));  // rows padded to whole slices
  pl->off_xsc = off;
  off = align16(off + (uint32_t)(mt * (k / 32) * 4));
  pl->off_part = off;
  off = align16(off + (uint32_t)(R * S * mt * 4));
  pl->off_rp = off;
  off = align16(off + (uint32_t)((R + 1) * 4));
  pl->off_bias = off;
  off = align16(off + (uint32_t)(R * 4));
  pl->off_ss = off;  // per-wave sums of squares (fused RMSNorm)
  off = align16(off + (uint32_t)(kMaxWaves * 4));
  pl->off_res = off;  // residual values of the outputs (16-bit)
  off = align16(off + (uint32_t)(R * mt * 2));
  pl->off_oprod = off;
  if (off > 163840) return false;
  // outlier products staged in LDS: the entries one load round covers (four per thread
  // for CSR, one for dense columns), as many as the LDS left holds (entries beyond that
  // are read from the side tensor in the per-row phase)
  int ocap = outliers ? (csr ? 4 * BD - 3 : BD) : 0;
  const int fit = (int)((163840 - off) / (uint32_t)(mt * 4));
  if (ocap > fit) ocap = fit;
  // grids beyond one workgroup per CU: keep two resident per CU when the staging still
  // covers a useful share of the entries (the rest are read in the per-row phase)
  if (pl->grid > ncu && mt == 1 && off < 81920) {
    const int fit2 = (int)((81920 - off) / (uint32_t)(mt * 4));
    if (fit2 >= 256 && ocap > fit2) ocap = fit2;
  }
  pl->ocap = ocap;
  off = align16(off + (uint32_t)((ocap > 0 ? ocap : 1) * mt * 4));  // at least one entry: the per-row reads index it
  pl->lds_bytes = off;
  return off <= 163840;
}

static bool ptr_aligned(const void* p, int a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// ---------------------------------------------------------------------------
// stream kernel plan (one activation row, NF4, K a multiple of 1024)
// ---------------------------------------------------------------------------
struct StreamPlan {
  int W, P, RG, NS, R, grid, ocap, pmagic, cpr;
  uint32_t off_xp, off_xsc, off_part, off_rp, off_bias, off_res, off_ss, off_sc, off_op, lds_bytes;
};

// R = ceil(N / CUs) rows per workgroup (one workgroup per CU); W waves with 2W a multiple
// of P = K / 1024, the most waves among those that give the fewest slots per lane
static bool plan_stream(int64_t n, int64_t k, int64_t ldp, int64_t lda, int block, int ncu, StreamPlan* pl) {
  if (k % 1024 != 0 || k > 16384 || ncu <= 0) return false;
  if ((k / block) % 8 != 0 || (lda * 2) % 16 != 0) return false;  // absmax rows in whole 16-byte chunks
  const int P = (int)(k / 1024);
  const int64_t R = (n + ncu - 1) / ncu;
  int bestW = 0, bestNS = 1 << 30;
  for (int W = 16; W >= 4; --W) {
    if ((2 * W) % P != 0 || 64 * W < k / 16) continue;  // one activation half-run per thread
    const int RG = 2 * W / P;
    const int NS = (int)((R + RG - 1) / RG);
    if (NS < bestNS) {
      bestNS = NS;
      bestW = W;
    }
  }
  if (bestW == 0 || bestNS > kStreamMaxSlots) return false;
  // 32-bit per-lane byte offsets from the workgroup's first row
  if (R * ldp >= (int64_t(1) << 31) || R * lda * 2 >= (int64_t(1) << 31)) return false;
  pl->W = bestW;
  pl->P = P;
  pl->RG = 2 * bestW / P;
  pl->NS = bestNS;
  pl->R = (int)R;
  pl->grid = (int)((n + R - 1) / R);
  pl->pmagic = (65536 + P - 1) / P;
  pl->cpr = (int)(k / block / 8);
  if (R * pl->cpr > 64 * bestW) return false;  // one absmax chunk per thread
  uint32_t off = kLutBytes;
  pl->off_xp = off;
  off = align16(off + (uint32_t)(k * 2));
  pl->off_xsc = off;
  off = align16(off + (uint32_t)(k / 32 * 4));
  pl->off_part = off;
  off = align16(off + (uint32_t)(R * P * 4));
  pl->off_rp = off;
  off = align16(off + (uint32_t)((R + 1) * 4));
  pl->off_bias = off;
  off = align16(off + (uint32_t)(R * 4));
  pl->off_res = off;
  off = align16(off + (uint32_t)(R * 2));
  pl->off_ss = off;
  off = align16(off + (uint32_t)(kMaxWaves * 4));
  pl->off_sc = off;
  off = align16(off + (uint32_t)(R * pl->cpr * 16));
  pl->off_op = off;
  if (off + 4 > 163840) return false;
  int ocap = kStreamOutlierLoads * 64 * bestW;
  const int fit = (int)((163840 - off) / 4u);
  if (ocap > fit) ocap = fit;
  pl->ocap = ocap;
  pl->lds_bytes = align16(off + (uint32_t)(ocap * 4));
  return pl->lds_bytes <= 163840;
}

static int stream_launch(const spectra_qweight_t* w, const StreamPlan& pl, const void* x, int act_dtype, void* out,
                         hipStream_t stream, const spectra_gemv_fusion_t* fu, int kpro) {
  StreamParams p;
  p.packed = w->packed; p.ldp = w->packed_stride;
  p.absmax = w->scales; p.lda = w->scales_stride;
  const bool csr = w->outlier_kind == SPECTRA_OUTLIERS_CSR && w->csr_nnz > 0;
  p.rowptr = csr ? w->csr_rowptr : nullptr;
  p.ccol = csr ? w->csr_col : nullptr;
  p.cval = csr ? w->csr_val : nullptr;
  p.csr = csr ? 1 : 0;
  p.csr_nnz = csr ? (int)w->csr_nnz : 0;
  p.bias = w->bias; p.bias_dt = w->bias_dtype;
  p.x = x; p.out = out;
  p.nw = fu ? fu->norm_weight : nullptr;
  p.res = fu ? fu->residual : nullptr;
  p.eps = fu ? fu->eps : 0.0f;
  p.out_scale = w->hadamard_block ? (float)(1.0 / std::sqrt((double)w->hadamard_block)) : 1.0f;
  p.n = (int)w->n; p.k = (int)w->k;
  p.W = pl.W; p.R = pl.R; p.P = pl.P; p.RG = pl.RG; p.pmagic = pl.pmagic;
  int gs = 0;
  while ((1 << gs) < w->group_size) ++gs;
  p.gshift = gs;
  p.log_had = 0;
  while (p.log_had < 30 && (1 << p.log_had) < w->hadamard_block) ++p.log_had;
  p.marlin = w->marlin_layout ? 1 : 0;
  p.ocap = pl.ocap;
  p.cpr = pl.cpr;
  p.cmagic = (65536 + pl.cpr - 1) / pl.cpr;
  p.off_sc = pl.off_sc;
  p.off_xp = pl.off_xp; p.off_xsc = pl.off_xsc; p.off_part = pl.off_part; p.off_rp = pl.off_rp;
  p.off_bias = pl.off_bias; p.off_res = pl.off_res; p.off_ss = pl.off_ss; p.off_op = pl.off_op;
  gemv_stream_fn fn = act_dtype == SPECTRA_BF16 ? gemv_stream_pick_bf16(pl.NS) : gemv_stream_pick_f16(pl.NS, kpro);
  const int st = ensure_lds_limit((const void*)fn, true);
  if (st != SPECTRA_OK) return st;
  hipLaunchKernelGGL(fn, dim3(pl.grid), dim3(64 * pl.W), pl.lds_bytes, stream, p);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

// ---------------------------------------------------------------------------
// row-owning kernel plan (1 .. 4 activation rows, NF4, Hadamard block 128 or none)
// ---------------------------------------------------------------------------
struct RowsPlan {
  int G, SPR, RPG, XC, W, WR, R, grid, nchunk, cpr, mr;
  bool split;
  uint32_t off_xp, off_xsc, off_sc, off_ss, off_bias, off_res, xp_row, xsc_row, lds_bytes;
};

static gemv_rows_fn rows_fn(int g, int spr, int rpg, int xc, bool split, bool bf, int pro, int mr) {
  if (mr > 1)
    return bf ? gemv_rows_pick_multi_bf16(g, spr, rpg, xc, split, mr) : gemv_rows_pick_multi_f16(g, spr, rpg, xc, split, mr);
  return pro == kProNone ? gemv_rows_pick_plain(g, spr, rpg, xc, split, bf) : gemv_rows_pick_pro(g, spr, rpg, xc, split, pro);
}

// R = ceil(N / CUs) rows per workgroup (one workgroup per CU); lane groups of G = 64 lanes
// (32 when K / 1024 is odd) own RPG rows each.  Preferred: the fewest rows per group whose
// row waves leave spare waves (up to 16 per workgroup) to produce the activations, each
// rotating at most four 512-value chunks (measured: for down_proj 12 row waves with 4
// producers beat 6 row waves of twice the rows with 10); otherwise every wave does both
// jobs.  Several activation rows (mr = 2 .. 4): every wave producing first, all rows'
// chunks loaded up front (measured, down_proj M = 2 / 3 / 4: 7.8 / 9.1 / 10.4 us against
// 7.9 / 9.3 / 10.8 with split producer waves and 9.0-9.5 / 11.3 / 13.0 with two rows per
// group).
static bool plan_rows(int64_t n, int64_t k, int64_t ldp, int64_t lda, int block, int ncu, bool bf, int pro, int mr,
                      RowsPlan* pl) {
  if (k % 1024 != 0 || k > 14336 || ncu <= 0 || block < 32 || block > 1024) return false;
  if ((k / block) % 8 != 0 || (lda * 2) % 16 != 0) return false;  // absmax rows in whole 16-byte chunks
  const int P = (int)(k / 1024);
  const int G = P % 2 == 0 ? 64 : 32;
  const int SPR = P * 32 / G;
  const int64_t R = (n + ncu - 1) / ncu;
  const int nchunk = (int)(k / 512);
  const int cpr = (int)(k / block / 8);
  const int nsmax = SPR == 3 ? 12 : 8;
  if (R * ldp >= (int64_t(1) << 31) || R * lda * 2 >= (int64_t(1) << 31)) return false;
  bool found = false;
  for (int pass = 0; pass < 2 && !found; ++pass) {
    const bool split = mr > 1 ? pass == 1 : pass == 0;
    for (int RPG = 1; RPG <= 8 && !found; RPG *= 2) {
      if (SPR * RPG > nsmax) break;
      const int64_t NG = (R + RPG - 1) / RPG;
      const int64_t WR = (NG * G + 63) / 64;
      if (WR > 16) continue;
      int W, XC;
      if (split) {
        const int nh = std::min(16 - (int)WR, nchunk);
        if (nh < 1) continue;
        XC = (nchunk + nh - 1) / nh;
        XC = XC <= 1 ? 1 : XC <= 2 ? 2 : XC <= 4 ? 4 : 0;
        if (XC == 0 || R * cpr > 64 * nh) continue;
        W = (int)WR + nh;
      } else {
        W = std::max((int)WR, std::min(nchunk, 16));
        XC = (nchunk + W - 1) / W;
        if (XC > 1 || R * cpr > 64 * W) continue;
      }
      if (rows_fn(G, SPR, RPG, XC, split, bf, pro, mr) == nullptr) continue;
      pl->G = G; pl->SPR = SPR; pl->RPG = RPG; pl->XC = XC; pl->W = W; pl->WR = (int)WR; pl->split = split;
      found = true;
    }
  }
  if (!found) return false;
  pl->R = (int)R; pl->nchunk = nchunk; pl->cpr = cpr; pl->mr = mr;
  pl->grid = (int)((n + R - 1) / R);
  // each activation row's rotated pairs and block scales in a slot of its own
  pl->xp_row = align16((uint32_t)(k * 2));
  pl->xsc_row = align16((uint32_t)(k / 128 * 4));
  uint32_t off = kLutBytes;
  pl->off_xp = off;
  off += (uint32_t)mr * pl->xp_row;
  pl->off_xsc = off;
  off += (uint32_t)mr * pl->xsc_row;
  pl->off_sc = off;
  off = align16(off + (uint32_t)(R * (k / block) * 4));
  pl->off_ss = off;
  off = align16(off + (uint32_t)(kMaxWaves * 4));
  pl->off_bias = off;
  off = align16(off + (uint32_t)(R * 4));
  pl->off_res = off;
  off = align16(off + (uint32_t)(R * 2));
  pl->lds_bytes = off;
  return off <= 163840;
}

// The multi-pass row kernel (gemv_rows_lm.h): one workgroup per CU of 8 waves, R = ceil(N /
// CUs) rows each, streamed in passes of 8 x RW rows; for the shapes whose rows outgrow the
// row kernel's plan (the lm_head) and for the fused greedy pick.
struct LmPlan {
  int G, SPR, R, W, grid;
  uint32_t off_xp, off_xsc, off_ss, lds_bytes;
};

static bool rows_lm_serves(const spectra_qweight_t* w, int m, int act_dtype, int kpro,
                           const spectra_gemv_fusion_t* fu, LmPlan* pl) {
  if (m != 1 || w->format != SPECTRA_FMT_NF4 || w->group_size < 32 || w->group_size > 1024) return false;
  if (w->hadamard_block != 0 && w->hadamard_block != 128) return false;
  if (w->outlier_kind == SPECTRA_OUTLIERS_COLUMNS) return false;
  if (w->outlier_kind == SPECTRA_OUTLIERS_CSR && w->csr_nnz >= (int64_t(1) << 29)) return false;
  if (w->bias != nullptr || (fu != nullptr && fu->residual != nullptr)) return false;
  if (kpro != kProNone && kpro != kProRms) return false;
  if (kpro != kProNone && act_dtype != SPECTRA_F16) return false;
  const int64_t k = w->k;
  if (k % 1024 != 0) return false;
  const int P = (int)(k / 1024);
  const int G = P % 2 == 0 ? 64 : 32;
  const int SPR = P * 32 / G;
  if (gemv_rows_lm_pick(G, SPR, act_dtype == SPECTRA_BF16, kpro) == nullptr) return false;
  const int ncu = device_cu_count();
  const int64_t R = (w->n + ncu - 1) / ncu;
  if (R * w->packed_stride >= (int64_t(1) << 31) || R * w->scales_stride * 2 >= (int64_t(1) << 31)) return false;
  pl->G = G; pl->SPR = SPR; pl->R = (int)R; pl->W = kLmWaves;
  pl->grid = (int)((w->n + R - 1) / R);
  uint32_t off = kLutBytes;
  pl->off_xp = off;
  off = align16(off + (uint32_t)(k * 2));
  pl->off_xsc = off;
  off = align16(off + (uint32_t)(k / 128 * 4));
  pl->off_ss = off;
  off = align16(off + (uint32_t)(kMaxWaves * 4));
  pl->lds_bytes = off;
  return off <= 163840;
}

static int rows_lm_launch(const spectra_qweight_t* w, const LmPlan& pl, const void* x, int act_dtype, void* out,
                          hipStream_t stream, const spectra_gemv_fusion_t* fu, int kpro) {
  RowsParams p{};
  p.packed = w->packed; p.ldp = w->packed_stride;
  p.absmax = w->scales; p.lda = w->scales_stride;
  const bool csr = w->outlier_kind == SPECTRA_OUTLIERS_CSR && w->csr_nnz > 0;
  p.rowptr = csr ? w->csr_rowptr : nullptr;
  p.ccol = csr ? w->csr_col : nullptr;
  p.cval = csr ? w->csr_val : nullptr;
  p.csr = csr ? 1 : 0;
  p.csr_nnz = csr ? (int)w->csr_nnz : 0;
  p.bias = nullptr;
  p.x = x; p.out = out;
  p.nw = fu ? fu->norm_weight : nullptr;
  p.res = nullptr;
  p.eps = fu ? fu->eps : 0.0f;
  p.had = w->hadamard_block;
  p.out_scale = w->hadamard_block ? (float)(1.0 / std::sqrt((double)w->hadamard_block)) : 1.0f;
  p.n = (int)w->n; p.k = (int)w->k;
  p.R = 0;  // the producers stage no block scales: the row waves read them with the runs
  p.nchunk = (int)(w->k / 512);
  int gs = 0;
  while ((1 << gs) < w->group_size) ++gs;
  p.gshift = gs;
  p.marlin = w->marlin_layout ? 1 : 0;
  p.cpr = (int)(w->k / w->group_size / 8);
  p.cmagic = p.cpr > 0 ? (65536 + p.cpr - 1) / p.cpr : 0;
  p.off_xp = pl.off_xp; p.off_xsc = pl.off_xsc; p.off_ss = pl.off_ss;
  p.wr = 0;
  p.W = pl.W;
  unsigned long long* akey = fu != nullptr ? (unsigned long long*)fu->argmax_key : nullptr;
  const gemv_rows_lm_fn fn = gemv_rows_lm_pick(pl.G, pl.SPR, act_dtype == SPECTRA_BF16, kpro);
  const int st = ensure_lds_limit((const void*)fn, true);
  if (st != SPECTRA_OK) return st;
  hipLaunchKernelGGL(fn, dim3(pl.grid), dim3(64 * pl.W), pl.lds_bytes, stream, p, pl.R, akey);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

// several rows (m = 2 .. 4): no prologue (each row would need its own norm)
static bool rows_serves(const spectra_qweight_t* w, int m, int act_dtype, int kpro, const spectra_gemv_fusion_t* fu,
                        RowsPlan* pl) {
  if (m < 1 || m > 4 || w->format != SPECTRA_FMT_NF4 || w->group_size < 32) return false;
  if (m > 1 && kpro != kProNone) return false;
  if (m > 1 && fu != nullptr && fu->residual != nullptr && (int64_t)(m - 1) * fu->residual_stride + w->n >= (int64_t(1) << 31))
    return false;  // the residual's byte offsets in 32 bits
  if (w->hadamard_block != 0 && w->hadamard_block != 128) return false;
  if (w->outlier_kind == SPECTRA_OUTLIERS_COLUMNS) return false;
  if (w->outlier_kind == SPECTRA_OUTLIERS_CSR && w->csr_nnz >= (int64_t(1) << 29)) return false;
  if (!ptr_aligned(w->scales, 16)) return false;
  if (kpro != kProNone && act_dtype != SPECTRA_F16) return false;
  return plan_rows(w->n, w->k, w->packed_stride, w->scales_stride, w->group_size, device_cu_count(),
                   act_dtype == SPECTRA_BF16, kpro, m, pl);
}

static int rows_launch(const spectra_qweight_t* w, const RowsPlan& pl, const void* x, int64_t ldx, int act_dtype,
                       void* out, int64_t ldo, hipStream_t stream, const spectra_gemv_fusion_t* fu, int kpro) {
  RowsParams p;
  p.packed = w->packed; p.ldp = w->packed_stride;
  p.absmax = w->scales; p.lda = w->scales_stride;
  const bool csr = w->outlier_kind == SPECTRA_OUTLIERS_CSR && w->csr_nnz > 0;
  p.rowptr = csr ? w->csr_rowptr : nullptr;
  p.ccol = csr ? w->csr_col : nullptr;
  p.cval = csr ? w->csr_val : nullptr;
  p.csr = csr ? 1 : 0;
  p.csr_nnz = csr ? (int)w->csr_nnz : 0;
  p.bias = w->bias; p.bias_dt = w->bias_dtype;
  p.x = x; p.out = out;
  p.ldx = ldx; p.ldo = ldo;
  p.ldr = fu ? fu->residual_stride : 0;
  p.xp_row = pl.xp_row; p.xsc_row = pl.xsc_row;
  p.nw = fu ? fu->norm_weight : nullptr;
  p.res = fu ? fu->residual : nullptr;
  p.eps = fu ? fu->eps : 0.0f;
  p.had = w->hadamard_block;
  p.out_scale = w->hadamard_block ? (float)(1.0 / std::sqrt((double)w->hadamard_block)) : 1.0f;
  p.n = (int)w->n; p.k = (int)w->k;
  p.R = pl.R; p.nchunk = pl.nchunk;
  int gs = 0;
  while ((1 << gs) < w->group_size) ++gs;
  p.gshift = gs;
  p.marlin = w->marlin_layout ? 1 : 0;
  p.cpr = pl.cpr;
  p.cmagic = (65536 + pl.cpr - 1) / pl.cpr;
  p.off_xp = pl.off_xp; p.off_xsc = pl.off_xsc; p.off_sc = pl.off_sc; p.off_ss = pl.off_ss;
  p.off_bias = pl.off_bias; p.off_res = pl.off_res;
  p.wr = pl.WR;
  p.W = pl.W;
  const gemv_rows_fn fn = rows_fn(pl.G, pl.SPR, pl.RPG, pl.XC, pl.split, act_dtype == SPECTRA_BF16, kpro, pl.mr);
  const int st = ensure_lds_limit((const void*)fn, true);
  if (st != SPECTRA_OK) return st;
  hipLaunchKernelGGL(fn, dim3(pl.grid), dim3(64 * pl.W), pl.lds_bytes, stream, p);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

// the stream kernel serves one row of NF4 activations with CSR outliers or none, K a
// multiple of 1024 up to 16384, and at most kStreamMaxSlots rows per lane
static bool stream_serves(const spectra_qweight_t* w, int m, StreamPlan* pl) {
  if (m != 1 || w->format != SPECTRA_FMT_NF4 || w->group_size < 32) return false;
  if (w->outlier_kind == SPECTRA_OUTLIERS_COLUMNS) return false;
  if (w->outlier_kind == SPECTRA_OUTLIERS_CSR && w->csr_nnz >= (int64_t(1) << 29)) return false;
  if (!ptr_aligned(w->scales, 16)) return false;
  return plan_stream(w->n, w->k, w->packed_stride, w->scales_stride, w->group_size, device_cu_count(), pl);
}

// workgroups of the plan for m activation rows (0 when the family does not serve the shape);
// the descriptor is already validated
int gemv_plan_grid(const spectra_qweight_t* w, int m) {
  RowsPlan rp;
  if (rows_serves(w, m, SPECTRA_F16, kProNone, nullptr, &rp)) return rp.grid;
  StreamPlan sp;
  if (stream_serves(w, m, &sp)) return sp.grid;
  const bool csr = w->outlier_kind == SPECTRA_OUTLIERS_CSR && w->csr_nnz > 0;
  const bool outliers = w->outlier_kind == SPECTRA_OUTLIERS_COLUMNS || csr;
  GemvPlan pl;
  if (!plan_gemv(w->n, w->k, m, outliers, csr, &pl, gemv_rpw_two_per_cu(w->format, kProNone))) return 0;
  return pl.grid;
}

int gemv_launch(const spectra_qweight_t* w, const void* x, int64_t ldx, int m, int act_dtype, void* out,
                int64_t ldo, hipStream_t stream, const spectra_gemv_fusion_t* fu) {
  const bool outliers = w->outlier_kind == SPECTRA_OUTLIERS_COLUMNS ||
                        (w->outlier_kind == SPECTRA_OUTLIERS_CSR && w->csr_nnz > 0);
  GemvPlan pl;
  const bool csr = outliers && w->outlier_kind == SPECTRA_OUTLIERS_CSR;
  const int pro = fu ? fu->prologue : SPECTRA_PROLOGUE_NONE;
  const int kpro = pro == SPECTRA_PROLOGUE_RMSNORM ? kProRms : pro == SPECTRA_PROLOGUE_SILU_MUL ? kProSiluMul : kProNone;
  if (!plan_gemv(w->n, w->k, m, outliers, csr, &pl, gemv_rpw_two_per_cu(w->format, kpro)))
    return fail(SPECTRA_ERR_UNSUPPORTED, "shape not served by the GEMV family (use the GEMM family)");
  SPECTRA_REQUIRE(w->hadamard_block == 0 || w->hadamard_block <= 512, "GEMV serves hadamard_block <= 512");
  SPECTRA_REQUIRE(ptr_aligned(x, 16) && ldx % 8 == 0, "x must be 16-byte aligned with a row stride multiple of 8");
  SPECTRA_REQUIRE((int64_t)m * ldx < (int64_t(1) << 30), "x rows must span fewer than 2^30 elements");
  SPECTRA_REQUIRE(ptr_aligned(w->packed, 16) && w->packed_stride % 16 == 0,
                  "packed weights must be 16-byte aligned with a row stride multiple of 16");
  if (csr)
    SPECTRA_REQUIRE(ptr_aligned(w->csr_col, 16) && ptr_aligned(w->csr_val, 8) && w->csr_nnz < (int64_t(1) << 31),
                    "CSR columns must be 16-byte and values 8-byte aligned (nnz < 2^31)");
  // the kernels pair each format with its own outlier kind and scale scheme: Format B
  // (NF4, blocks >= 64, CSR outliers), Format A (groups of 32, dense outlier columns)
  // (the greedy pick rides on the epilogues of the multi-pass row kernel and the multi-row kernel)
  const bool pick = fu != nullptr && fu->argmax_key != nullptr;
  RowsPlan rp;
  if (!pick && rows_serves(w, m, act_dtype, kpro, fu, &rp))
    return rows_launch(w, rp, x, ldx, act_dtype, out, ldo, stream, fu, kpro);
  LmPlan lp;
  if (rows_lm_serves(w, m, act_dtype, kpro, fu, &lp)) return rows_lm_launch(w, lp, x, act_dtype, out, stream, fu, kpro);
  StreamPlan sp;
  if (!pick && stream_serves(w, m, &sp)) return stream_launch(w, sp, x, act_dtype, out, stream, fu, kpro);
  if (w->format == SPECTRA_FMT_NF4 && w->group_size < 64)
    return fail(SPECTRA_ERR_UNSUPPORTED, "the GEMV family needs an NF4 block of at least 64");
  if (outliers && (w->format == SPECTRA_FMT_NF4) != csr)
    return fail(SPECTRA_ERR_UNSUPPORTED, "the GEMV family serves CSR outliers with NF4 and dense columns with Format A");
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
  p.csr_nnz = csr ? (int)w->csr_nnz : 0;
  p.n_out = w->num_outliers; p.ow_dt = w->outlier_w_dtype; p.bias_dt = w->bias_dtype; p.act_dt = act_dtype;
  p.R = pl.R; p.S = pl.S; p.G = pl.G; p.ocap = pl.ocap;
  p.s_magic = (256 + pl.S - 1) / pl.S;
  p.off_xp = pl.off_xp; p.off_xsc = pl.off_xsc; p.off_part = pl.off_part;
  p.off_rp = pl.off_rp; p.off_bias = pl.off_bias; p.off_oprod = pl.off_oprod;
  p.off_ss = pl.off_ss; p.off_res = pl.off_res;
  p.out_scale = w->hadamard_block ? (float)(1.0 / std::sqrt((double)w->hadamard_block)) : 1.0f;
  p.inv_n_out = w->num_outliers > 0 ? 1.0f / (float)w->num_outliers : 1.0f;
  p.nw = fu ? fu->norm_weight : nullptr;
  p.eps = fu ? fu->eps : 0.0f;
  p.res = fu ? fu->residual : nullptr;
  p.ldr = fu ? fu->residual_stride : 0;
  p.akey = pick ? (unsigned long long*)fu->argmax_key : nullptr;
  gemv_fn fn = pro != SPECTRA_PROLOGUE_NONE
                   ? gemv_pick_f16_pro(pro == SPECTRA_PROLOGUE_RMSNORM ? kProRms : kProSiluMul, pl.rpw, pl.wide)
               : act_dtype == SPECTRA_BF16 ? gemv_pick_bf16(w->format, pl.mt, pl.rpw, pl.wide)
                                           : gemv_pick_f16(w->format, pl.mt, pl.rpw, pl.wide);
  const int st = ensure_lds_limit((const void*)fn, true);
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
  return spectra::gemv_launch(w, x, ldx, m, act_dtype, out, ldo, (hipStream_t)stream, nullptr);
}

extern "C" int spectra_w4a16_gemv_fused(const spectra_qweight_t* w, const void* x, int64_t ldx, int32_t m,
                                        int32_t act_dtype, const spectra_gemv_fusion_t* fusion, void* out,
                                        int64_t ldo, spectra_stream_t stream) {
  int st = spectra::validate_qweight(w);
  if (st != SPECTRA_OK) return st;
  SPECTRA_REQUIRE(x != nullptr && out != nullptr && fusion != nullptr, "x/out/fusion is NULL");
  SPECTRA_REQUIRE(m >= 1 && m <= 4, "the GEMV family serves 1 <= m <= 4");
  SPECTRA_REQUIRE(act_dtype == SPECTRA_F16 || act_dtype == SPECTRA_BF16, "activations must be fp16 or bf16");
  const int pro = fusion->prologue;
  SPECTRA_REQUIRE(pro == SPECTRA_PROLOGUE_NONE || pro == SPECTRA_PROLOGUE_RMSNORM || pro == SPECTRA_PROLOGUE_SILU_MUL,
                  "unknown prologue");
  SPECTRA_REQUIRE(ldx >= (pro == SPECTRA_PROLOGUE_SILU_MUL ? 2 * w->k : w->k) && ldo >= w->n, "row stride too small");
  if (pro != SPECTRA_PROLOGUE_NONE) {
    if (m != 1 || act_dtype != SPECTRA_F16 || w->format != SPECTRA_FMT_NF4)
      return spectra::fail(SPECTRA_ERR_UNSUPPORTED, "fused prologues serve one fp16 row of an NF4 weight");
    if (pro == SPECTRA_PROLOGUE_RMSNORM)
      SPECTRA_REQUIRE(fusion->norm_weight != nullptr && (reinterpret_cast<uintptr_t>(fusion->norm_weight) & 15) == 0,
                      "RMSNorm needs a 16-byte aligned fp16 weight");
  }
  if (fusion->residual != nullptr) SPECTRA_REQUIRE(fusion->residual_stride >= w->n, "residual row stride too small");
  if (fusion->argmax_key != nullptr)
    SPECTRA_REQUIRE(m == 1 && (reinterpret_cast<uintptr_t>(fusion->argmax_key) & 7) == 0 && w->n < (int64_t(1) << 31),
                    "the fused greedy pick serves one row, with 8-byte aligned slots");
  return spectra::gemv_launch(w, x, ldx, m, act_dtype, out, ldo, (hipStream_t)stream, fusion);
}
