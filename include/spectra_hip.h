/*
 * spectra_hip.h -- C ABI of the MI355X (gfx950) W4A16 quantized-linear library.
 *
 * Plain pointers, sizes and strides only: no torch types cross this boundary.
 * Every device pointer is a HIP device address; every call is asynchronous on
 * the given stream (0 = the null stream), performs no host synchronisation and
 * no device allocation, so it can be captured into a HIP graph.
 *
 * Return value: SPECTRA_OK (0) on success, a negative spectra_status_t on
 * failure; spectra_last_error() then returns a message (thread-local).
 *
 * Reference interfaces replaced (paths in the NeuraCryption/SPECTRA tree):
 *   spectra_w4a16_gemv      <- spectra/kernels.py:132-184 fused_w4a16_gemv_hdsq
 *   spectra_w4a16_gemm      <- spectra/kernels.py:333-389 batched_w4a16_gemm
 *   spectra_w4a16_linear    <- spectra/engine.py:90-124  SpectraFusedLinear.forward
 *   spectra_w4_dequant      <- tests/test_kernels.py:31-39, spectra/engine.py:185-210
 *   spectra_quantize_group32<- spectra/compressor.py:71-156
 *   spectra_quantize_nf4    <- Format B quantizer (no reference code; built on
 *                              compressor.py:22-42 codebook and FWHT)
 *   spectra_fwht_rows       <- spectra/compressor.py:29-42 fast_walsh_hadamard_transform
 *   spectra_outlier_columns <- spectra/compressor.py:158-215 _isolate_hdsq_outliers
 *   spectra_w4_embedding    <- spectra/engine.py:127-212 SpectraFusedEmbedding.forward
 *   spectra_rmsnorm, spectra_rope_append, spectra_attend_decode, spectra_silu_mul
 *                           <- the Inductor-fused RMSNorm / RoPE / SiLU submodules and the
 *                              static-cache attention of the decode step (engine.py:1240-1250,
 *                              :1387-1415)
 *   spectra_greedy_next, spectra_greedy_finish
 *                           <- spectra/engine.py:1690-1697 sample_token (temperature 0)
 *   spectra_kv4_quantize, spectra_kv4_dequantize, spectra_attend_decode_q4
 *                           <- spectra/engine.py:614-700 the 4-bit KV cache
 */
#ifndef SPECTRA_HIP_H_
#define SPECTRA_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* spectra_stream_t; /* == hipStream_t */

typedef enum {
  SPECTRA_OK = 0,
  SPECTRA_ERR_INVALID = -1,     /* bad argument (shape, dtype, stride, alignment) */
  SPECTRA_ERR_UNSUPPORTED = -2, /* valid but not served by this build */
  SPECTRA_ERR_HIP = -3,         /* a HIP runtime call failed */
  SPECTRA_ERR_WORKSPACE = -4    /* workspace missing or too small */
} spectra_status_t;

typedef enum { SPECTRA_F16 = 0, SPECTRA_BF16 = 1, SPECTRA_F32 = 2 } spectra_dtype_t;

typedef enum {
  SPECTRA_FMT_ASYM_G32 = 0, /* Format A: (q - z) * s, group 32, fp16 scale, uint8 zero */
  SPECTRA_FMT_NF4 = 1       /* Format B: NF4 code * fp16 absmax, block = group_size */
} spectra_format_t;

typedef enum {
  SPECTRA_OUTLIERS_NONE = 0,
  SPECTRA_OUTLIERS_COLUMNS = 1, /* Format A: idx int64 [n_out] + dense w [N, n_out] */
  SPECTRA_OUTLIERS_CSR = 2      /* Format B: row_ptr int32 [N+1], col int32, val fp16 */
} spectra_outlier_kind_t;

/*
 * A quantized weight W[N, K] (out_features x in_features) and its side tensors.
 * Strides are in elements of the pointed-to type; the inner stride of every
 * 2-D operand is 1.
 */
typedef struct spectra_qweight {
  int64_t n, k;
  int32_t format;         /* spectra_format_t */
  int32_t group_size;     /* 32 (Format A) or the NF4 block size (64) */
  int32_t hadamard_block; /* 0, or a power of two in [2, 1024] dividing k (GEMV: <= 512) */
  int32_t marlin_layout;  /* 1: byte j of a 32-run = q[j] | q[j+16]<<4; 0: q[2j] | q[2j+1]<<4 */
  const uint8_t* packed;  int64_t packed_stride;  /* uint8 [N, K/2] */
  const uint16_t* scales; int64_t scales_stride;  /* fp16 [N, K/group] (absmax for NF4) */
  const uint8_t* zeros;   int64_t zeros_stride;   /* uint8 [N, K/32] (Format A only) */
  int32_t outlier_kind;   /* spectra_outlier_kind_t */
  int32_t num_outliers;   /* COLUMNS: n_out */
  const int64_t* outlier_idx;                      /* COLUMNS: int64 [n_out], ascending */
  const void* outlier_w; int64_t outlier_w_stride; /* COLUMNS: [N, n_out] */
  int32_t outlier_w_dtype;                         /* COLUMNS: SPECTRA_F16 or SPECTRA_BF16 */
  const int32_t* csr_rowptr;                       /* CSR: int32 [N+1] */
  const int32_t* csr_col;                          /* CSR: int32 [nnz], ascending per row */
  const uint16_t* csr_val;                         /* CSR: fp16 [nnz] */
  int64_t csr_nnz;                                 /* CSR: number of stored outliers */
  const void* bias; int32_t bias_dtype;            /* optional [N] */
} spectra_qweight_t;

/* Library identity and the last error message of the calling thread. */
const char* spectra_version(void);
const char* spectra_last_error(void);

/*
 * Decode GEMV family (M = 1..4 rows of activations):
 *   out[m, :] = FWHT_hb(x[m, :]) . W_eff^T + bias,   fp32 accumulation, RNE store.
 * x: act_dtype (F16/BF16) [m, K] row stride ldx; out: act_dtype [m, N] row stride ldo.
 * Replaces kernels.py:132-184 (which serves one row; this serves up to 4).
 */
int spectra_w4a16_gemv(const spectra_qweight_t* w, const void* x, int64_t ldx, int32_t m,
                       int32_t act_dtype, void* out, int64_t ldo, spectra_stream_t stream);

/*
 * The GEMV with the work around a decoder's linears fused in (no reference counterpart:
 * the reference runs these as separate Inductor-fused submodules, engine.py:1240-1250):
 *   prologue RMSNORM:  x is the residual stream h; the product uses
 *                      rmsnorm(h) = h * rsqrt(mean(h^2) + eps) * norm_weight, with the
 *                      row scale applied to the accumulated output (one fp16 rounding of
 *                      the normalised activations fewer than the separate kernels);
 *   prologue SILU_MUL: x rows hold [g | u] (2K values, ldx >= 2K); the product uses
 *                      fp16(silu(g) * u), bit-identical to spectra_silu_mul;
 *   residual:          out = act(residual + act(y)) (act = the activation dtype), residual
 *                      [m, N] row stride residual_stride, may alias out (in-place update).
 * Prologues serve m = 1, fp16 activations and NF4 weights (SPECTRA_ERR_UNSUPPORTED
 * otherwise); the residual serves every GEMV.
 *   argmax_key:        optional (m = 1): the outputs' greedy pick folded into the epilogue.
 *                      Points at SPECTRA_ARGMAX_SLOTS slots of SPECTRA_ARGMAX_STRIDE device
 *                      uint64 each (the first of each slot is used; one slot per 256 bytes,
 *                      so that the slots' atomics spread over the memory channels), all 0
 *                      before the call (spectra_greedy_finish leaves them 0); each wave
 *                      merges its best (value, index) of the stored outputs into one slot
 *                      with an atomic max.  spectra_greedy_finish then reads the token.
 */
#define SPECTRA_ARGMAX_SLOTS 256
#define SPECTRA_ARGMAX_STRIDE 32
typedef enum {
  SPECTRA_PROLOGUE_NONE = 0,
  SPECTRA_PROLOGUE_RMSNORM = 1,
  SPECTRA_PROLOGUE_SILU_MUL = 2
} spectra_prologue_t;

typedef struct spectra_gemv_fusion {
  int32_t prologue;          /* spectra_prologue_t */
  float eps;                 /* RMSNORM */
  const uint16_t* norm_weight; /* RMSNORM: fp16 [K], 16-byte aligned */
  const void* residual;      /* optional, act dtype [m, N] */
  int64_t residual_stride;
  void* argmax_key;          /* optional: SPECTRA_ARGMAX_SLOTS x SPECTRA_ARGMAX_STRIDE uint64, 8-byte aligned */
} spectra_gemv_fusion_t;

int spectra_w4a16_gemv_fused(const spectra_qweight_t* w, const void* x, int64_t ldx, int32_t m,
                             int32_t act_dtype, const spectra_gemv_fusion_t* fusion, void* out, int64_t ldo,
                             spectra_stream_t stream);

/*
 * Batched / prefill GEMM family (any M >= 1, MFMA):
 *   out = FWHT_hb(a) . W_eff^T + bias,   fp32 accumulation.
 * a: act_dtype [m, K] row stride lda; out: act_dtype [m, N] row stride ldo.
 * 2 <= m <= 16: small-batch stream; otherwise the hand-written GEMM (fp16 operands); from
 * m >= 512, when the workspace holds it, W_eff dequantized into the workspace in act_dtype
 * and one hipBLASLt GEMM on it (the reference kernel's operand rounding).
 * workspace: device scratch of spectra_w4a16_gemm_workspace() bytes, which serves every
 * family (from m >= 512 it includes N*K*2 + m*K*2 bytes + 32 MiB for the library path); a
 * smaller one that holds the hand-written GEMM's buffers runs that GEMM.  May be NULL when
 * the size is 0.  Replaces kernels.py:333-389.
 */
size_t spectra_w4a16_gemm_workspace(const spectra_qweight_t* w, int64_t m, int32_t act_dtype);
int spectra_w4a16_gemm(const spectra_qweight_t* w, const void* a, int64_t lda, int64_t m,
                       int32_t act_dtype, void* out, int64_t ldo, void* workspace,
                       size_t workspace_bytes, spectra_stream_t stream);

/*
 * Module dispatch (engine.py:90-124): m <= 4 -> GEMV family, else GEMM family; 2 <= m <= 4
 * rows of a shape that only the older multi-row GEMV kernels serve, with a plan of more
 * than one workgroup per CU, go to the GEMM entry's small-batch MFMA family instead, when
 * it serves the operands and the workspace is large enough (otherwise they stay on the
 * GEMV family).
 * workspace as for spectra_w4a16_gemm (sized by spectra_w4a16_gemm_workspace).
 */
int spectra_w4a16_linear(const spectra_qweight_t* w, const void* x, int64_t ldx, int64_t m,
                         int32_t act_dtype, void* out, int64_t ldo, void* workspace,
                         size_t workspace_bytes, spectra_stream_t stream);

/*
 * spectra_w4a16_linear without a workspace argument and without any allocation.  No
 * counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc).  The
 * workspace is a file-scope device array of SPECTRA_NOALLOC_SCRATCH_BYTES, one copy per GPU,
 * held until the process ends; its address is looked up on the first call on each device.
 * Calls whose workspace (spectra_w4a16_gemm_workspace) exceeds it return
 * SPECTRA_ERR_WORKSPACE before launching anything (m <= 16 on every Llama-3.2-3B shape fits).
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU (two streams,
 * two threads) race and give undefined results.  No part of the array needs to start at
 * zero (every kernel writes what it reads), so nothing is cleared between calls.
 */
#define SPECTRA_NOALLOC_SCRATCH_BYTES (8u << 20)
int spectra_w4a16_linear_noalloc(const spectra_qweight_t* w, const void* x, int64_t ldx, int64_t m,
                                 int32_t act_dtype, void* out, int64_t ldo, spectra_stream_t stream);

/*
 * Materialise W_eff [N, K] in out_dtype (F16/BF16/F32), bit-exact:
 *   Format A: round((q - z) * s in fp32), then outlier columns := round(outlier_w)
 *   Format B: round(fp32(NF4[q]) * fp32(absmax)), then CSR positions := round(val)
 * Bias is ignored.  (tests/test_kernels.py:31-39, engine.py:185-210)
 */
int spectra_w4_dequant(const spectra_qweight_t* w, void* out, int64_t ldo, int32_t out_dtype,
                       spectra_stream_t stream);

/*
 * Embedding gather (engine.py:127-212): out[b, :] = W_eff[ids[b], :] for b < n_ids,
 * bit-identical to the same rows of spectra_w4_dequant (ids: device int64 [n_ids]; an id
 * outside [0, N) yields a row of zeros).  out: out_dtype [n_ids, K], row stride ldo.
 */
int spectra_w4_embedding(const spectra_qweight_t* w, const int64_t* ids, int64_t n_ids, void* out, int64_t ldo,
                         int32_t out_dtype, spectra_stream_t stream);

/*
 * Format A quantizer (compressor.py:71-156): w [n, k] (F16/BF16/F32, row stride ldw);
 * columns listed in outlier_idx (int64 [n_out], may be NULL) are zeroed first.
 * Outputs: packed uint8 [n, k/2] (marlin layout), scales fp16 [n, k/32],
 * packed_zeros uint8 [n, ceil(k/64)] (two zero points per byte).  group_size must be 32.
 */
int spectra_quantize_group32(const void* w, int64_t ldw, int32_t w_dtype, int64_t n, int64_t k,
                             int32_t group_size, const int64_t* outlier_idx, int32_t n_out,
                             uint8_t* packed, uint16_t* scales, uint8_t* packed_zeros,
                             spectra_stream_t stream);

/*
 * Format B quantizer: w [n, k] (F16/BF16/F32, row stride ldw) -> optional blockwise
 * FWHT of each row (hadamard_block) -> CSR positions (csr_rowptr/csr_col, may be
 * NULL for none) are recorded into csr_val (fp16) and zeroed -> fp16 absmax per
 * blocksize block -> nearest NF4 code (fp32 distances, lowest index on ties),
 * packed per marlin_layout.  Outputs packed uint8 [n, k/2], absmax fp16 [n, k/blocksize].
 */
int spectra_quantize_nf4(const void* w, int64_t ldw, int32_t w_dtype, int64_t n, int64_t k,
                         int32_t blocksize, int32_t hadamard_block, int32_t marlin_layout,
                         const int32_t* csr_rowptr, const int32_t* csr_col, uint16_t* csr_val,
                         uint8_t* packed, uint16_t* absmax, spectra_stream_t stream);

/*
 * Blockwise normalised FWHT of rows (compressor.py:29-42), fp32 arithmetic in the
 * reference's butterfly order, division by fp32(sqrt(block)).
 * x [rows, k] in_dtype (row stride ldx) -> out [rows, k] out_dtype (row stride ldo).
 * block: power of two in [2, 1024] dividing k.
 */
int spectra_fwht_rows(const void* x, int64_t ldx, int32_t in_dtype, int64_t rows, int64_t k,
                      int32_t block, void* out, int64_t ldo, int32_t out_dtype,
                      spectra_stream_t stream);

/*
 * Outlier-column selection of the compressor (compressor.py:158-215): column saliency
 * sqrt(sum_r w[r, j]^2) (times norm_vector[j] when given; fp32, 4096-row chunks),
 * kurtosis of the saliencies (clamped to >= 1), ratio = base_ratio, or with `adaptive`
 * clamp(fp32(base_ratio * (1 + 0.15 log1p(max(0, kurtosis - 3)))), 0.005, 0.03),
 * n_out = max(1, round-half-even(K * ratio)) columns of largest saliency (ties at the
 * threshold: lowest column first), written ascending.
 * w [n, k] (F16/BF16/F32, row stride ldw); norm_vector fp32 [k] or NULL.
 * Outputs (device): idx int32 [k] (the first *n_out entries are valid), n_out int32 [1],
 * stats fp32 [2] = {ratio, kurtosis}.  workspace: spectra_outlier_columns_workspace(k)
 * bytes.  k <= 32768.
 */
size_t spectra_outlier_columns_workspace(int64_t k);
int spectra_outlier_columns(const void* w, int64_t ldw, int32_t w_dtype, int64_t n, int64_t k,
                            const float* norm_vector, double base_ratio, int32_t adaptive, int32_t* idx,
                            int32_t* n_out, float* stats, void* workspace, size_t workspace_bytes,
                            spectra_stream_t stream);

/* ---- decode-layer kernels between the quantized linears ----------------------------------
 * Replace the reference's Inductor-fused non-linear submodules (RMSNorm, SiLU, RoPE;
 * spectra/engine.py:1240-1250) and its static-cache attention for graph replay
 * (engine.py:1387-1415).  All activations fp16.  The token positions are device int64, so
 * a decode step captures into a HIP graph with no host-side value.
 */

/* Optional residual add then RMSNorm of `rows` rows: when residual != NULL,
 * h = fp16(h + residual) in place; x = fp16(h * rsqrt(mean(h^2) + eps) * weight).
 * h, residual, x [rows, hidden] contiguous; weight fp32 [hidden]. */
int spectra_rmsnorm(void* h, const void* residual, const float* weight, float eps, int64_t rows, int64_t hidden,
                    void* x, spectra_stream_t stream);

/* Rotary embedding (pairs (i, i + head_dim/2), fp32 math) of the q and k heads of `tokens`
 * fused-QKV rows (row stride ldqkv: heads q heads, kv_heads k heads, kv_heads v heads), and
 * the KV-cache append at pos[t]: q_rot [tokens, heads, head_dim]; k_cache and v_cache
 * [kv_heads, max_seq, head_dim].  cos_t, sin_t fp32 [max_seq, head_dim/2].  A position
 * outside [0, max_seq) writes nothing. */
int spectra_rope_append(const void* qkv, int64_t ldqkv, int64_t tokens, const int64_t* pos, const float* cos_t,
                        const float* sin_t, int32_t heads, int32_t kv_heads, int32_t head_dim, int32_t max_seq,
                        void* q_rot, void* k_cache, void* v_cache, spectra_stream_t stream);

/* Batch-1 decode attention on the fused-QKV row of the decoded token (qkv: heads q heads,
 * kv_heads k heads, kv_heads v heads of head_dim fp16 each) at position *pos (device int64):
 * rotates q and the new k (as spectra_rope_append; cos_t / sin_t NULL = no rotation),
 * appends k and v at *pos to k_cache / v_cache [kv_heads, max_seq, head_dim], and writes
 * out [heads, head_dim] fp16 = softmax(q k^T / sqrt(head_dim)) v over positions [0, *pos]
 * (fp32 softmax; grouped-query: query head h reads KV head h / (heads / kv_heads); 1, 2, 3,
 * 4, 6 or 8 query heads per KV head; head_dim 16, 32, 64, 128 or 256; operands 16-byte aligned).
 * One kernel: spectra_attend_spans(max_seq) workgroups of 64 positions per KV head; the
 * last of a head to finish merges the spans (log-sum-exp).  workspace: >=
 * spectra_attend_workspace(heads, head_dim, max_seq) bytes, 16-byte aligned: per-KV-head
 * arrival counters at its start (the same offset for every shape), then the span partials.
 * ZERO the workspace before its first use; every complete call leaves the counters at zero
 * again, so a workspace stays valid for later calls of any shape that fits it.  Calls
 * sharing a workspace must not overlap.  A *pos outside
 * [0, max_seq) appends nothing (the caches are left as they are) and yields NaN outputs. */
int32_t spectra_attend_spans(int32_t max_seq);
size_t spectra_attend_workspace(int32_t heads, int32_t head_dim, int32_t max_seq);
int spectra_attend_decode(const void* qkv, const int64_t* pos, const float* cos_t, const float* sin_t, int32_t heads,
                          int32_t kv_heads, int32_t head_dim, int32_t max_seq, void* k_cache, void* v_cache,
                          void* workspace, size_t workspace_bytes, void* out, spectra_stream_t stream);

/* The 4-bit KV cache (engine.py:614-680 SpectraGroup32QuantizedLayer / :683-700
 * SpectraQuantizedCache).  Quantizer: per row of the head dimension, groups of 32,
 * asymmetric min-max codes 0..15 with fp16 scale and uint8 zero point, two codes per byte
 * (even index low nibble), bit-identical to the reference's _quantize on fp16 values (whose
 * 1e-8 threshold and scale floor are 0 in fp16: a constant group gets scale 0).  Dequant:
 * (q - z) * s rounded to bf16, the reference's _dequantize.
 * spectra_kv4_quantize: x fp16 rows of d values, row r of head h at x + h * x_head_stride +
 * r * ldx; outputs at row h * out_head_rows + r: codes uint8 [*, d/2], scales fp16
 * [*, d/32], zeros uint8 [*, d/32].  spectra_kv4_dequantize: bf16 [rows, d].
 * spectra_attend_decode_q4: spectra_attend_decode over a 4-bit cache: every position in
 * codes / scales / zeros [kv_heads, max_seq, ...] (the new token quantized as it is
 * appended), the last `window` positions also in fp16 rings k_window / v_window
 * [kv_heads, window, head_dim] (slot = position % window), which attention reads for them
 * (the reference keeps a recent window unquantized); older positions are read through the
 * dequant.  RoPE tables required; head_dim 32, 64, 128 or 256 (groups of 32 dims). */
int spectra_kv4_quantize(const void* x, int64_t ldx, int64_t rows, int32_t heads, int64_t x_head_stride, int32_t d,
                         void* codes, void* scales, void* zeros, int64_t out_head_rows, spectra_stream_t stream);
int spectra_kv4_dequantize(const void* codes, const void* scales, const void* zeros, int64_t rows, int32_t d,
                           void* out_bf16, spectra_stream_t stream);
int spectra_attend_decode_q4(const void* qkv, const int64_t* pos, const float* cos_t, const float* sin_t,
                             int32_t heads, int32_t kv_heads, int32_t head_dim, int32_t max_seq, int32_t window,
                             void* k_window, void* v_window, void* k_codes, void* v_codes, void* k_scales,
                             void* v_scales, void* k_zeros, void* v_zeros, void* workspace, size_t workspace_bytes,
                             void* out, spectra_stream_t stream);

/* act [rows, inter] = fp16(silu(g) * u) where g = gate_up[:, :inter], u = gate_up[:, inter:]
 * (row stride ldgu >= 2 * inter). */
int spectra_silu_mul(const void* gate_up, int64_t ldgu, int64_t rows, int64_t inter, void* act,
                     spectra_stream_t stream);

/* Greedy sampling of one decode step (the temperature-0 branch of the reference's
 * sample_token, engine.py:1690-1697):
 * *token = index of the largest of n fp16 logits (16-byte aligned; lowest index among equal
 * maxima, NaN counts as largest, as torch.argmax).  When pos != NULL: history[*pos + 1] =
 * *token (if inside [0, hist_len) and history != NULL), then *pos += 1. */
int spectra_greedy_next(const void* logits, int64_t n, int64_t* token, int64_t* history, int64_t hist_len,
                        int64_t* pos, spectra_stream_t stream);

/* spectra_greedy_next for outputs whose pick a fused GEMV already gathered into argmax_key
 * (spectra_gemv_fusion_t): same token, history and position update, same tie and NaN
 * rule; resets the slots to 0 for the next call.  One 64-thread launch
 * instead of a scan of the logits (engine.py:1690-1697, with the argmax in the lm_head). */
int spectra_greedy_finish(void* argmax_key, int64_t* token, int64_t* history, int64_t hist_len, int64_t* pos,
                          spectra_stream_t stream);

/* Measurement only (no counterpart in the reference): the fixed cost of one launch and
 * the time of a plain HBM stream, the floor and ceiling a one-launch GEMV is held against.
 * spectra_measure_empty: a kernel that does nothing, grid x block threads.
 * spectra_measure_read: reads `bytes` (a positive multiple of 16) at src (16-byte aligned)
 * with the GEMV's load pattern -- workgroup b reads the b-th contiguous slice, each thread
 * issues every 16-byte non-temporal load of its share before the first use -- and stores
 * nothing unless the XOR of all it read equals a fixed value (sink: block uint32 words,
 * 4-byte aligned).  block a multiple of 64 up to 1024; at most 16 loads per thread. */
int spectra_measure_empty(int32_t grid, int32_t block, spectra_stream_t stream);
int spectra_measure_read(const void* src, size_t bytes, int32_t grid, int32_t block, void* sink,
                         spectra_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* SPECTRA_HIP_H_ */
