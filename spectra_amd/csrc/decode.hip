// Fused kernels of a Llama-shaped layer between its quantized linears.  The reference
// fuses the same non-linear submodules (RMSNorm, SiLU, RoPE) with Inductor
// (engine.py:1240-1250) and keeps keys/values in a static cache for graph replay
// (engine.py:1387-1415).  Here each is one HIP kernel:
//
//   rmsnorm_kernel      h (+)= r (the add rounds to fp16), x = fp16(h * rsqrt(mean h^2 + eps) * w)
//   rope_append_kernel  rotates q and k of T tokens (pairs (i, i + d/2), fp32), writes the
//                       rotated q and appends k and v to the caches [kv][L][d] at the tokens'
//                       positions
//   attend_kernel       batch-1 decode attention on the fused-QKV row: rotates q and the new
//                       k, appends k and v to the caches, and attends over [0, pos] split
//                       into spans of 64 positions (one workgroup per KV head and span,
//                       fp32 softmax pieces); the last span workgroup of a KV head merges
//                       the spans (log-sum-exp) into fp16
//   silu_mul_kernel     act = fp16(silu(g) * u) on the fused gate_up output
//   greedy_kernel       greedy sampling: token = argmax(logits), appended to the history at
//                       pos + 1, pos advanced (the decode step's whole sampling tail)
//   greedy_finish_kernel the same tail for a pick gathered in a GEMV epilogue
//
// The position of the decoded token is read from device memory, so a decode step has no
// host-side value and is captured once as a HIP graph.
#include <cmath>

#include "common.h"

namespace spectra {

constexpr int kDecThreads = 256;
constexpr int kSpanMax = 64;  // positions per attention workgroup (one per lane of wave 0)


// One workgroup per row.  Rows of hidden % 8 == 0 (<= 8192) are read as 16-byte chunks, all
// issued before the first use (every chunk of the row is in flight at once); other rows take
// the element loop.
template <bool VEC>
__global__ void __launch_bounds__(kDecThreads) rmsnorm_kernel(uint16_t* __restrict__ h, const uint16_t* __restrict__ r,
                                                               const float* __restrict__ w, float eps, int hidden,
                                                               uint16_t* __restrict__ x) {
  __shared__ float red[kDecThreads / 64];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  uint16_t* hr = h + row * hidden;
  float ss = 0.0f;
  if constexpr (VEC) {
    constexpr int C = 4;  // chunks of 8 per thread: hidden <= 8192
    const int nch = hidden >> 3;
    uint4 hv[C], rv[C];
    float4 w0[C], w1[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int ch = tid + c * kDecThreads;
      if (ch < nch) {
        hv[c] = ((const uint4*)hr)[ch];
        if (r != nullptr) rv[c] = ((const uint4*)(r + row * hidden))[ch];
        w0[c] = ((const float4*)w)[2 * ch];
        w1[c] = ((const float4*)w)[2 * ch + 1];
      }
    }
    float v[C][8];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int ch = tid + c * kDecThreads;
      if (ch < nch) {
        const uint32_t hw[4] = {hv[c].x, hv[c].y, hv[c].z, hv[c].w};
        const uint32_t rw[4] = {rv[c].x, rv[c].y, rv[c].z, rv[c].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float t = h2f((uint16_t)(hw[e >> 1] >> (16 * (e & 1))));
          if (r != nullptr) t = h2f(f2h(t + h2f((uint16_t)(rw[e >> 1] >> (16 * (e & 1))))));
          v[c][e] = t;
          ss += t * t;
        }
        if (r != nullptr) {
          uint32_t o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = (uint32_t)f2h(v[c][2 * e]) | ((uint32_t)f2h(v[c][2 * e + 1]) << 16);
          ((uint4*)hr)[ch] = make_uint4(o[0], o[1], o[2], o[3]);
        }
      }
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float inv = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)hidden + eps);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int ch = tid + c * kDecThreads;
      if (ch < nch) {
        const float wv[8] = {w0[c].x, w0[c].y, w0[c].z, w0[c].w, w1[c].x, w1[c].y, w1[c].z, w1[c].w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = (uint32_t)f2h(v[c][2 * e] * inv * wv[2 * e]) | ((uint32_t)f2h(v[c][2 * e + 1] * inv * wv[2 * e + 1]) << 16);
        ((uint4*)(x + row * hidden))[ch] = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
  } else {
    for (int i = tid; i < hidden; i += kDecThreads) {
      float v = h2f(hr[i]);
      if (r != nullptr) {
        v = h2f(f2h(v + h2f(r[row * hidden + i])));
        hr[i] = f2h(v);
      }
      ss += v * v;
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float inv = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)hidden + eps);
    for (int i = tid; i < hidden; i += kDecThreads) x[row * hidden + i] = f2h(h2f(hr[i]) * inv * w[i]);
  }
}

// grid (heads + kv_heads, T), blockDim head_dim / 2.  Block b < heads rotates query head b;
// b >= heads rotates key head b - heads and appends it and the matching value head to the
// caches ([kv][L][d] both).
__global__ void rope_append_kernel(const uint16_t* __restrict__ qkv, int64_t ldqkv, const int64_t* __restrict__ pos_p,
                                   const float* __restrict__ cos_t, const float* __restrict__ sin_t, int heads,
                                   int kv_heads, int hd, int lmax, uint16_t* __restrict__ q_rot,
                                   uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache) {
  const int b = blockIdx.x, t = blockIdx.y, i = threadIdx.x, h2 = hd >> 1;
  const int64_t pos = pos_p[t];
  if (pos < 0 || pos >= lmax) return;  // outside the cache: nothing is written
  const float c = cos_t[pos * h2 + i], s = sin_t[pos * h2 + i];
  const uint16_t* row = qkv + t * ldqkv;
  const uint16_t* src = row + (int64_t)b * hd;  // q heads, then k heads, then v heads
  const float a = h2f(src[i]), bb = h2f(src[i + h2]);
  const uint16_t lo = f2h(a * c - bb * s), hi = f2h(bb * c + a * s);
  if (b < heads) {
    uint16_t* q = q_rot + ((int64_t)t * heads + b) * hd;
    q[i] = lo;
    q[i + h2] = hi;
  } else {
    const int kh = b - heads;
    uint16_t* kc = k_cache + ((int64_t)kh * lmax + pos) * hd;
    kc[i] = lo;
    kc[i + h2] = hi;
    const uint16_t* vs = row + (int64_t)(heads + kv_heads + kh) * hd;
    uint16_t* vc = v_cache + ((int64_t)kh * lmax + pos) * hd;
    vc[i] = vs[i];
    vc[i + h2] = vs[i + h2];
  }
}

// Sum over groups of W consecutive lanes (W a power of two <= 64): every lane of a group
// ends with the group's total.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  const int lane = __lane_id();
  if constexpr (W > 1) v += lane_xor<1>(v, lane);
  if constexpr (W > 2) v += lane_xor<2>(v, lane);
  if constexpr (W > 4) v += lane_xor<4>(v, lane);
  if constexpr (W > 8) v += lane_xor<8>(v, lane);
  if constexpr (W > 16) v += lane_xor<16>(v, lane);
  if constexpr (W > 32) v += lane_xor<32>(v, lane);
  return v;
}

// Sum over the lanes of a wave that are W, 2W, ... apart (W a power of two < 64): every
// lane ends with the total of its residue class mod W.
template <int W>
__device__ __forceinline__ float stride_sum(float v) {
  const int lane = __lane_id();
  if constexpr (W <= 1) v += lane_xor<1>(v, lane);
  if constexpr (W <= 2) v += lane_xor<2>(v, lane);
  if constexpr (W <= 4) v += lane_xor<4>(v, lane);
  if constexpr (W <= 8) v += lane_xor<8>(v, lane);
  if constexpr (W <= 16) v += lane_xor<16>(v, lane);
  return v + lane_xor<32>(v, lane);
}

__device__ __forceinline__ void unpack8(const uint4& u, float (&f)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = h2f((uint16_t)w[e]);
    f[2 * e + 1] = h2f((uint16_t)(w[e] >> 16));
  }
}

// KV cache of one layer.  fp16: k / v [kv][L][hd].  4-bit (Q4): every position quantized in
// kq / vq (two codes per byte, [kv][L][hd/2]), ks / vs (fp16 scales) and kz / vz (zero
// points) [kv][L][hd/32], and the last `window` positions also kept in fp16 in k / v, a ring
// [kv][window][hd] indexed by position % window.
struct KvCache {
  uint16_t* k;
  uint16_t* v;
  uint8_t* kq;
  uint8_t* vq;
  uint16_t* ks;
  uint16_t* vs;
  uint8_t* kz;
  uint8_t* vz;
  int lmax, window;
};

// The reference's 4-bit KV quantizer (engine.py:624-656) on fp16 values, for the 8 values
// of one lane; the 32-value group is 4 consecutive lanes.  Each torch op rounds where the
// reference's does: range and scale to fp16 (range / 15), zero point fp16(-min / scale)
// rounded half to even and clamped to [0, 15], codes round((t + z * s) / s) in fp32 clamped
// to [0, 15]; in fp16 the reference's 1e-8 threshold and scale floor are 0, so a constant
// group has scale 0 (its codes and zero point come from inf / NaN: NaN -> 0, +inf -> 15).
__device__ __forceinline__ void kv4_quant_chunk(const uint4& x, uint32_t& packed, uint16_t& sbits, uint8_t& zero) {
  float f[8];
  unpack8(x, f);
  float mn = f[0], mx = f[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) {
    mn = fminf(mn, f[e]);
    mx = fmaxf(mx, f[e]);
  }
  mn = fminf(mn, __shfl_xor(mn, 1, 64));
  mn = fminf(mn, __shfl_xor(mn, 2, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
  const float diff = h2f(f2h(mx - mn));
  const float sc = h2f(f2h(diff / 15.0f));
  const float zq = h2f(f2h(-mn / sc));
  const float zf = fminf(fmaxf(rintf(zq), 0.0f), 15.0f);  // NaN -> 0 (fmaxf returns the number)
  uint32_t pk = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float qv = fminf(fmaxf(rintf((f[e] + zf * sc) / sc), 0.0f), 15.0f);
    pk |= (uint32_t)qv << (4 * e);
  }
  packed = pk;
  sbits = f2h(sc);
  zero = (uint8_t)zf;
}

// (q - z) * s in fp32 rounded to bf16 (the reference's dequantized cache dtype), as fp32
__device__ __forceinline__ void kv4_dequant_chunk(uint32_t packed, uint32_t sz, float (&f)[8]) {
  const float s = h2f((uint16_t)sz), z = (float)(sz >> 16);
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = bf2f(f2bf(((float)((packed >> (4 * e)) & 15u) - z) * s));
}

// Rotation of the 8-dim chunk `own` of a head whose partner chunk (dims -+ head_dim/2) is
// `partner`, with the cos/sin of the chunk's pair indices: the lower half takes
// a*c - b*s, the upper half b*c + a*s (a = dim i, b = dim i + head_dim/2), each product and
// the sum rounded in fp32 as written, the result to fp16 -- the rope_append arithmetic.
__device__ __forceinline__ uint4 rope_chunk(const uint4& own, const uint4& partner, const float (&c)[8],
                                            const float (&s)[8], bool upper) {
  float x[8], y[8];
  unpack8(own, x);
  unpack8(partner, y);
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float r[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = 2 * e + h;
      r[h] = upper ? x[i] * c[i] + y[i] * s[i] : x[i] * c[i] - y[i] * s[i];
    }
    o[e] = (uint32_t)f2h(r[0]) | ((uint32_t)f2h(r[1]) << 16);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// Partials cross workgroups (and XCDs, whose L2 caches are not coherent with each other)
// as device-scope relaxed atomics: stores write through to the device's coherence point,
// loads read from it.
__device__ __forceinline__ void store_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Arrival of a span workgroup, and the merge by the last one of its KV head: every thread's
// partial stores have completed before the workgroup counts itself in (one device-scope
// atomic on the head's counter, 256 bytes apart per head); the workgroup that brings the
// count to nspan merges the G (<= 8) heads' spans exactly as a separate merge kernel would
// and leaves the counter at 0.  Spans are merged in batches of 16 (one batch up to 1024
// positions), every load of a batch in flight at once: lane (j, u) of the first 16 G
// threads (16-lane rows: j = tid / 16, u = tid % 16) loads (m, l) of head j, span u of the
// batch and, with 16-lane reductions, keeps the head's running maximum and sum of
// exponentials and turns the batch into weights exp(m - M) (m = -inf marks an empty span,
// weight 0) in LDS; every thread loads the V sums of its outputs (o, o + 256, ...) and folds
// them in with those weights.
template <int HD>
__device__ __forceinline__ void attend_arrive_merge(const float* part, uint32_t* counter, uint16_t* out, int kh,
                                                    int G, int nspan, int tid, int* last_l) {
  constexpr int B = 16, GM = 8, O = (GM * HD + kDecThreads - 1) / kDecThreads;
  __shared__ __align__(16) float fw[GM][B + 4];  // the batch's span weights per head, then the rescale
  __shared__ float hl_s[GM];
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0)
    *last_l = __hip_atomic_fetch_add(counter + kh * 64, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              (uint32_t)(nspan - 1);
  __syncthreads();
  if (!*last_l) return;
  if (tid == 0) __hip_atomic_store(counter + kh * 64, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int total = G * HD;
  const float* ph0 = part + (int64_t)kh * G * nspan * (HD + 2);  // head j, span s: + (j nspan + s)(HD + 2)
  const int lane = tid & 63;
  const int wj = tid / B, wu = tid % B;
  const bool wrow = wj < G;  // a weight lane (whole 16-lane rows)
  float hm = -INFINITY, hl = 0.0f;  // weight lanes: the head's running max and sum
  float a[O];
#pragma unroll
  for (int q = 0; q < O; ++q) a[q] = 0.0f;
  for (int s0 = 0; s0 < nspan; s0 += B) {
    float wmv = -INFINITY, wlv = 0.0f;
    if (wrow && s0 + wu < nspan) {
      const float* pp = ph0 + ((int64_t)wj * nspan + s0 + wu) * (HD + 2);
      wmv = load_dev(pp + HD);
      wlv = load_dev(pp + HD + 1);
    }
    float av[O][B];
#pragma unroll
    for (int q = 0; q < O; ++q) {
      const int o = tid + q * kDecThreads;
      const int oc = o < total ? o : 0;
      const int j = oc / HD, d = oc - j * HD;
      const float* pj = ph0 + (int64_t)j * nspan * (HD + 2) + d;
#pragma unroll
      for (int u = 0; u < B; ++u) av[q][u] = load_dev(pj + (int64_t)(s0 + u < nspan ? s0 + u : 0) * (HD + 2));
    }
    if (wrow) {
      float mb = wmv;
      mb = fmaxf(mb, lane_xor<1>(mb, lane));
      mb = fmaxf(mb, lane_xor<2>(mb, lane));
      mb = fmaxf(mb, lane_xor<4>(mb, lane));
      mb = fmaxf(mb, lane_xor<8>(mb, lane));
      mb = fmaxf(mb, hm);
      const float r = mb == -INFINITY ? 1.0f : __expf(hm - mb);  // rescale of what came before (0 if nothing)
      const float f = wmv == -INFINITY ? 0.0f : __expf(wmv - mb);  // empty span: weight 0
      float lb = wlv * f;
      lb += lane_xor<1>(lb, lane);
      lb += lane_xor<2>(lb, lane);
      lb += lane_xor<4>(lb, lane);
      lb += lane_xor<8>(lb, lane);
      hl = hl * r + lb;
      hm = mb;
      fw[wj][wu] = f;
      if (wu == 0) fw[wj][B] = r;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < O; ++q) {
      const int o = tid + q * kDecThreads;
      if (o < total) {
        const int j = o / HD;
        float t = a[q] * fw[j][B];
#pragma unroll
        for (int u = 0; u < B; ++u) {
          const float f = fw[j][u];
          t = f == 0.0f ? t : t + av[q][u] * f;  // an empty span's V sums were never written
        }
        a[q] = t;
      }
    }
    __syncthreads();  // (the weights are consumed before the next batch's)
  }
  if (wrow && wu == 0) hl_s[wj] = hl;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < O; ++q) {
    const int o = tid + q * kDecThreads;
    if (o < total) out[(int64_t)kh * G * HD + o] = f2h(a[q] / hl_s[o / HD]);
  }
}

// grid (kv_heads, nspan), 256 threads.  Span sp covers positions [64 sp, 64 sp + 64) of
// [0, pos]; spans past the position only mark themselves empty.  Each workgroup:
//   * rotates the query heads of its group from the fused-QKV row (ROPE) -- every
//     workgroup of the group computes the same values -- and, when its span holds pos,
//     rotates the new key, appends key and value to the caches and uses them from registers;
//   * thread = (dg: 8 consecutive head dims, pr: position row), pass i = positions
//     pr + i * PPW; every K and V chunk of the span is loaded up front (16 bytes each);
//   * writes its span's max score, sum of exponentials and exponential-weighted V sums
//     to part [heads][nspan][hd + 2] (fp32, device-coherent stores); the last span
//     workgroup of the KV head merges them into out (attend_arrive_merge).
template <int G, int HD, bool ROPE, bool Q4>
__global__ void __launch_bounds__(kDecThreads) attend_kernel(const uint16_t* __restrict__ qkv,
                                                              const int64_t* __restrict__ pos_p,
                                                              const float* __restrict__ cos_t,
                                                              const float* __restrict__ sin_t, int heads,
                                                              int kv_heads, float scale, const KvCache kvc,
                                                              float* __restrict__ part,
                                                              uint32_t* __restrict__ counter,
                                                              uint16_t* __restrict__ out) {
  const int lmax = kvc.lmax;
  constexpr int DG = HD / 8;               // lanes per position
  // positions per pass: at HD 16 the workgroup has more position rows than the span has
  // positions, and the threads of rows >= kSpanMax only take part in the reductions (zeros)
  constexpr int PPW = kDecThreads / DG < kSpanMax ? kDecThreads / DG : kSpanMax;
  constexpr int NP = kSpanMax / PPW;       // passes
  constexpr int H2 = HD / 2;
  static_assert(HD % 16 == 0 && (!Q4 || HD % 32 == 0), "head_dim: a multiple of 16 (of 32 for the 4-bit cache)");
  __shared__ float sc[G][kSpanMax];        // scores, then exponentials
  __shared__ float wsum[4][G][HD];         // V sums of the four waves
  const int kh = blockIdx.x, sp = blockIdx.y, nspan = gridDim.y, tid = threadIdx.x;
  const int t0 = sp * kSpanMax;
  const int dg = tid % DG, pr = tid / DG;
  const bool act = pr < PPW;  // a position row of the span
  // fp16 cache: the span's K / V rows first, at addresses independent of the position (rows
  // clamped into the cache; those past the position are masked below), so they are in
  // flight while the position arrives (a scalar load)
  uint4 kr[NP], vr[NP];
  if constexpr (!Q4) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int64_t t = min(t0 + pr + i * PPW, lmax - 1);
      kr[i] = *(const uint4*)(kvc.k + ((int64_t)kh * lmax + t) * HD + dg * 8);
      vr[i] = *(const uint4*)(kvc.v + ((int64_t)kh * lmax + t) * HD + dg * 8);
    }
  }
  const int64_t pos = *pos_p;
  // a position outside the cache: every span reports itself empty, so nothing is appended
  // and the merge's 0 / 0 gives NaN outputs (rope_append likewise writes nothing)
  const bool outside = pos < 0 || pos >= lmax;
  const int n = outside ? 0 : (int)min((int64_t)kSpanMax, pos + 1 - t0);  // uniform
  float* pbase = part + ((int64_t)kh * G * nspan + sp) * (HD + 2);  // head j: + j * nspan * (HD + 2)
  __shared__ int last_l;
  if (n <= 0) {  // span past the position: an empty piece for the merge
    if (tid < G) {
      store_dev(pbase + (int64_t)tid * nspan * (HD + 2) + HD, -INFINITY);
      store_dev(pbase + (int64_t)tid * nspan * (HD + 2) + HD + 1, 0.0f);
    }
    attend_arrive_merge<HD>(part, counter, out, kh, G, nspan, tid, &last_l);  // (waits for the span's loads)
    return;
  }
  const bool upper = dg * 8 >= H2;
  const int pdg = upper ? dg - H2 / 8 : dg + H2 / 8;  // partner chunk
  const int tnew = (int)(pos - t0);                   // < 64 when this span holds pos
  const bool mine = tnew < kSpanMax;
  const int64_t ldh = (int64_t)HD;
  // ---- loads: the group's query chunks, the new key / value, cos / sin, the span's cache
  const uint16_t* qrow = qkv + (int64_t)kh * G * ldh;
  const uint16_t* krow = qkv + (int64_t)(heads + kh) * ldh;
  const uint16_t* vrow = qkv + (int64_t)(heads + kv_heads + kh) * ldh;
  uint4 qo[G], qp[G], ko = make_uint4(0, 0, 0, 0), kp = ko, vo = ko;
#pragma unroll
  for (int j = 0; j < G; ++j) {
    qo[j] = *(const uint4*)(qrow + j * ldh + dg * 8);
    if (ROPE) qp[j] = *(const uint4*)(qrow + j * ldh + pdg * 8);
  }
  if (mine) {
    ko = *(const uint4*)(krow + dg * 8);
    if (ROPE) kp = *(const uint4*)(krow + pdg * 8);
    vo = *(const uint4*)(vrow + dg * 8);
  }
  float cs[8], sn[8];
  if (ROPE) {
    const int i0 = (upper ? dg * 8 - H2 : dg * 8);
    const float4* cp = (const float4*)(cos_t + pos * H2 + i0);
    const float4* spp = (const float4*)(sin_t + pos * H2 + i0);
    const float4 c0 = cp[0], c1 = cp[1], s0 = spp[0], s1 = spp[1];
    cs[0] = c0.x; cs[1] = c0.y; cs[2] = c0.z; cs[3] = c0.w; cs[4] = c1.x; cs[5] = c1.y; cs[6] = c1.z; cs[7] = c1.w;
    sn[0] = s0.x; sn[1] = s0.y; sn[2] = s0.z; sn[3] = s0.w; sn[4] = s1.x; sn[5] = s1.y; sn[6] = s1.z; sn[7] = s1.w;
  }
  // fp16 rows of position t: the cache itself, or (Q4) the window ring
  const int W = Q4 ? kvc.window : lmax;
  auto row16 = [&](const uint16_t* base, int64_t t) __attribute__((always_inline)) {
    return base + ((int64_t)kh * W + (Q4 ? t % W : t)) * HD + dg * 8;
  };
  uint32_t inwin = 0;  // Q4: bit i = pass i's position is in the fp16 window
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int tl = pr + i * PPW;
    if constexpr (!Q4) {
      // rows past the position hold whatever the cache held: their scores are masked, and
      // their values are zeroed so that a zero weight cannot meet a NaN
      if (tl >= n) vr[i] = make_uint4(0, 0, 0, 0);
      continue;
    }
    const int64_t t = t0 + (tl < n ? tl : 0);  // past the end: re-read the first (in bounds)
    if (t > pos - W) {
      inwin |= 1u << i;
      kr[i] = *(const uint4*)row16(kvc.k, t);
      vr[i] = *(const uint4*)row16(kvc.v, t);
    } else {
      const int64_t r = (int64_t)kh * lmax + t;
      const int64_t sg = r * (HD / 32) + dg / 4;
      kr[i] = make_uint4(*(const uint32_t*)(kvc.kq + r * (HD / 2) + dg * 4),
                         (uint32_t)kvc.ks[sg] | ((uint32_t)kvc.kz[sg] << 16), 0, 0);
      vr[i] = make_uint4(*(const uint32_t*)(kvc.vq + r * (HD / 2) + dg * 4),
                         (uint32_t)kvc.vs[sg] | ((uint32_t)kvc.vz[sg] << 16), 0, 0);
    }
  }
  // ---- the new token: rotate, append, and take it from registers
  if (mine) {
    const uint4 knew = ROPE ? rope_chunk(ko, kp, cs, sn, upper) : ko;
    if constexpr (Q4) {  // every position is quantized as it is appended (all lanes: the group's lanes meet)
      uint32_t kpk, vpk;
      uint16_t ksb, vsb;
      uint8_t kzb, vzb;
      kv4_quant_chunk(knew, kpk, ksb, kzb);
      kv4_quant_chunk(vo, vpk, vsb, vzb);
      if (pr == tnew % PPW) {
        const int64_t r = (int64_t)kh * lmax + pos;
        *(uint32_t*)(kvc.kq + r * (HD / 2) + dg * 4) = kpk;
        *(uint32_t*)(kvc.vq + r * (HD / 2) + dg * 4) = vpk;
        if ((dg & 3) == 0) {
          const int64_t sg = r * (HD / 32) + dg / 4;
          kvc.ks[sg] = ksb;
          kvc.vs[sg] = vsb;
          kvc.kz[sg] = kzb;
          kvc.vz[sg] = vzb;
        }
      }
    }
    if (pr == tnew % PPW) {
      *(uint4*)row16(kvc.k, pos) = knew;
      *(uint4*)row16(kvc.v, pos) = vo;
    }
#pragma unroll
    for (int i = 0; i < NP; ++i)
      if (pr + i * PPW == tnew) {
        kr[i] = knew;
        vr[i] = vo;
        if (Q4) inwin |= 1u << i;
      }
  }
  // ---- scores
  float qf[G][8];
#pragma unroll
  for (int j = 0; j < G; ++j) unpack8(ROPE ? rope_chunk(qo[j], qp[j], cs, sn, upper) : qo[j], qf[j]);
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    float kf[8];
    if (!Q4 || ((inwin >> i) & 1)) unpack8(kr[i], kf);
    else kv4_dequant_chunk(kr[i].x, kr[i].y, kf);
#pragma unroll
    for (int j = 0; j < G; ++j) {
      float d = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) d += qf[j][e] * kf[e];
      d = group_sum<DG>(d);
      if (dg == 0 && act) sc[j][pr + i * PPW] = d * scale;
    }
  }
  __syncthreads();
  if (tid < 64) {  // wave 0: lane = position of the span
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const float s = tid < n ? sc[j][tid] : -INFINITY;
      const float m = wave_max(s);  // finite: n >= 1
      const float e = tid < n ? __expf(s - m) : 0.0f;
      sc[j][tid] = e;
      const float l = wave_sum(e);
      if (tid == 0) {
        store_dev(pbase + (int64_t)j * nspan * (HD + 2) + HD, m);
        store_dev(pbase + (int64_t)j * nspan * (HD + 2) + HD + 1, l);
      }
    }
  }
  __syncthreads();
  // ---- exponential-weighted V sums: G x 8 partials per thread, then across the position
  // rows of the wave (lanes DG apart) and across the four waves
  float acc[G][8];
#pragma unroll
  for (int j = 0; j < G; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0.0f;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    float vf[8];
    if (!Q4 || ((inwin >> i) & 1)) unpack8(vr[i], vf);
    else kv4_dequant_chunk(vr[i].x, vr[i].y, vf);
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const float pw = act ? sc[j][pr + i * PPW] : 0.0f;  // 0 past the end
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[j][e] += pw * vf[e];
    }
  }
  const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
  for (int j = 0; j < G; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = stride_sum<DG>(acc[j][e]);
  if (lane < DG) {
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) wsum[wave][j][lane * 8 + e] = acc[j][e];
  }
  __syncthreads();
  for (int o = tid; o < G * HD; o += kDecThreads) {
    const int j = o / HD, d = o - j * HD;
    store_dev(pbase + (int64_t)j * nspan * (HD + 2) + d,
              (wsum[0][j][d] + wsum[1][j][d]) + (wsum[2][j][d] + wsum[3][j][d]));
  }
  attend_arrive_merge<HD>(part, counter, out, kh, G, nspan, tid, &last_l);
}

// MFMA decode attention on the fp16 cache (head_dim 64, 128 or 256, at most 8 query heads
// per KV head).  Same grid, spans, partials and merge as attend_kernel; inside a span
// workgroup wave w takes positions t0 + 16 w .. + 15 and lane (i, g) = (lane & 15, lane >> 4):
//   * holds the 16-byte chunks 32 c + 8 g .. + 7 (c < head_dim / 32) of position t0 + 16 w + i
//     for K and V, and of query head i for q (zero for i >= G): the A and B operands of
//     v_mfma_f32_16x16x32_f16, so scores = K q^T is head_dim / 32 MFMAs;
//   * ends the score MFMAs with the scores of positions 4 g + r (r < 4) for head i -- exactly
//     the A operand of v_mfma_f32_16x16x16_f16 for P V, so the wave's softmax piece (max and
//     sum per head over its 16 positions) feeds P V without moving;
//   * reads the V operand (4 positions x 1 dim) from the wave's V tile, staged in LDS.
// The rotated query heads and new key are computed once per workgroup (one thread per 8
// rotation pairs of a row) into LDS.  The four waves' pieces are combined (log-sum-exp)
// through LDS into the span's partials.  Rows past the position are masked: scores by
// select, V rows zeroed before they reach the MFMA (a cache row past the position may hold
// anything, NaN included).
typedef _Float16 ah8_t __attribute__((ext_vector_type(8)));
typedef _Float16 ah4_t __attribute__((ext_vector_type(4)));
typedef float af4_t __attribute__((ext_vector_type(4)));
constexpr int kMfmaMaxGroup = 8;  // query heads per KV head served by attend_mfma_kernel

template <int HD, bool ROPE>
__global__ void __launch_bounds__(kDecThreads) attend_mfma_kernel(const uint16_t* __restrict__ qkv,
                                                                   const int64_t* __restrict__ pos_p,
                                                                   const float* __restrict__ cos_t,
                                                                   const float* __restrict__ sin_t, int heads,
                                                                   int kv_heads, float scale, const KvCache kvc,
                                                                   float* __restrict__ part,
                                                                   uint32_t* __restrict__ counter,
                                                                   uint16_t* __restrict__ out) {
  constexpr int KI = HD / 32;  // 32-dim blocks (score MFMAs; 16-byte chunks per lane and row)
  constexpr int DB = HD / 16;  // 16-dim blocks (P V MFMAs)
  constexpr int VS = HD + 8;   // LDS row stride (halves) of the V tiles and the rotated rows
  constexpr int GM = kMfmaMaxGroup;
  constexpr int RB = HD / 16;  // rotation work items per row (8 pairs (d, d + HD / 2) each)
  static_assert(HD == 64 || HD == 128 || HD == 256, "head_dim 64, 128 or 256");
  // the V tiles [wave][16][VS] (fp16), then, once every wave is past its P V, the per-wave
  // V sums [wave][GM][HD] (fp32) in the same bytes
  __shared__ __align__(16) uint8_t lds[4 * 16 * VS * 2];
  static_assert(4 * GM * HD * 4 <= 4 * 16 * VS * 2, "per-wave V sums fit the V tiles");
  __shared__ __align__(16) uint16_t qs[GM + 1][VS];  // rotated query heads, then the new key
  __shared__ float wm[4][16], wl[4][16];              // per-wave max and sum of exponentials
  __shared__ int last_l;
  // every kernel argument in one round trip, before the first load
  asm volatile("" ::"s"(qkv), "s"(pos_p), "s"(cos_t), "s"(sin_t), "s"(heads), "s"(kv_heads), "s"(scale),
               "s"(kvc.k), "s"(kvc.v), "s"(kvc.lmax), "s"(part), "s"(counter), "s"(out));
  const int G = heads / kv_heads;
  const int lmax = kvc.lmax;
  const int kh = blockIdx.x, sp = blockIdx.y, nspan = gridDim.y, tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, i16 = lane & 15, g4 = lane >> 4;
  const int t0 = sp * kSpanMax;
  const int tp = t0 + 16 * wave + i16;  // the position of this lane's K / V chunks
  // rotation item of this lane: row i (< G: query head, G: the new key), pair block
  // b = RBW w + g (pairs (d, d + HD / 2), d = 8 b .. + 7); its query / key halves load first,
  // so that waiting for them waits for no K / V chunk
  constexpr int RBW = RB / 4;  // pair blocks per wave
  const bool ritem = g4 < RBW && i16 <= G;
  const int rblk = RBW * wave + g4;
  uint4 rlo = make_uint4(0, 0, 0, 0), rhi = rlo;
  if (ritem) {
    const uint32_t o = (uint32_t)((i16 < G ? kh * G + i16 : heads + kh) * HD) * 2u + 16u * rblk;
    rlo = load_at<uint4>(qkv, o);
    rhi = load_at<uint4>(qkv, o + (uint32_t)HD);
  }
  // ---- K / V chunks at addresses independent of the position (rows clamped into the cache)
  const uint16_t* kbase = kvc.k + (int64_t)kh * lmax * HD;
  const uint16_t* vbase = kvc.v + (int64_t)kh * lmax * HD;
  uint4 kr[KI], vr[KI];
  {
    const uint32_t o = (uint32_t)(min(tp, lmax - 1) * HD + 8 * g4) * 2u;
#pragma unroll
    for (int c = 0; c < KI; ++c) {
      kr[c] = load_at<uint4>(kbase, o + 64u * c);
      vr[c] = load_at<uint4>(vbase, o + 64u * c);
    }
  }
  asm volatile("" ::: "memory");  // the K / V chunks are requested here, not sunk behind the position
  // the position: a scalar load (it waits for no vector load)
  const int64_t pos = *(const __attribute__((address_space(4))) int64_t*)pos_p;
  const bool outside = pos < 0 || pos >= lmax;
  const int n = outside ? 0 : (int)min((int64_t)kSpanMax, pos + 1 - t0);  // uniform
  float* pbase = part + ((int64_t)kh * G * nspan + sp) * (HD + 2);     // head j: + j * nspan * (HD + 2)
  if (n <= 0) {  // span past the position: an empty piece for the merge
    if (tid < G) {
      store_dev(pbase + (int64_t)tid * nspan * (HD + 2) + HD, -INFINITY);
      store_dev(pbase + (int64_t)tid * nspan * (HD + 2) + HD + 1, 0.0f);
    }
    attend_arrive_merge<HD>(part, counter, out, kh, G, nspan, tid, &last_l);
    return;
  }
  // ---- rotation: the cos / sin of the position for the wave's pair blocks (scalar loads:
  //      they wait for no vector load), the rope_append arithmetic, into LDS
  if constexpr (ROPE) {
    typedef const __attribute__((address_space(4))) float* cfp_t;
    const cfp_t ct = (cfp_t)(cos_t + pos * (HD / 2) + 8 * RBW * wave);
    const cfp_t st = (cfp_t)(sin_t + pos * (HD / 2) + 8 * RBW * wave);
    float cw[8 * RBW], sw[8 * RBW];
#pragma unroll
    for (int e = 0; e < 8 * RBW; ++e) {
      cw[e] = ct[e];
      sw[e] = st[e];
    }
    if (ritem) {
      float cs[8], sn[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float cv = cw[e], sv = sw[e];
#pragma unroll
        for (int b = 1; b < RBW; ++b) {
          cv = g4 == b ? cw[8 * b + e] : cv;
          sv = g4 == b ? sw[8 * b + e] : sv;
        }
        cs[e] = cv;
        sn[e] = sv;
      }
      const uint4 lo = rope_chunk(rlo, rhi, cs, sn, false), hi = rope_chunk(rhi, rlo, cs, sn, true);
      rlo = lo;
      rhi = hi;
    }
  }
  if (ritem) {
    *(uint4*)&qs[i16][8 * rblk] = rlo;
    *(uint4*)&qs[i16][HD / 2 + 8 * rblk] = rhi;
  }
  const bool mine = tp == pos;  // the lanes of the new token's row
  uint4 vn[KI];
  if (mine) {
    const uint16_t* vrow = qkv + (int64_t)(heads + kv_heads + kh) * HD;
#pragma unroll
    for (int c = 0; c < KI; ++c) vn[c] = load_at<uint4>(vrow, 16u * (4 * c + g4));
  }
  __syncthreads();
  // ---- the new token: appended to the caches, and taken from registers
  if (mine) {
    const uint32_t o = (uint32_t)(pos * HD + 8 * g4) * 2u;
#pragma unroll
    for (int c = 0; c < KI; ++c) {
      kr[c] = *(const uint4*)&qs[G][32 * c + 8 * g4];
      vr[c] = vn[c];
      *(uint4*)((uint8_t*)kvc.k + (int64_t)kh * lmax * HD * 2 + o + 64u * c) = kr[c];
      *(uint4*)((uint8_t*)kvc.v + (int64_t)kh * lmax * HD * 2 + o + 64u * c) = vr[c];
    }
  }
  // ---- this wave's V tile, rows past the position zeroed
  uint16_t* vt = (uint16_t*)lds + wave * 16 * VS;
  {
    const bool vok = tp - t0 < n;
#pragma unroll
    for (int c = 0; c < KI; ++c)
      *(uint4*)(vt + i16 * VS + 32 * c + 8 * g4) = vok ? vr[c] : make_uint4(0, 0, 0, 0);
  }
  // ---- scores: D[position 4 g + r][head i]
  af4_t sc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < KI; ++c) {
    const uint4 qc = i16 < G ? *(const uint4*)&qs[i16][32 * c + 8 * g4] : make_uint4(0, 0, 0, 0);
    sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(ah8_t, kr[c]), __builtin_bit_cast(ah8_t, qc), sc,
                                                0, 0, 0);
  }
  // ---- the wave's softmax piece for head i over its 16 positions
  const int pb = 16 * wave + 4 * g4;  // span-relative position of row r = pb + r
  float e[4];
  float mx = -INFINITY;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    e[r] = pb + r < n ? sc[r] * scale : -INFINITY;
    mx = fmaxf(mx, e[r]);
  }
  mx = fmaxf(mx, lane_xor<16>(mx, lane));
  mx = fmaxf(mx, lane_xor<32>(mx, lane));
  float l = 0.0f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    e[r] = pb + r < n ? __expf(e[r] - mx) : 0.0f;  // (no valid row: mx = -inf, every e 0)
    l += e[r];
  }
  l += lane_xor<16>(l, lane);
  l += lane_xor<32>(l, lane);
  // ---- P V: D[head 4 g + r][dim 16 b + i]
  const ah4_t pa = {(_Float16)e[0], (_Float16)e[1], (_Float16)e[2], (_Float16)e[3]};
  af4_t acc[DB];
  const uint16_t* vrd = vt + (4 * g4) * VS + i16;
#pragma unroll
  for (int b = 0; b < DB; ++b) {
    const ah4_t vb = {__builtin_bit_cast(_Float16, vrd[16 * b]), __builtin_bit_cast(_Float16, vrd[VS + 16 * b]),
                      __builtin_bit_cast(_Float16, vrd[2 * VS + 16 * b]),
                      __builtin_bit_cast(_Float16, vrd[3 * VS + 16 * b])};
    acc[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, vb, af4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
  }
  // ---- the four waves' pieces -> the span's partials: each wave's V sums (unscaled) and
  //      softmax piece to LDS, then per output the log-sum-exp combination in wave order
  if (g4 == 0) {
    wm[wave][i16] = mx;
    wl[wave][i16] = l;
  }
  __syncthreads();  // (every wave is also past its V tile)
  float* ws = (float*)lds;  // [wave][GM][HD]
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int h = 4 * g4 + r;
    if (h < G) {
#pragma unroll
      for (int b = 0; b < DB; ++b) ws[(wave * GM + h) * HD + 16 * b + i16] = acc[b][r];
    }
  }
  __syncthreads();
  for (int o = tid; o < G * HD; o += kDecThreads) {
    const int j = o / HD, d = o - j * HD;
    const float m4 = fmaxf(fmaxf(wm[0][j], wm[1][j]), fmaxf(wm[2][j], wm[3][j]));
    float a = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) a += wm[w][j] == -INFINITY ? 0.0f : ws[(w * GM + j) * HD + d] * __expf(wm[w][j] - m4);
    store_dev(pbase + (int64_t)j * nspan * (HD + 2) + d, a);
  }
  if (tid < G) {
    const int j = tid;
    const float m4 = fmaxf(fmaxf(wm[0][j], wm[1][j]), fmaxf(wm[2][j], wm[3][j]));
    float lt = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) lt += wm[w][j] == -INFINITY ? 0.0f : wl[w][j] * __expf(wm[w][j] - m4);
    store_dev(pbase + (int64_t)j * nspan * (HD + 2) + HD, m4);
    store_dev(pbase + (int64_t)j * nspan * (HD + 2) + HD + 1, lt);
  }
  attend_arrive_merge<HD>(part, counter, out, kh, G, nspan, tid, &last_l);
}

// grid (ceil(rows * d / 8 / 256), heads): one lane per 8 values (groups of 32 = 4 lanes)
__global__ void __launch_bounds__(kDecThreads) kv4_quantize_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                    int64_t xhs, int64_t rows, int d,
                                                                    int64_t out_rows, uint8_t* __restrict__ packed,
                                                                    uint16_t* __restrict__ scales,
                                                                    uint8_t* __restrict__ zeros) {
  const int64_t gid = (int64_t)blockIdx.x * kDecThreads + threadIdx.x;
  const int cpr = d >> 3;  // chunks per row (a multiple of 4: groups never straddle lanes of two rows)
  const int64_t r = gid / cpr;
  const int c = (int)(gid - r * cpr);
  if (r >= rows) return;  // whole groups of 4 lanes leave together
  const int h = blockIdx.y;
  const uint4 v = *(const uint4*)(x + h * xhs + r * ldx + c * 8);
  uint32_t pk;
  uint16_t sb;
  uint8_t zb;
  kv4_quant_chunk(v, pk, sb, zb);
  const int64_t orow = (int64_t)h * out_rows + r;
  *(uint32_t*)(packed + orow * (d / 2) + c * 4) = pk;
  if ((c & 3) == 0) {
    scales[orow * (d / 32) + c / 4] = sb;
    zeros[orow * (d / 32) + c / 4] = zb;
  }
}

// the reference's dequantized values: bf16 [rows, d]
__global__ void __launch_bounds__(kDecThreads) kv4_dequantize_kernel(const uint8_t* __restrict__ packed,
                                                                      const uint16_t* __restrict__ scales,
                                                                      const uint8_t* __restrict__ zeros, int64_t rows,
                                                                      int d, uint16_t* __restrict__ out) {
  const int64_t gid = (int64_t)blockIdx.x * kDecThreads + threadIdx.x;
  const int cpr = d >> 3;
  const int64_t r = gid / cpr;
  const int c = (int)(gid - r * cpr);
  if (r >= rows) return;
  const int64_t sg = r * (d / 32) + c / 4;
  float f[8];
  kv4_dequant_chunk(*(const uint32_t*)(packed + r * (d / 2) + c * 4), (uint32_t)scales[sg] | ((uint32_t)zeros[sg] << 16), f);
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = (uint32_t)f2bf(f[2 * e]) | ((uint32_t)f2bf(f[2 * e + 1]) << 16);
  *(uint4*)(out + r * d + c * 8) = make_uint4(o[0], o[1], o[2], o[3]);
}

__global__ void __launch_bounds__(kDecThreads) silu_mul_kernel(const uint16_t* __restrict__ gu, int64_t ldgu,
                                                                int inter, int64_t total,
                                                                uint16_t* __restrict__ act) {
  const int64_t i = (int64_t)blockIdx.x * kDecThreads + threadIdx.x;
  if (i >= total) return;
  const int64_t r = i / inter, c = i - r * inter;
  const float g = h2f(gu[r * ldgu + c]), u = h2f(gu[r * ldgu + inter + c]);
  act[i] = f2h(g / (1.0f + __expf(-g)) * u);
}

// One workgroup of 1024 threads: token = index of the largest logit (lowest index among
// equal maxima, NaN counts as largest, as torch.argmax); history[pos + 1] = token; pos += 1.
constexpr int kArgThreads = 1024;
__device__ __forceinline__ bool arg_better(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na || nb) return na && (!nb || ia < ib);
  return a > b || (a == b && ia < ib);
}
__global__ void __launch_bounds__(kArgThreads) greedy_kernel(const uint16_t* __restrict__ logits, int n,
                                                              int64_t* __restrict__ token,
                                                              int64_t* __restrict__ history, int64_t hist_len,
                                                              int64_t* __restrict__ pos) {
  __shared__ float bv[kArgThreads / 64];
  __shared__ int bi[kArgThreads / 64];
  const int tid = threadIdx.x;
  // A thread visits its indices in increasing order, so inside the thread "better" is a
  // strict > (the first of equal maxima stays) or a first NaN; the scan starts from the
  // thread's first element.  Across threads arg_better applies the full rule.
  float best = -INFINITY;
  int besti = 0x7fffffff;
  bool first = true;
  auto visit = [&](float f, int i) __attribute__((always_inline)) {
    const bool take = first || f > best || (f != f && best == best);
    best = take ? f : best;
    besti = take ? i : besti;
    first = false;
  };
  constexpr int Q = 16;  // chunks of 8 in flight per thread: 131072 logits per round trip
  const int nch = n >> 3;
  for (int c0 = 0; c0 < nch; c0 += Q * kArgThreads) {
    uint4 u[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int ch = c0 + tid + q * kArgThreads;
      u[q] = ((const uint4*)logits)[ch < nch ? ch : 0];
    }
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int ch = c0 + tid + q * kArgThreads;
      if (ch < nch) {
        float f[8];
        unpack8(u[q], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) visit(f[e], 8 * ch + e);
      }
    }
  }
  for (int i = (nch << 3) + tid; i < n; i += kArgThreads) visit(h2f(logits[i]), i);  // tail
  // across the wave: DPP / permlane butterflies (partners 32, 16, ..., 1), value and index
  // moved as bits
  const int lane = tid & 63;
  auto take = [&](float ov, float oib) __attribute__((always_inline)) {
    const int oi = __builtin_bit_cast(int, oib);
    if (arg_better(ov, oi, best, besti)) {
      best = ov;
      besti = oi;
    }
  };
  take(lane_xor<32>(best, lane), lane_xor<32>(__builtin_bit_cast(float, besti), lane));
  take(lane_xor<16>(best, lane), lane_xor<16>(__builtin_bit_cast(float, besti), lane));
  take(lane_xor<8>(best, lane), lane_xor<8>(__builtin_bit_cast(float, besti), lane));
  take(lane_xor<4>(best, lane), lane_xor<4>(__builtin_bit_cast(float, besti), lane));
  take(lane_xor<2>(best, lane), lane_xor<2>(__builtin_bit_cast(float, besti), lane));
  take(lane_xor<1>(best, lane), lane_xor<1>(__builtin_bit_cast(float, besti), lane));
  if ((tid & 63) == 0) {
    bv[tid >> 6] = best;
    bi[tid >> 6] = besti;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgThreads / 64; ++w)
      if (arg_better(bv[w], bi[w], best, besti)) {
        best = bv[w];
        besti = bi[w];
      }
    *token = besti;
    if (pos != nullptr) {
      const int64_t p = *pos + 1;
      if (history != nullptr && p >= 0 && p < hist_len) history[p] = besti;
      *pos = p;
    }
  }
}

// The token of a fused greedy pick: the largest of the SPECTRA_ARGMAX_SLOTS keys (value
// order in the high word, complemented index in the low word), then the history / position
// update of greedy_kernel; the slots are left at 0 for the next pick.
__global__ void __launch_bounds__(64) greedy_finish_kernel(unsigned long long* __restrict__ key,
                                                           int64_t* __restrict__ token, int64_t* __restrict__ history,
                                                           int64_t hist_len, int64_t* __restrict__ pos) {
  const int lane = threadIdx.x;
  constexpr int PER = SPECTRA_ARGMAX_SLOTS / 64;
  unsigned long long k = 0ull;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const unsigned long long t = key[(lane + 64 * i) * SPECTRA_ARGMAX_STRIDE];
    k = t > k ? t : k;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const unsigned long long t = __shfl_xor(k, o);
    k = t > k ? t : k;
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) key[(lane + 64 * i) * SPECTRA_ARGMAX_STRIDE] = 0ull;
  if (lane == 0) {
    const int64_t tok = (int64_t)(0xffffffffu - (uint32_t)(k & 0xffffffffull));
    *token = tok;
    if (pos != nullptr) {
      const int64_t p = *pos + 1;
      if (history != nullptr && p >= 0 && p < hist_len) history[p] = tok;
      *pos = p;
    }
  }
}

}  // namespace spectra

using namespace spectra;

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

extern "C" int spectra_rmsnorm(void* h, const void* residual, const float* weight, float eps, int64_t rows,
                               int64_t hidden, void* x, spectra_stream_t stream) {
  SPECTRA_REQUIRE(h && weight && x, "NULL pointer");
  SPECTRA_REQUIRE(rows >= 1 && rows < (int64_t(1) << 31) && hidden >= 1 && hidden < (1 << 24), "bad shape");
  const bool vec = hidden % 8 == 0 && hidden <= 8 * 4 * kDecThreads && aligned16(h) && aligned16(x) &&
                   aligned16(weight) && (residual == nullptr || aligned16(residual));
  auto kern = vec ? rmsnorm_kernel<true> : rmsnorm_kernel<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)rows), dim3(kDecThreads), 0, (hipStream_t)stream, (uint16_t*)h,
                     (const uint16_t*)residual, weight, eps, (int)hidden, (uint16_t*)x);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

extern "C" int spectra_rope_append(const void* qkv, int64_t ldqkv, int64_t tokens, const int64_t* pos,
                                   const float* cos_t, const float* sin_t, int32_t heads, int32_t kv_heads,
                                   int32_t head_dim, int32_t max_seq, void* q_rot, void* k_cache, void* v_cache,
                                   spectra_stream_t stream) {
  SPECTRA_REQUIRE(qkv && pos && cos_t && sin_t && q_rot && k_cache && v_cache, "NULL pointer");
  SPECTRA_REQUIRE(heads >= 1 && kv_heads >= 1 && heads % kv_heads == 0, "heads must be a multiple of kv_heads");
  SPECTRA_REQUIRE(head_dim >= 2 && head_dim <= 2048 && head_dim % 2 == 0, "head_dim must be even, <= 2048");
  SPECTRA_REQUIRE(tokens >= 1 && tokens <= 65535 && max_seq >= 1, "bad token count");
  SPECTRA_REQUIRE(ldqkv >= (int64_t)(heads + 2 * kv_heads) * head_dim, "qkv row stride too small");
  hipLaunchKernelGGL(rope_append_kernel, dim3((unsigned)(heads + kv_heads), (unsigned)tokens),
                     dim3((unsigned)(head_dim / 2)), 0, (hipStream_t)stream, (const uint16_t*)qkv, ldqkv, pos, cos_t,
                     sin_t, heads, kv_heads, head_dim, max_seq, (uint16_t*)q_rot, (uint16_t*)k_cache,
                     (uint16_t*)v_cache);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

extern "C" int32_t spectra_attend_spans(int32_t max_seq) { return (max_seq + kSpanMax - 1) / kSpanMax; }

// Workspace: one arrival counter per KV head, 256 bytes apart, at the start (the same
// offset for every shape, so counters left at zero by one call stay zero for a call of
// another shape on the same workspace), then [heads][nspan][head_dim + 2] fp32 partials.
static size_t attend_counter_bytes(int32_t heads) { return (size_t)heads * 256; }
static size_t attend_part_bytes(int32_t heads, int32_t head_dim, int32_t max_seq) {
  const size_t b = (size_t)heads * spectra_attend_spans(max_seq) * (head_dim + 2) * sizeof(float);
  return (b + 255) & ~(size_t)255;
}

extern "C" size_t spectra_attend_workspace(int32_t heads, int32_t head_dim, int32_t max_seq) {
  if (heads < 1 || head_dim < 1 || max_seq < 1) return 0;
  return attend_counter_bytes(heads) + attend_part_bytes(heads, head_dim, max_seq);
}

typedef void (*attend_fn)(const uint16_t*, const int64_t*, const float*, const float*, int, int, float, const KvCache,
                          float*, uint32_t*, uint16_t*);

template <int HD, bool ROPE, bool Q4>
static attend_fn pick_attend(int g) {
  switch (g) {
    case 1: return attend_kernel<1, HD, ROPE, Q4>;
    case 2: return attend_kernel<2, HD, ROPE, Q4>;
    case 3: return attend_kernel<3, HD, ROPE, Q4>;
    case 4: return attend_kernel<4, HD, ROPE, Q4>;
    case 6: return attend_kernel<6, HD, ROPE, Q4>;
    case 8: return attend_kernel<8, HD, ROPE, Q4>;
    default: return nullptr;
  }
}

template <bool ROPE, bool Q4>
static attend_fn pick_attend_hd(int hd, int g) {
  switch (hd) {
    case 16: if constexpr (Q4) return nullptr; else return pick_attend<16, ROPE, Q4>(g);
    case 32: return pick_attend<32, ROPE, Q4>(g);
    case 64: return pick_attend<64, ROPE, Q4>(g);
    case 128: return pick_attend<128, ROPE, Q4>(g);
    case 256: return pick_attend<256, ROPE, Q4>(g);
    default: return nullptr;
  }
}

static int attend_launch(const void* qkv, const int64_t* pos, const float* cos_t, const float* sin_t, int32_t heads,
                         int32_t kv_heads, int32_t head_dim, const KvCache& kvc, bool q4, void* workspace,
                         size_t workspace_bytes, void* out, spectra_stream_t stream) {
  SPECTRA_REQUIRE(qkv && pos && kvc.k && kvc.v && out, "NULL pointer");
  SPECTRA_REQUIRE((cos_t == nullptr) == (sin_t == nullptr), "cos and sin must both be given or both be NULL");
  SPECTRA_REQUIRE(heads >= 1 && kv_heads >= 1 && heads % kv_heads == 0, "heads must be a multiple of kv_heads");
  SPECTRA_REQUIRE(head_dim == 16 || head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256,
                  "head_dim must be 16, 32, 64, 128 or 256");
  SPECTRA_REQUIRE(!q4 || head_dim >= 32, "the 4-bit cache needs head_dim >= 32 (groups of 32 dims)");
  SPECTRA_REQUIRE(kvc.lmax >= 1 && kvc.lmax <= (1 << 20), "bad max_seq");
  SPECTRA_REQUIRE(aligned16(qkv) && aligned16(kvc.k) && aligned16(kvc.v) &&
                      (cos_t == nullptr || (aligned16(cos_t) && aligned16(sin_t))),
                  "qkv, the caches and the cos / sin tables must be 16-byte aligned");
  if (q4) {
    SPECTRA_REQUIRE(kvc.kq && kvc.vq && kvc.ks && kvc.vs && kvc.kz && kvc.vz, "NULL 4-bit cache pointer");
    SPECTRA_REQUIRE(kvc.window >= 1 && kvc.window <= kvc.lmax, "window must be in [1, max_seq]");
    SPECTRA_REQUIRE((reinterpret_cast<uintptr_t>(kvc.kq) & 3) == 0 && (reinterpret_cast<uintptr_t>(kvc.vq) & 3) == 0 &&
                        (reinterpret_cast<uintptr_t>(kvc.ks) & 1) == 0 && (reinterpret_cast<uintptr_t>(kvc.vs) & 1) == 0,
                    "4-bit codes must be 4-byte and scales 2-byte aligned");
  }
  if (workspace == nullptr || workspace_bytes < spectra_attend_workspace(heads, head_dim, kvc.lmax) ||
      (reinterpret_cast<uintptr_t>(workspace) & 15))
    return fail(SPECTRA_ERR_WORKSPACE, "workspace missing, unaligned or smaller than spectra_attend_workspace()");
  const int g = heads / kv_heads;
  attend_fn fn;
  if (q4) fn = cos_t ? pick_attend_hd<true, true>(head_dim, g) : nullptr;
  else if (g <= kMfmaMaxGroup && head_dim >= 64)  // the MFMA kernel
    fn = cos_t ? (head_dim == 64 ? attend_mfma_kernel<64, true> : head_dim == 128 ? attend_mfma_kernel<128, true>
                                                                                 : attend_mfma_kernel<256, true>)
               : (head_dim == 64 ? attend_mfma_kernel<64, false> : head_dim == 128 ? attend_mfma_kernel<128, false>
                                                                                  : attend_mfma_kernel<256, false>);
  else fn = cos_t ? pick_attend_hd<true, false>(head_dim, g) : pick_attend_hd<false, false>(head_dim, g);
  if (fn == nullptr)
    return fail(SPECTRA_ERR_UNSUPPORTED, "decode attention serves 1, 2, 3, 4, 6 or 8 query heads per KV head "
                                         "(the 4-bit cache with RoPE)");
  const int nspan = spectra_attend_spans(kvc.lmax);
  const float scale = 1.0f / sqrtf((float)head_dim);
  uint32_t* counter = (uint32_t*)workspace;
  float* part = (float*)((uint8_t*)workspace + attend_counter_bytes(heads));
  const hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(fn, dim3((unsigned)kv_heads, (unsigned)nspan), dim3(kDecThreads), 0, s, (const uint16_t*)qkv,
                     pos, cos_t, sin_t, heads, kv_heads, scale, kvc, part, counter, (uint16_t*)out);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

extern "C" int spectra_attend_decode(const void* qkv, const int64_t* pos, const float* cos_t, const float* sin_t,
                                     int32_t heads, int32_t kv_heads, int32_t head_dim, int32_t max_seq,
                                     void* k_cache, void* v_cache, void* workspace, size_t workspace_bytes, void* out,
                                     spectra_stream_t stream) {
  KvCache kvc{};
  kvc.k = (uint16_t*)k_cache;
  kvc.v = (uint16_t*)v_cache;
  kvc.lmax = max_seq;
  kvc.window = max_seq;
  return attend_launch(qkv, pos, cos_t, sin_t, heads, kv_heads, head_dim, kvc, false, workspace, workspace_bytes, out,
                       stream);
}

extern "C" int spectra_attend_decode_q4(const void* qkv, const int64_t* pos, const float* cos_t, const float* sin_t,
                                        int32_t heads, int32_t kv_heads, int32_t head_dim, int32_t max_seq,
                                        int32_t window, void* k_window, void* v_window, void* k_codes, void* v_codes,
                                        void* k_scales, void* v_scales, void* k_zeros, void* v_zeros,
                                        void* workspace, size_t workspace_bytes, void* out, spectra_stream_t stream) {
  KvCache kvc;
  kvc.k = (uint16_t*)k_window;
  kvc.v = (uint16_t*)v_window;
  kvc.kq = (uint8_t*)k_codes;
  kvc.vq = (uint8_t*)v_codes;
  kvc.ks = (uint16_t*)k_scales;
  kvc.vs = (uint16_t*)v_scales;
  kvc.kz = (uint8_t*)k_zeros;
  kvc.vz = (uint8_t*)v_zeros;
  kvc.lmax = max_seq;
  kvc.window = window;
  return attend_launch(qkv, pos, cos_t, sin_t, heads, kv_heads, head_dim, kvc, true, workspace, workspace_bytes, out,
                       stream);
}

extern "C" int spectra_kv4_quantize(const void* x, int64_t ldx, int64_t rows, int32_t heads, int64_t x_head_stride,
                                    int32_t d, void* codes, void* scales, void* zeros, int64_t out_head_rows,
                                    spectra_stream_t stream) {
  SPECTRA_REQUIRE(x && codes && scales && zeros, "NULL pointer");
  SPECTRA_REQUIRE(d >= 32 && d % 32 == 0 && d <= 4096, "d must be a multiple of 32 in [32, 4096]");
  SPECTRA_REQUIRE(rows >= 1 && heads >= 1 && heads <= 65535 && ldx >= d && out_head_rows >= rows, "bad shape");
  SPECTRA_REQUIRE(aligned16(x) && ldx % 8 == 0 && x_head_stride % 8 == 0, "x must be 16-byte aligned rows");
  SPECTRA_REQUIRE((reinterpret_cast<uintptr_t>(codes) & 3) == 0 && (reinterpret_cast<uintptr_t>(scales) & 1) == 0,
                  "codes must be 4-byte and scales 2-byte aligned");
  const int64_t work = rows * (d / 8);
  SPECTRA_REQUIRE((work + kDecThreads - 1) / kDecThreads < (int64_t(1) << 31), "too many rows");
  hipLaunchKernelGGL(kv4_quantize_kernel, dim3((unsigned)((work + kDecThreads - 1) / kDecThreads), (unsigned)heads),
                     dim3(kDecThreads), 0, (hipStream_t)stream, (const uint16_t*)x, ldx, x_head_stride, rows, d,
                     out_head_rows, (uint8_t*)codes, (uint16_t*)scales, (uint8_t*)zeros);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

extern "C" int spectra_kv4_dequantize(const void* codes, const void* scales, const void* zeros, int64_t rows, int32_t d,
                                      void* out_bf16, spectra_stream_t stream) {
  SPECTRA_REQUIRE(codes && scales && zeros && out_bf16, "NULL pointer");
  SPECTRA_REQUIRE(d >= 32 && d % 32 == 0 && d <= 4096 && rows >= 1, "bad shape");
  SPECTRA_REQUIRE(aligned16(out_bf16) && (reinterpret_cast<uintptr_t>(codes) & 3) == 0, "misaligned operands");
  const int64_t work = rows * (d / 8);
  SPECTRA_REQUIRE((work + kDecThreads - 1) / kDecThreads < (int64_t(1) << 31), "too many rows");
  hipLaunchKernelGGL(kv4_dequantize_kernel, dim3((unsigned)((work + kDecThreads - 1) / kDecThreads)),
                     dim3(kDecThreads), 0, (hipStream_t)stream, (const uint8_t*)codes, (const uint16_t*)scales,
                     (const uint8_t*)zeros, rows, d, (uint16_t*)out_bf16);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

extern "C" int spectra_silu_mul(const void* gate_up, int64_t ldgu, int64_t rows, int64_t inter, void* act,
                                spectra_stream_t stream) {
  SPECTRA_REQUIRE(gate_up && act, "NULL pointer");
  SPECTRA_REQUIRE(rows >= 1 && inter >= 1 && inter < (int64_t(1) << 30) && ldgu >= 2 * inter, "bad shape");
  const int64_t n = rows * inter;
  SPECTRA_REQUIRE((n + kDecThreads - 1) / kDecThreads < (int64_t(1) << 31), "too many elements");
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n + kDecThreads - 1) / kDecThreads)), dim3(kDecThreads), 0,
                     (hipStream_t)stream, (const uint16_t*)gate_up, ldgu, (int)inter, n, (uint16_t*)act);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

extern "C" int spectra_greedy_finish(void* argmax_key, int64_t* token, int64_t* history, int64_t hist_len,
                                     int64_t* pos, spectra_stream_t stream) {
  SPECTRA_REQUIRE(argmax_key && token, "NULL pointer");
  SPECTRA_REQUIRE((reinterpret_cast<uintptr_t>(argmax_key) & 7) == 0, "argmax slots must be 8-byte aligned");
  SPECTRA_REQUIRE(history == nullptr || (pos != nullptr && hist_len >= 1), "history needs pos and a length");
  static_assert(SPECTRA_ARGMAX_SLOTS % 64 == 0, "one wave reads the slots, the same count per lane");
  hipLaunchKernelGGL(greedy_finish_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (unsigned long long*)argmax_key, token, history, hist_len, pos);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

extern "C" int spectra_greedy_next(const void* logits, int64_t n, int64_t* token, int64_t* history, int64_t hist_len,
                                   int64_t* pos, spectra_stream_t stream) {
  SPECTRA_REQUIRE(logits && token, "NULL pointer");
  SPECTRA_REQUIRE(n >= 1 && n < (int64_t(1) << 31), "bad logit count");
  SPECTRA_REQUIRE(aligned16(logits), "logits must be 16-byte aligned");
  SPECTRA_REQUIRE(history == nullptr || (pos != nullptr && hist_len >= 1), "history needs pos and a length");
  hipLaunchKernelGGL(greedy_kernel, dim3(1), dim3(kArgThreads), 0, (hipStream_t)stream, (const uint16_t*)logits,
                     (int)n, token, history, hist_len, pos);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}
