// Shared device/host helpers for the gfx950 W4A16 library.
// Compiled with -ffp-contract=off: every float operation below rounds exactly
// where it is written, which the bit-exact quantizer/dequant kernels rely on.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "spectra_hip.h"

namespace spectra {

// ---------------------------------------------------------------------------
// error reporting (host)
// ---------------------------------------------------------------------------
void set_error(const std::string& msg);
int fail(int status, const std::string& msg);
#define SPECTRA_REQUIRE(cond, msg)                                   \
  do {                                                               \
    if (!(cond)) return ::spectra::fail(SPECTRA_ERR_INVALID, (msg)); \
  } while (0)
// On failure the runtime's sticky error is read back (cleared) so that it cannot be
// reported again by an unrelated later call.
#define SPECTRA_HIP_CHECK(expr)                                                        \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess) {                                                            \
      (void)hipGetLastError();                                                         \
      return ::spectra::fail(SPECTRA_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    }                                                                                  \
  } while (0)

// Validates a spectra_qweight_t (shapes, pointers, alignment); returns status.
int validate_qweight(const spectra_qweight_t* w);
// Raises a kernel's dynamic-LDS limit to the device maximum once per (kernel, device).
// dyn_at_zero: the kernel addresses dynamic LDS from address 0 (fails if it has static LDS).
int ensure_lds_limit(const void* kernel, bool dyn_at_zero = false);
inline bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }
// Compute units of the current device (hipDeviceAttributeMultiprocessorCount, queried once
// per device): the launch plans size their grids to it.  Falls back to 256 (MI355X) if the
// query fails.
int device_cu_count();

// ---------------------------------------------------------------------------
// NF4 codebook (compressor.py:22-27): fp32 literals and their fp16 roundings
// ---------------------------------------------------------------------------
__device__ __forceinline__ float nf4_code_f32(int i) {
  // select chain over literal constants: no memory access, any lane index
  float r = -1.0f;
  r = (i == 1) ? -0.6961928009986877f : r;
  r = (i == 2) ? -0.5250730514526367f : r;
  r = (i == 3) ? -0.39491748809814453f : r;
  r = (i == 4) ? -0.28444138169288635f : r;
  r = (i == 5) ? -0.18477343022823334f : r;
  r = (i == 6) ? -0.09105003625154495f : r;
  r = (i == 7) ? 0.0f : r;
  r = (i == 8) ? 0.07958029955625534f : r;
  r = (i == 9) ? 0.16093020141124725f : r;
  r = (i == 10) ? 0.24611230194568634f : r;
  r = (i == 11) ? 0.33791524171829224f : r;
  r = (i == 12) ? 0.44070982933044434f : r;
  r = (i == 13) ? 0.5626170039176941f : r;
  r = (i == 14) ? 0.7229568362236023f : r;
  r = (i == 15) ? 1.0f : r;
  return r;
}

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

// ---------------------------------------------------------------------------
// 16-bit float conversions (round-to-nearest-even)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);  // v_cvt_f16_f32, RNE
}
__device__ __forceinline__ float bf2f(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
// Nibble-pair LUT at LDS address 0: row v (a packed byte) holds the fp16 pair
// (code[v & 15], code[v >> 4]) -- NF4 levels, or the integers 0..15 for Format A -- in 64
// copies, so lane l reads its own copy at v * 256 + 4 l (one bank per lane).  Wave w of
// nwaves fills the rows of high codes h = w, w + nwaves, ...: 16 rows of 256 B as four
// wave-instructions of 1 KB (lane >> 4 picks the row, lane & 15 the 16-byte chunk:
// conflict-free).  The high code is wave-uniform (scalar work) and the low code one of
// four per lane, so the build reads no LDS and selects nothing per entry.
// fp16 bits of the 16 codes, two per dword (code 2i in the low half): NF4 levels, and the
// integers 0..15 (Format A)
constexpr uint32_t kNf4CodePairs[8] = {0xb992bc00u, 0xb652b833u, 0xb1eab48du, 0x0000add4u,
                                       0x31262d18u, 0x356833e0u, 0x3880370du, 0x3c0039c9u};
constexpr uint32_t kIntCodePairs[8] = {0x3c000000u, 0x42004000u, 0x45004400u, 0x47004600u,
                                       0x48804800u, 0x49804900u, 0x4a804a00u, 0x4b804b00u};

template <int FMT>
__device__ __forceinline__ void build_pair_lut(uint8_t* smem, int wave, int nwaves, int lane) {
  const uint32_t* pairs = FMT == SPECTRA_FMT_NF4 ? kNf4CodePairs : kIntCodePairs;
  // low code 4 c + j (j = lane >> 4): bytes 2j, 2j + 1 of the dword pair (2c, 2c + 1)
  const uint32_t j2 = (uint32_t)(lane >> 4) * 2u;
  const uint32_t sel = 0x0c0c0000u | ((j2 + 1u) << 8) | j2;
  uint32_t lo4[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) lo4[c] = __builtin_amdgcn_perm(pairs[2 * c + 1], pairs[2 * c], sel);
  uint4* lut = (uint4*)smem;
  for (int h = wave; h < 16; h += nwaves) {
    // the high code (wave-uniform): code h sits in lo4[h >> 2] of lane 16 (h & 3)
    const int hq = h >> 2;
    const uint32_t src = hq == 0 ? lo4[0] : hq == 1 ? lo4[1] : hq == 2 ? lo4[2] : lo4[3];
    const uint32_t hb = (uint32_t)__builtin_amdgcn_readlane((int)src, 16 * (h & 3)) << 16;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t e = lo4[c] | hb;
      lut[(16 * h + 4 * c + (lane >> 4)) * 16 + (lane & 15)] = make_uint4(e, e, e, e);
    }
  }
}

// The same table in 32 copies (lanes l and l + 32 share copy l & 31: the LDS serves a
// wave's 4-byte reads in two halves of 32 lanes, one bank per lane in each): row v at
// v * 256, copy c at + 4 c (the upper 128 bytes of every row are not written), half the
// LDS writes of build_pair_lut.  Wave w of nwaves fills the rows of high codes w,
// w + nwaves, ...: 16 rows of 128 B as two wave-instructions of 1 KB (lane >> 3 picks the
// row, lane & 7 the 16-byte chunk).  Readers address it with ((lane & 31) << 2).
template <int FMT>
__device__ __forceinline__ void build_pair_lut32(uint8_t* smem, int wave, int nwaves, int lane) {
  const uint32_t* pairs = FMT == SPECTRA_FMT_NF4 ? kNf4CodePairs : kIntCodePairs;
  const int m = lane >> 3;  // low codes m and 8 + m
  const uint32_t pa = m < 2 ? pairs[0] : m < 4 ? pairs[1] : m < 6 ? pairs[2] : pairs[3];
  const uint32_t pb = m < 2 ? pairs[4] : m < 4 ? pairs[5] : m < 6 ? pairs[6] : pairs[7];
  const uint32_t c0 = (m & 1) ? (pa >> 16) : (pa & 0xffffu), c1 = (m & 1) ? (pb >> 16) : (pb & 0xffffu);
  uint4* lut = (uint4*)smem;
  for (int h = wave; h < 16; h += nwaves) {
    // the high code (wave-uniform): code h sits in c0 (h < 8) or c1 of lane 8 (h & 7)
    const uint32_t hb = (uint32_t)__builtin_amdgcn_readlane((int)(h < 8 ? c0 : c1), 8 * (h & 7)) << 16;
    const uint32_t e0 = c0 | hb, e1 = c1 | hb;
    lut[(16 * h + m) * 16 + (lane & 7)] = make_uint4(e0, e0, e0, e0);
    lut[(16 * h + 8 + m) * 16 + (lane & 7)] = make_uint4(e1, e1, e1, e1);
  }
}

// Load through a wave-uniform base plus a 32-bit per-lane byte offset: the global_load
// saddr form (base in SGPRs, offset in one VGPR), with no per-lane 64-bit address math.
template <typename T>
__device__ __forceinline__ T load_at(const void* base, uint32_t byte_off) {
  typedef const __attribute__((address_space(1))) uint8_t* gbyte_t;
  typedef const __attribute__((address_space(1))) T* gT_t;
  gbyte_t b = (gbyte_t)base;  // global memory (the kernels take device pointers)
  asm("" : "+s"(b));          // keep the base in SGPRs (no re-association into per-lane math)
  // loaded as a plain integer vector of the same size (the HIP vector types have no
  // constructor from a global-address-space reference)
  if constexpr (sizeof(T) == 16) {
    typedef uint32_t v4_t __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(T, *(const __attribute__((address_space(1))) v4_t*)(b + byte_off));
  } else if constexpr (sizeof(T) == 8) {
    typedef uint32_t v2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(T, *(const __attribute__((address_space(1))) v2_t*)(b + byte_off));
  } else {
    return *(gT_t)(b + byte_off);
  }
}

// ---------------------------------------------------------------------------
// cross-lane Walsh-Hadamard butterflies (activation prep of the GEMM and small-batch families)
// ---------------------------------------------------------------------------
// Value of lane (lane ^ LB) for LB = 1 .. 32, on the VALU: DPP quad permutes (1, 2), a
// half-row mirror then a quad reversal (4), a row rotation by 8 (8), and the row swaps
// v_permlane16_swap / v_permlane32_swap (16, 32).
template <int LB>
__device__ __forceinline__ float lane_xor(float v, int lane) {
  const int iv = __builtin_bit_cast(int, v);
  if constexpr (LB == 1) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0xB1, 0xF, 0xF, false));
  else if constexpr (LB == 2) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x4E, 0xF, 0xF, false));
  else if constexpr (LB == 4) {
    const int t = __builtin_amdgcn_mov_dpp(iv, 0x141, 0xF, 0xF, false);  // l -> 7 - l inside 8 lanes
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(t, 0x1B, 0xF, 0xF, false));  // then quad reversed
  } else if constexpr (LB == 8) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x128, 0xF, 0xF, false));
  else if constexpr (LB == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(iv, iv, false, false);
    return __builtin_bit_cast(float, (int)((lane & 16) ? r[0] : r[1]));
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(iv, iv, false, false);
    return __builtin_bit_cast(float, (int)((lane & 32) ? r[0] : r[1]));
  }
}

// All-reductions across the wave through lane_xor (no LDS round trips): partners 32, 16,
// ..., 1, the order of a __shfl_xor butterfly, so the same result in every lane.
__device__ __forceinline__ float wave_sum(float v) {
  const int lane = __lane_id();
  v += lane_xor<32>(v, lane);
  v += lane_xor<16>(v, lane);
  v += lane_xor<8>(v, lane);
  v += lane_xor<4>(v, lane);
  v += lane_xor<2>(v, lane);
  return v + lane_xor<1>(v, lane);
}
__device__ __forceinline__ float wave_max(float v) {
  const int lane = __lane_id();
  v = fmaxf(v, lane_xor<32>(v, lane));
  v = fmaxf(v, lane_xor<16>(v, lane));
  v = fmaxf(v, lane_xor<8>(v, lane));
  v = fmaxf(v, lane_xor<4>(v, lane));
  v = fmaxf(v, lane_xor<2>(v, lane));
  return fmaxf(v, lane_xor<1>(v, lane));
}

// Butterfly across lanes at distance LB: v += c * partner with c = +1 on the low side and
// -1 on the high side, leaving u + v low and -(u - v) high (the product by +-1 is exact
// and the fma rounds once, as the reference's add / subtract does).  Partners share their
// sign before every stage, and the lane's final sign (-1)^(high sides taken) rides on
// the output scale.
// (distances 1, 2, 8: one v_fmac_f32_dpp per value, eight per block behind the two wait
// states a DPP source needs after its VALU write)
#define SPECTRA_PFLY(CTRL, A)                                                          \
  asm volatile("s_nop 1\n"                                                            \
               "v_fmac_f32_dpp %0, %0, %8 " CTRL " row_mask:0xf bank_mask:0xf\n"      \
               "v_fmac_f32_dpp %1, %1, %8 " CTRL " row_mask:0xf bank_mask:0xf\n"      \
               "v_fmac_f32_dpp %2, %2, %8 " CTRL " row_mask:0xf bank_mask:0xf\n"      \
               "v_fmac_f32_dpp %3, %3, %8 " CTRL " row_mask:0xf bank_mask:0xf\n"      \
               "v_fmac_f32_dpp %4, %4, %8 " CTRL " row_mask:0xf bank_mask:0xf\n"      \
               "v_fmac_f32_dpp %5, %5, %8 " CTRL " row_mask:0xf bank_mask:0xf\n"      \
               "v_fmac_f32_dpp %6, %6, %8 " CTRL " row_mask:0xf bank_mask:0xf\n"      \
               "v_fmac_f32_dpp %7, %7, %8 " CTRL " row_mask:0xf bank_mask:0xf\n"      \
               : "+v"(A[0]), "+v"(A[1]), "+v"(A[2]), "+v"(A[3]), "+v"(A[4]), "+v"(A[5]), \
                 "+v"(A[6]), "+v"(A[7])                                                 \
               : "v"(c))

template <int LB, int U>
__device__ __forceinline__ void prep_fly(float (&v)[U][8], float c, int lane) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if constexpr (LB == 1) SPECTRA_PFLY("quad_perm:[1,0,3,2]", v[u]);
    else if constexpr (LB == 2) SPECTRA_PFLY("quad_perm:[2,3,0,1]", v[u]);
    else if constexpr (LB == 8) SPECTRA_PFLY("row_ror:8", v[u]);
    else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[u][e] = __builtin_fmaf(lane_xor<LB>(v[u][e], lane), c, v[u][e]);
    }
  }
}

// dtype-tagged load/store of one element
__device__ __forceinline__ float load_elem(const void* p, int64_t i, int dtype) {
  if (dtype == SPECTRA_F16) return h2f(((const uint16_t*)p)[i]);
  if (dtype == SPECTRA_BF16) return bf2f(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}
__device__ __forceinline__ void store_elem(void* p, int64_t i, int dtype, float v) {
  if (dtype == SPECTRA_F16) ((uint16_t*)p)[i] = f2h(v);
  else if (dtype == SPECTRA_BF16) ((uint16_t*)p)[i] = f2bf(v);
  else ((float*)p)[i] = v;
}
__device__ __forceinline__ float to_f32_16(uint16_t v, int dtype) {
  return dtype == SPECTRA_BF16 ? bf2f(v) : h2f(v);
}
__device__ __forceinline__ uint16_t from_f32_16(float v, int dtype) {
  return dtype == SPECTRA_BF16 ? f2bf(v) : f2h(v);
}

// k index of nibble `half` (0 = low, 1 = high) of packed byte j in a row
__host__ __device__ __forceinline__ int64_t nibble_k(int64_t j, int half, int marlin) {
  return marlin ? ((j >> 4) << 5) + (j & 15) + (half << 4) : 2 * j + half;
}
// inverse: (byte j, half) holding element k
__host__ __device__ __forceinline__ void k_to_nibble(int64_t k, int marlin, int64_t* j, int* half) {
  if (marlin) {
    *j = ((k >> 5) << 4) + (k & 15);
    *half = (int)((k >> 4) & 1);
  } else {
    *j = k >> 1;
    *half = (int)(k & 1);
  }
}

inline int elem_size(int dtype) { return dtype == SPECTRA_F32 ? 4 : 2; }

}  // namespace spectra
