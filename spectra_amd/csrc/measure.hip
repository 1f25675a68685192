// Measurement-only kernels: the floor and the ceiling that bound a one-launch HBM stream on
// this GPU, timed by bench.py beside the GEMVs (no counterpart in the reference).
//
//  * spectra_measure_empty: a kernel that does nothing, launched with a given geometry; a
//    graph of such launches times the fixed cost of one launch (dispatch, wave launch and
//    retirement, the kernel-boundary cache maintenance).
//  * spectra_measure_read: a plain streaming read of `bytes` with the GEMV's load pattern
//    (workgroup b reads one contiguous slice; each thread issues all of its 16-byte
//    non-temporal loads before the first use; one wave-instruction covers 1 KB), XOR-folded
//    so the loads cannot be removed; nothing is stored unless the fold hits a magic value.
#include <hip/hip_runtime.h>

#include "common.h"
#include "gemv_stream.h"  // load_nt_u4

namespace spectra {

__global__ void measure_empty_kernel() {}

template <int U>
__global__ void __launch_bounds__(1024) measure_read_kernel(const uint8_t* __restrict__ src, int64_t units,
                                                            int64_t per_wg, uint32_t* __restrict__ sink) {
  const int64_t u0 = (int64_t)blockIdx.x * per_wg;
  if (u0 >= units) return;  // a workgroup past the end (wave-uniform)
  const int64_t u1 = min(u0 + per_wg, units);
  uint4 v[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const int64_t u = u0 + (int64_t)threadIdx.x + (int64_t)i * blockDim.x;
    v[i] = load_nt_u4(src + 16 * (u < u1 ? u : u0));  // past the slice: re-read its first unit
  }
  uint32_t a = 0;
#pragma unroll
  for (int i = 0; i < U; ++i) a ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  if (a == 0x5bd1e995u) sink[threadIdx.x] = a;
}

}  // namespace spectra

using namespace spectra;

extern "C" int spectra_measure_empty(int32_t grid, int32_t block, spectra_stream_t stream) {
  SPECTRA_REQUIRE(grid >= 1 && block >= 1 && block <= 1024, "bad launch geometry");
  hipLaunchKernelGGL(measure_empty_kernel, dim3((unsigned)grid), dim3((unsigned)block), 0, (hipStream_t)stream);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}

extern "C" int spectra_measure_read(const void* src, size_t bytes, int32_t grid, int32_t block, void* sink,
                                    spectra_stream_t stream) {
  SPECTRA_REQUIRE(src != nullptr && sink != nullptr, "NULL pointer");
  SPECTRA_REQUIRE((reinterpret_cast<uintptr_t>(src) & 15) == 0 && bytes >= 16 && bytes % 16 == 0,
                  "src must be 16-byte aligned and bytes a positive multiple of 16");
  SPECTRA_REQUIRE(grid >= 1 && block >= 64 && block <= 1024 && block % 64 == 0, "bad launch geometry");
  SPECTRA_REQUIRE((reinterpret_cast<uintptr_t>(sink) & 3) == 0, "sink must be 4-byte aligned (block words)");
  const int64_t units = (int64_t)(bytes / 16);
  const int64_t per_wg = (units + grid - 1) / grid;
  const int64_t per_thread = (per_wg + block - 1) / block;
  typedef void (*read_fn)(const uint8_t*, int64_t, int64_t, uint32_t*);
  read_fn fn = per_thread <= 1 ? measure_read_kernel<1> : per_thread <= 2 ? measure_read_kernel<2>
             : per_thread <= 4 ? measure_read_kernel<4> : per_thread <= 8 ? measure_read_kernel<8>
             : per_thread <= 16 ? measure_read_kernel<16> : nullptr;
  if (fn == nullptr) return fail(SPECTRA_ERR_UNSUPPORTED, "more than 16 loads per thread: raise grid or block");
  hipLaunchKernelGGL(fn, dim3((unsigned)grid), dim3((unsigned)block), 0, (hipStream_t)stream,
                     (const uint8_t*)src, units, per_wg, (uint32_t*)sink);
  SPECTRA_HIP_CHECK(hipGetLastError());
  return SPECTRA_OK;
}
