// Measurement probes (not part of the C ABI in include/pie_hip.h): plain kernels with the access
// pattern of a hot-path kernel and none of its arithmetic or index logic, so the bench can put a
// measured ceiling for that pattern beside the kernel's own figure.
//   pie_probe_copy:     dst[i] = src[i] over n 16-byte vectors, grid flattened like the
//                       streaming kernels (one vector per thread), non-temporal or cached.
//   pie_probe_scatter:  the paged append's pattern: row t (row_bytes, a multiple of 16) at
//                       src + src_off[t] bytes goes to dst + dst_off[t] bytes (offsets computed
//                       beforehand, so no page-table reads), one 16-byte vector per thread,
//                       non-temporal loads and stores.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__global__ __launch_bounds__(256) void probe_copy_kernel(const u32x4* __restrict__ src,
                                                         u32x4* __restrict__ dst, uint32_t n) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= n) return;
  if constexpr (NT) {
    __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
  } else {
    dst[i] = src[i];
  }
}

__global__ __launch_bounds__(256) void probe_scatter_kernel(const char* __restrict__ src,
                                                            char* __restrict__ dst,
                                                            const int64_t* __restrict__ src_off,
                                                            const int64_t* __restrict__ dst_off,
                                                            uint32_t vpr, uint32_t n) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= n) return;
  const uint32_t row = i / vpr, c = i - row * vpr;
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + src_off[row]) + c);
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dst + dst_off[row]) + c);
}

extern "C" int pie_probe_copy(const void* src, void* dst, int64_t bytes, int nt, void* stream) {
  if (bytes % 16 || bytes / 16 >= (1ll << 32) || (reinterpret_cast<uintptr_t>(src) & 15) ||
      (reinterpret_cast<uintptr_t>(dst) & 15))
    return 1;
  const uint32_t n = (uint32_t)(bytes / 16);
  const dim3 g((n + 255) / 256), b(256);
  if (nt) hipLaunchKernelGGL(probe_copy_kernel<true>, g, b, 0, (hipStream_t)stream, (const u32x4*)src, (u32x4*)dst, n);
  else hipLaunchKernelGGL(probe_copy_kernel<false>, g, b, 0, (hipStream_t)stream, (const u32x4*)src, (u32x4*)dst, n);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

extern "C" int pie_probe_scatter(const void* src, const int64_t* src_off, void* dst,
                                 const int64_t* dst_off, int64_t rows, int64_t row_bytes, void* stream) {
  if (row_bytes % 16 || rows * (row_bytes / 16) >= (1ll << 32)) return 1;
  const uint32_t vpr = (uint32_t)(row_bytes / 16), n = (uint32_t)(rows * vpr);
  hipLaunchKernelGGL(probe_scatter_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     (const char*)src, (char*)dst, src_off, dst_off, vpr, n);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
