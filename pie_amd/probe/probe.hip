// Measurement probes (not part of the C ABI in include/pie_hip.h): plain kernels with the access
// pattern of a hot-path kernel and none of its arithmetic or index logic, so the bench can put a
// measured ceiling for that pattern beside the kernel's own figure.
//   pie_probe_copy:     dst[i] = src[i] over n 16-byte vectors, grid flattened like the
//                       streaming kernels (one vector per thread), non-temporal or cached.
//   pie_probe_scatter:  the paged append's pattern: row t (row_bytes, a multiple of 16) at
//                       src + src_off[t] bytes goes to dst + dst_off[t] bytes (offsets computed
//                       beforehand, so no page-table reads), one 16-byte vector per thread,
//                       non-temporal loads and stores.
//   pie_probe_read:     reads n 16-byte vectors, each work group a contiguous chunk of
//                       threads x vpt vectors with all of a thread's vpt loads issued before any
//                       is used (the resident softmax's pattern at 1024 threads and vpt 16),
//                       one xor per work group written out.
//   pie_probe_read_rows: a row-per-work-group read on the kernels' own row layout: one 1024-thread
//                       work group per row of row_vec 16-byte vectors at a row stride of
//                       stride_vec vectors, in rounds of 16 loads per thread (indices past the
//                       row clamped to its last vector), each round's loads all issued before
//                       any is used (one round: the resident softmax's read phase; two: a
//                       sampler row of fp32 probabilities).
//   pie_probe_mfma:     dense bf16 v_mfma_f32_32x32x16 throughput, 2 work groups of 4 waves per
//                       CU: 4 independent accumulator chains per wave (valu = 0), with 128
//                       independent fp32 fma per 16 MFMAs (1: does vector work overlap the
//                       matrix pipe?).
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

template <int VPT>
__global__ __launch_bounds__(1024) void probe_read_kernel(const u32x4* __restrict__ src, uint32_t* __restrict__ out) {
  const u32x4* p = src + (size_t)blockIdx.x * blockDim.x * VPT;
  u32x4 v[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) v[j] = __builtin_nontemporal_load(p + threadIdx.x + j * blockDim.x);
  uint32_t x = 0;
#pragma unroll
  for (int j = 0; j < VPT; ++j) x ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  __shared__ uint32_t acc;
  if (threadIdx.x == 0) acc = 0;
  __syncthreads();
  atomicXor(&acc, x);
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = acc;
}

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
// VALU 0: 4 independent accumulator chains of v_mfma_f32_32x32x16_bf16 per wave; 1: the same
// with 128 independent fp32 fma per 16 MFMAs (does vector work overlap the matrix pipe?).
template <int VALU>
__global__ __launch_bounds__(256, 2) void probe_mfma_kernel(float* out, int iters) {
  f32x16 acc0 = {}, acc1 = {}, acc2 = {}, acc3 = {};
  bf16x8 a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(threadIdx.x * 0.001f + i);
    b[i] = (__bf16)(i * 0.5f);
  }
  float v[8];
  for (int i = 0; i < 8; ++i) v[i] = threadIdx.x + i;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc1, 0, 0, 0);
      acc2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc2, 0, 0, 0);
      acc3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc3, 0, 0, 0);
      if constexpr (VALU == 1) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] = fmaf(v[i], 1.0001f, 0.5f);
      }
    }
  }
  float s = 0.f;
  for (int i = 0; i < 8; ++i) s += v[i];
  for (int i = 0; i < 16; ++i) s += acc0[i] + acc1[i] + acc2[i] + acc3[i];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

// flops of one launch: blocks * 4 waves * iters * 16 MFMAs * 32768
extern "C" int pie_probe_mfma(float* out, int blocks, int iters, int valu, void* stream) {
  if (blocks <= 0 || iters <= 0) return 1;
  switch (valu) {
    case 0: hipLaunchKernelGGL(probe_mfma_kernel<0>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters); break;
    case 1: hipLaunchKernelGGL(probe_mfma_kernel<1>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters); break;
    default: return 1;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

__global__ __launch_bounds__(1024) void probe_read_rows_kernel(const u32x4* __restrict__ src, int row_vec,
                                                               int64_t stride_vec, int rounds,
                                                               uint32_t* __restrict__ out) {
  const u32x4* p = src + (int64_t)blockIdx.x * stride_vec;
  uint32_t x = 0;
  for (int q = 0; q < rounds; ++q) {
    u32x4 v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j)
      v[j] = __builtin_nontemporal_load(p + min((int)threadIdx.x + 1024 * (16 * q + j), row_vec - 1));
#pragma unroll
    for (int j = 0; j < 16; ++j) x ^= v[j].x ^ v[j].y ^ v[j].z ^ v[j].w;
  }
  if (x == 0x9e3779b9u) out[blockIdx.x] = x;  // keeps the loads; practically never written
}

extern "C" int pie_probe_read_rows(const void* src, int rows, int row_vec, int64_t stride_vec, uint32_t* out,
                                   void* stream) {
  if (rows <= 0 || row_vec <= 0 || row_vec > 2 * 16 * 1024 || stride_vec < row_vec ||
      (reinterpret_cast<uintptr_t>(src) & 15))
    return 1;
  const int rounds = (row_vec + 16 * 1024 - 1) / (16 * 1024);
  hipLaunchKernelGGL(probe_read_rows_kernel, dim3((unsigned)rows), dim3(1024), 0, (hipStream_t)stream,
                     (const u32x4*)src, row_vec, stride_vec, rounds, out);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

extern "C" int pie_probe_read(const void* src, int64_t bytes, int threads, int vpt, uint32_t* out, void* stream) {
  const int64_t chunk = (int64_t)threads * vpt * 16;
  if (threads < 64 || threads > 1024 || threads % 64 || bytes % chunk || (reinterpret_cast<uintptr_t>(src) & 15))
    return 1;
  const dim3 g((unsigned)(bytes / chunk)), b((unsigned)threads);
  switch (vpt) {
    case 4: hipLaunchKernelGGL(probe_read_kernel<4>, g, b, 0, (hipStream_t)stream, (const u32x4*)src, out); break;
    case 8: hipLaunchKernelGGL(probe_read_kernel<8>, g, b, 0, (hipStream_t)stream, (const u32x4*)src, out); break;
    case 16: hipLaunchKernelGGL(probe_read_kernel<16>, g, b, 0, (hipStream_t)stream, (const u32x4*)src, out); break;
    default: return 1;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
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
