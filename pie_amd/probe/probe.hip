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
//   pie_probe_mfma:     dense bf16 v_mfma_f32_32x32x16 throughput, 2 work groups of 4 waves per
//                       CU: 4 independent accumulator chains per wave (valu = 0), with 128
//                       independent fp32 fma per 16 MFMAs (1: does vector work overlap the
//                       matrix pipe?), one dependent chain (2), and a ladder towards the prefill
//                       attention tile (3-10: its dependency shape, its softmax, its operands
//                       from LDS, a barrier per tile; see probe_mfma_kernel).
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
// MODE 0: 4 independent accumulator chains; 1: the same with 128 independent fp32 fma per 16
// MFMAs; 2: one dependent chain of 16; 3: an attention tile's dependency shape without its
// vector math: a chain of 8 into a score accumulator, its 16 values packed to bf16 (8
// conversions), then 8 MFMAs over 4 output accumulators that take the packed scores as operand B;
// 4: MODE 3 with a softmax's vector work between the chains (maximum, 16 fma + exp2, sum);
// 5: MODE 4 with the K and V operands read from LDS; 6: MODE 5 with a work-group barrier per tile;
// 7: MODE 5 with only the K operands from LDS; 8: MODE 5 with only the V operands from LDS;
// 10: MODE 6 with V stored transposed (rows of 80 bytes), its operands read by ds_read_b128.
template <int MODE>
__global__ __launch_bounds__(256, 2) void probe_mfma_kernel(float* out, int iters) {
  f32x16 acc0 = {}, acc1 = {}, acc2 = {}, acc3 = {};
  bf16x8 a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(threadIdx.x * 0.001f + i);
    b[i] = (__bf16)(i * 0.5f);
  }
  float v[8];
  for (int i = 0; i < 8; ++i) v[i] = threadIdx.x + i;
  // MODE 5/6: K operands (16 B per lane per step) and V operands (two ds_read_b64_tr_b16 each)
  // read from a 16 KiB LDS tile, as the prefill kernel reads them
  __shared__ __attribute__((aligned(16))) uint16_t tile[2][32 * 128];
  if constexpr (MODE >= 5) {
    for (int i = threadIdx.x; i < 2 * 32 * 128; i += 256) (&tile[0][0])[i] = (uint16_t)(i * 7);
    __syncthreads();
  }
  const int lane = threadIdx.x & 63;
  for (int it = 0; it < iters; ++it) {
    if constexpr (MODE >= 3) {
      f32x16 s = {};
      int koff = 0;  // opaque to the compiler, so the tile reads stay inside the loop
      asm volatile("" : "+v"(koff));
      if constexpr (MODE >= 5 && MODE != 8) {
        bf16x8 kr[8];
#pragma unroll
        for (int k = 0; k < 8; ++k)
          kr[k] = *reinterpret_cast<const bf16x8*>(&tile[0][koff + (lane & 31) * 128 + 8 * ((2 * k + (lane >> 5)) ^ (lane & 15))]);
#pragma unroll
        for (int k = 0; k < 8; ++k) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kr[k], b, s, 0, 0, 0);
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, s, 0, 0, 0);
      }
      bf16x8 p0, p1;
      if constexpr (MODE >= 4) {
        float mx = s[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[i]);
        float e[16], l = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) e[i] = __builtin_amdgcn_exp2f(fmaf(s[i], 1e-3f, -mx));
#pragma unroll
        for (int i = 0; i < 16; ++i) l += e[i];
        v[it & 7] += l;
#pragma unroll
        for (int i = 0; i < 8; ++i) { p0[i] = (__bf16)e[i]; p1[i] = (__bf16)e[8 + i]; }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) { p0[i] = (__bf16)(s[i] * 1e-30f); p1[i] = (__bf16)(s[8 + i] * 1e-30f); }
      }
      if constexpr (MODE == 10) {
        f32x16* accs[4] = {&acc0, &acc1, &acc2, &acc3};
        const char* vt = reinterpret_cast<const char*>(&tile[1][0]);
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          const int d = 32 * (n % 4) + (lane & 31), j = n / 4;
          const bf16x8 va = *reinterpret_cast<const bf16x8*>(vt + koff + (d & 63) * 80 + 16 * ((2 * j + (lane >> 5)) ^ ((d >> 4) & 3)));
          *accs[n % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, n < 4 ? p0 : p1, *accs[n % 4], 0, 0, 0);
        }
        __syncthreads();
        continue;
      }
      if constexpr (MODE >= 5 && MODE != 7) {
        typedef short s4 __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) s4 lds_s4;
        f32x16* accs[4] = {&acc0, &acc1, &acc2, &acc3};
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          const int r = 16 * (n / 4) + 4 * (lane >> 5) + ((lane >> 2) & 3);
          const uint16_t* base = &tile[1][koff + r * 128 + 8 * ((4 * (n % 4) + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1)) ^ (((lane >> 2) & 3) << 2)) + 4 * (lane & 1)];
          const s4 h0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(base));
          const s4 h1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(base + 8 * 128));
          bf16x8 va;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            va[i] = __builtin_bit_cast(__bf16, h0[i]);
            va[4 + i] = __builtin_bit_cast(__bf16, h1[i]);
          }
          *accs[n % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, n < 4 ? p0 : p1, *accs[n % 4], 0, 0, 0);
        }
        if constexpr (MODE == 6) __syncthreads();
        continue;
      }
      if constexpr (MODE == 7) a[0] = __builtin_bit_cast(__bf16, (short)koff);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, p0, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, p0, acc1, 0, 0, 0);
      acc2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, p0, acc2, 0, 0, 0);
      acc3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, p0, acc3, 0, 0, 0);
      acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, p1, acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, p1, acc1, 0, 0, 0);
      acc2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, p1, acc2, 0, 0, 0);
      acc3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, p1, acc3, 0, 0, 0);
      continue;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if constexpr (MODE == 2) {
#pragma unroll
        for (int k = 0; k < 4; ++k) acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc0, 0, 0, 0);
      } else {
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc1, 0, 0, 0);
        acc2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc2, 0, 0, 0);
        acc3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc3, 0, 0, 0);
      }
      if constexpr (MODE == 1) {
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
// MODE 9: the MODE 5 tile (softmax, K and V operands from LDS) with 64 query rows per wave, two
// 32-row blocks that share every K and V operand read, one wave per SIMD (a work group of 4
// waves per CU; blocks / 2 work groups, so a launch does the same flops as the other modes).
__global__ __launch_bounds__(256, 1) void probe_attn64_kernel(float* out, int iters) {
  __shared__ __attribute__((aligned(16))) uint16_t tile[2][32 * 128];
  for (int i = threadIdx.x; i < 2 * 32 * 128; i += 256) (&tile[0][0])[i] = (uint16_t)(i * 7);
  __syncthreads();
  typedef short s4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s4 lds_s4;
  const int lane = threadIdx.x & 63;
  f32x16 o[2][4];
  for (int g = 0; g < 2; ++g)
    for (int n = 0; n < 4; ++n) o[g][n] = f32x16{};
  bf16x8 q[2];
  for (int i = 0; i < 8; ++i) {
    q[0][i] = (__bf16)(i * 0.5f);
    q[1][i] = (__bf16)(i * 0.25f);
  }
  float v = 0.f;
  for (int it = 0; it < iters; ++it) {
    int koff = 0;
    asm volatile("" : "+v"(koff));
    f32x16 sc[2] = {f32x16{}, f32x16{}};
    bf16x8 kr[8];
#pragma unroll
    for (int k = 0; k < 8; ++k)
      kr[k] = *reinterpret_cast<const bf16x8*>(&tile[0][koff + (lane & 31) * 128 + 8 * ((2 * k + (lane >> 5)) ^ (lane & 15))]);
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int g = 0; g < 2; ++g) sc[g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kr[k], q[g], sc[g], 0, 0, 0);
    bf16x8 p[2][2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      float mx = sc[g][0];
#pragma unroll
      for (int i = 1; i < 16; ++i) mx = fmaxf(mx, sc[g][i]);
      float e[16], l = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) e[i] = __builtin_amdgcn_exp2f(fmaf(sc[g][i], 1e-3f, -mx));
#pragma unroll
      for (int i = 0; i < 16; ++i) l += e[i];
      v += l;
#pragma unroll
      for (int i = 0; i < 8; ++i) { p[g][0][i] = (__bf16)e[i]; p[g][1][i] = (__bf16)e[8 + i]; }
    }
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const int r = 16 * (n / 4) + 4 * (lane >> 5) + ((lane >> 2) & 3);
      const uint16_t* base = &tile[1][koff + r * 128 + 8 * ((4 * (n % 4) + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1)) ^ (((lane >> 2) & 3) << 2)) + 4 * (lane & 1)];
      const s4 h0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(base));
      const s4 h1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(base + 8 * 128));
      bf16x8 va;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        va[i] = __builtin_bit_cast(__bf16, h0[i]);
        va[4 + i] = __builtin_bit_cast(__bf16, h1[i]);
      }
#pragma unroll
      for (int g = 0; g < 2; ++g)
        o[g][n % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, p[g][n / 4], o[g][n % 4], 0, 0, 0);
    }
  }
  float s = v;
  for (int g = 0; g < 2; ++g)
    for (int n = 0; n < 4; ++n)
      for (int i = 0; i < 16; ++i) s += o[g][n][i];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

// (valu selects the MODE above)
extern "C" int pie_probe_mfma(float* out, int blocks, int iters, int valu, void* stream) {
  if (blocks <= 0 || iters <= 0) return 1;
  switch (valu) {
    case 0: hipLaunchKernelGGL(probe_mfma_kernel<0>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters); break;
    case 1: hipLaunchKernelGGL(probe_mfma_kernel<1>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters); break;
    case 2: hipLaunchKernelGGL(probe_mfma_kernel<2>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters); break;
    case 3: hipLaunchKernelGGL(probe_mfma_kernel<3>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters); break;
    case 4: hipLaunchKernelGGL(probe_mfma_kernel<4>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters); break;
    case 5: hipLaunchKernelGGL(probe_mfma_kernel<5>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters); break;
    case 6: hipLaunchKernelGGL(probe_mfma_kernel<6>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters); break;
    case 7: hipLaunchKernelGGL(probe_mfma_kernel<7>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters); break;
    case 8: hipLaunchKernelGGL(probe_mfma_kernel<8>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters); break;
    case 10: hipLaunchKernelGGL(probe_mfma_kernel<10>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, iters); break;
    case 9: hipLaunchKernelGGL(probe_attn64_kernel, dim3(blocks / 2), dim3(256), 0, (hipStream_t)stream, out, iters); break;
    default: return 1;
  }
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
