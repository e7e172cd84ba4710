// Host emulation of the small HIP subset the kernels in pie_amd/csrc use. TEST INFRASTRUCTURE:
// it lets the unchanged kernel sources run on the CPU (each lane an OS thread, one block at a
// time) so that indexing can be checked under AddressSanitizer with exact-size buffers.
//
// Emulated: thread/block indices, __shared__ (function-local statics: blocks run one after
// another), __syncthreads (block barrier), DPP row_ror / quad_perm, readlane, readfirstlane
// (wave barriers), ballot, ds_bpermute, MFMA 16x16x32 and 32x32x16 bf16, ds_read_b64_tr_b16 (wave-wide
// gathers), global_load_lds (a per-lane copy), the fp builtins used, hipLaunchKernelGGL and the few runtime calls made.
#pragma once

#include <atomic>
#include <barrier>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <thread>
#include <vector>

struct dim3 {
  unsigned x, y, z;
  dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
struct uint2 { unsigned x, y; };
struct uint4 { unsigned x, y, z, w; };
struct float2 { float x, y; };
struct float4 { float x, y, z, w; };
inline uint4 make_uint4(unsigned a, unsigned b, unsigned c, unsigned d) { return uint4{a, b, c, d}; }
inline float2 make_float2(float a, float b) { return float2{a, b}; }
inline float4 make_float4(float a, float b, float c, float d) { return float4{a, b, c, d}; }

#define PIE_HOST_EMULATION 1  // the kernels' compiler-only register fences become identities

typedef void* hipStream_t;
typedef int hipError_t;
enum { hipSuccess = 0 };
enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount = 1 };
inline hipError_t hipGetLastError() { return hipSuccess; }
inline const char* hipGetErrorString(hipError_t) { return "emulated"; }
inline hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
inline hipError_t hipGetSymbolAddress(void** p, const void* sym) { *p = const_cast<void*>(sym); return hipSuccess; }
#define HIP_SYMBOL(x) (&(x))
// streams and events: the emulator runs every launch synchronously, so nothing is ever in flight
typedef void* hipEvent_t;
enum { hipErrorNotReady = 600, hipEventDisableTiming = 2 };
enum hipStreamCaptureStatus { hipStreamCaptureStatusNone = 0, hipStreamCaptureStatusActive = 1 };
inline hipError_t hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus* s) {
  *s = hipStreamCaptureStatusNone;
  return hipSuccess;
}
inline hipError_t hipEventCreateWithFlags(hipEvent_t* e, unsigned) { *e = (hipEvent_t)1; return hipSuccess; }
inline hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
inline hipError_t hipEventQuery(hipEvent_t) { return hipSuccess; }
inline hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t, int) {
  const char* e = getenv("EMU_CUS");
  *v = e ? atoi(e) : 1;  // few "CUs" so grid caps engage and grid-stride loops iterate
  return hipSuccess;
}

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __align__(n) __attribute__((aligned(n)))
#define __shared__ static

namespace emu {
struct Wave {
  std::barrier<> bar{64};
  uint32_t xchg[64];
  bool live[64] = {};
  uint16_t ma[64][8], mb[64][8];  // MFMA operands of every lane
  const void* addr[64];           // LDS addresses of a transpose read
};
struct Ctx {
  dim3 tid, bid, bdim, gdim;
  int lane;
  std::barrier<>* block;
  Wave* wave;
};
inline thread_local Ctx* ctx = nullptr;

inline uint32_t exchange_read(uint32_t v, int src) {
  Wave* w = ctx->wave;
  w->xchg[ctx->lane] = v;
  w->live[ctx->lane] = true;
  w->bar.arrive_and_wait();
  if (!w->live[src]) { fprintf(stderr, "emu: cross-lane read from inactive lane %d\n", src); abort(); }
  uint32_t r = w->xchg[src];
  w->bar.arrive_and_wait();
  w->live[ctx->lane] = false;
  return r;
}

inline int update_dpp(int old, int src, int ctrl, int, int, bool) {
  const int lane = ctx->lane;
  int from;
  if (ctrl < 0x100) {
    from = (lane & ~3) + ((ctrl >> (2 * (lane & 3))) & 3);
  } else if (ctrl > 0x120 && ctrl < 0x130) {  // row_ror:n, lane i reads lane i - n (mod 16)
    const int n = ctrl - 0x120;
    from = (lane & ~15) + (((lane & 15) - n + 16) & 15);
  } else if ((ctrl > 0x100 && ctrl < 0x110) || (ctrl > 0x110 && ctrl < 0x120)) {
    // row_shl:n (lane i reads lane i + n) and row_shr:n (lane i - n) within the row; a lane
    // whose source lies outside its row keeps `old` (bound_ctrl off)
    const int n = ctrl & 15, s = ctrl < 0x110 ? (lane & 15) + n : (lane & 15) - n;
    const uint32_t r = exchange_read((uint32_t)src, s >= 0 && s < 16 ? (lane & ~15) + s : lane);
    return s >= 0 && s < 16 ? (int)r : old;
  } else {
    fprintf(stderr, "emu: unsupported dpp ctrl 0x%x\n", ctrl);
    abort();
  }
  return (int)exchange_read((uint32_t)src, from);
}
inline int readlane(int v, int l) { return (int)exchange_read((uint32_t)v, l); }
inline int readfirstlane(int v) {
  Wave* w = ctx->wave;
  w->xchg[ctx->lane] = (uint32_t)v;
  w->live[ctx->lane] = true;
  w->bar.arrive_and_wait();
  int first = 0;
  while (!w->live[first]) ++first;
  uint32_t r = w->xchg[first];
  w->bar.arrive_and_wait();
  w->live[ctx->lane] = false;
  return (int)r;
}

// __builtin_amdgcn_wave_barrier: on the GPU a compiler-only fence (the lanes of a wave run in
// lockstep); lanes here are threads, so it is a wave barrier.
inline void wave_sync() { ctx->wave->bar.arrive_and_wait(); }

inline uint64_t ballot(bool v) {
  Wave* w = ctx->wave;
  w->xchg[ctx->lane] = v ? 1u : 0u;
  w->bar.arrive_and_wait();
  uint64_t r = 0;
  for (int l = 0; l < 64; ++l) r |= (uint64_t)(w->xchg[l] & 1u) << l;
  w->bar.arrive_and_wait();
  return r;
}

inline int bpermute(int addr, int v) { return (int)exchange_read((uint32_t)v, (addr >> 2) & 63); }

// v_permlane16_swap_b32 / v_permlane32_swap_b32: the odd 16-lane rows (32-lane halves) of `old`
// trade places with the even rows (halves) of `src`; element 0 is the new `old`, 1 the new `src`.
struct Swap2 {
  uint32_t v[2];
  uint32_t operator[](int i) const { return v[i]; }
};
inline Swap2 permlane_swap(uint32_t old, uint32_t src, int span) {
  const bool even = (ctx->lane & span) == 0;
  const uint32_t x = exchange_read(even ? src : old, ctx->lane ^ span);
  return even ? Swap2{{old, x}} : Swap2{{x, src}};
}
inline Swap2 permlane16_swap(uint32_t old, uint32_t src, bool, bool) { return permlane_swap(old, src, 16); }
inline Swap2 permlane32_swap(uint32_t old, uint32_t src, bool, bool) { return permlane_swap(old, src, 32); }


inline float bf16_bits_to_float(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// v_mfma_f32_16x16x32_bf16: lane l supplies A[l%16][8(l/16)+j] and B[8(l/16)+j][l%16] and
// receives C[4(l/16)+i][l%16]; fp32 products of bf16 values are exact, summed in fp32.
template <typename VA, typename VB, typename VC>
VC mfma_16x16x32_bf16(VA a, VB b, VC c, int, int, int) {
  static_assert(sizeof(VA) == 16 && sizeof(VB) == 16 && sizeof(VC) == 16, "operand sizes");
  Wave* w = ctx->wave;
  const int lane = ctx->lane;
  memcpy(w->ma[lane], &a, 16);
  memcpy(w->mb[lane], &b, 16);
  w->bar.arrive_and_wait();
  float cf[4];
  memcpy(cf, &c, 16);
  const int col = lane % 16;
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * (lane / 16) + i;
    float acc = cf[i];
    for (int k = 0; k < 32; ++k)
      acc += bf16_bits_to_float(w->ma[row + 16 * (k / 8)][k % 8]) *
             bf16_bits_to_float(w->mb[col + 16 * (k / 8)][k % 8]);
    cf[i] = acc;
  }
  w->bar.arrive_and_wait();
  VC r;
  memcpy(&r, cf, 16);
  return r;
}

// v_mfma_f32_32x32x16_bf16: lane l supplies A[l%32][8(l/32)+j] and B[8(l/32)+j][l%32] and
// receives C[8(i/4) + 4(l/32) + i%4][l%32] for i = 0..15.
template <typename VA, typename VB, typename VC>
VC mfma_32x32x16_bf16(VA a, VB b, VC c, int, int, int) {
  static_assert(sizeof(VA) == 16 && sizeof(VB) == 16 && sizeof(VC) == 64, "operand sizes");
  Wave* w = ctx->wave;
  const int lane = ctx->lane;
  memcpy(w->ma[lane], &a, 16);
  memcpy(w->mb[lane], &b, 16);
  w->bar.arrive_and_wait();
  float cf[16];
  memcpy(cf, &c, 64);
  const int col = lane % 32;
  for (int i = 0; i < 16; ++i) {
    const int row = 8 * (i / 4) + 4 * (lane / 32) + i % 4;
    float acc = cf[i];
    for (int k = 0; k < 16; ++k)
      acc += bf16_bits_to_float(w->ma[row + 32 * (k / 8)][k % 8]) *
             bf16_bits_to_float(w->mb[col + 32 * (k / 8)][k % 8]);
    cf[i] = acc;
  }
  w->bar.arrive_and_wait();
  VC r;
  memcpy(&r, cf, 64);
  return r;
}

// ds_read_b64_tr_b16: within each 16-lane group, output lane r element j is element r%4 of
// the 8 bytes addressed by lane 4j + r/4 of the group.
template <typename P>
auto ds_read_tr16_b64(P p) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  Wave* w = ctx->wave;
  const int lane = ctx->lane;
  w->addr[lane] = (const void*)p;
  w->bar.arrive_and_wait();
  const int g = lane / 16, r = lane % 16;
  s4 out;
  for (int j = 0; j < 4; ++j) {
    const uint16_t* src = (const uint16_t*)w->addr[16 * g + 4 * j + r / 4];
    out[j] = (short)src[r % 4];
  }
  w->bar.arrive_and_wait();
  return out;
}

// global_load_lds_dwordx4: each lane copies `size` bytes from its own global address to
// lds_base + offset + lane * size.
template <typename G, typename L>
inline void global_load_lds(G src, L lds_base, unsigned size, int offset, int) {
  memcpy((char*)(void*)lds_base + offset + (size_t)ctx->lane * size, (const void*)src, size);
}

template <typename K, typename... A>
void launch(K kernel, dim3 grid, dim3 block, A... args) {
  const unsigned nt = block.x * block.y * block.z;
  if (nt % 64 != 0) { fprintf(stderr, "emu: block size %u not a multiple of 64\n", nt); abort(); }
  for (unsigned b = 0; b < grid.x * grid.y * grid.z; ++b) {
    std::barrier<> bb(nt);
    std::vector<std::unique_ptr<Wave>> waves;
    for (unsigned w = 0; w < nt / 64; ++w) waves.emplace_back(new Wave());
    std::vector<std::thread> ths;
    ths.reserve(nt);
    for (unsigned t = 0; t < nt; ++t) {
      ths.emplace_back([&, t]() {
        Ctx c;
        c.tid = dim3(t, 0, 0);
        c.bid = dim3(b % grid.x, (b / grid.x) % grid.y, b / (grid.x * grid.y));
        c.bdim = block;
        c.gdim = grid;
        c.lane = t & 63;
        c.block = &bb;
        c.wave = waves[t / 64].get();
        ctx = &c;
        kernel(args...);
        bb.arrive_and_drop();
        c.wave->bar.arrive_and_drop();
        ctx = nullptr;
      });
    }
    for (auto& th : ths) th.join();
  }
}
}  // namespace emu

#define threadIdx (emu::ctx->tid)
#define blockIdx (emu::ctx->bid)
#define blockDim (emu::ctx->bdim)
#define gridDim (emu::ctx->gdim)
#define __syncthreads() (emu::ctx->block->arrive_and_wait())
#define __threadfence() std::atomic_thread_fence(std::memory_order_seq_cst)
#define __builtin_amdgcn_update_dpp emu::update_dpp
#define __builtin_amdgcn_readlane emu::readlane
#define __builtin_amdgcn_readfirstlane emu::readfirstlane
#define __builtin_amdgcn_exp2f exp2f
#define __builtin_amdgcn_ballot_w64 emu::ballot
#define __builtin_amdgcn_wave_barrier emu::wave_sync
#define __builtin_amdgcn_ds_bpermute emu::bpermute
#define __builtin_amdgcn_permlane16_swap emu::permlane16_swap
#define __builtin_amdgcn_permlane32_swap emu::permlane32_swap
#define __builtin_amdgcn_mfma_f32_16x16x32_bf16 emu::mfma_16x16x32_bf16
#define __builtin_amdgcn_mfma_f32_32x32x16_bf16 emu::mfma_32x32x16_bf16
#define __builtin_amdgcn_ds_read_tr16_b64_v4i16 emu::ds_read_tr16_b64
#define __builtin_amdgcn_global_load_lds emu::global_load_lds
#define __builtin_amdgcn_s_waitcnt(x) ((void)(x))
#define __builtin_amdgcn_sched_barrier(x) ((void)(x))
#define __builtin_amdgcn_s_getreg(x) ((void)(x), 0u)  // hardware registers (XCC_ID): XCD 0
#define __builtin_amdgcn_sched_group_barrier(m, n, id) ((void)(m), (void)(n), (void)(id))
// Hardware sine / cosine of x revolutions, and the fractional part.
inline float __builtin_amdgcn_sinf(float x) { return (float)sin(6.283185307179586 * (double)x); }
inline float __builtin_amdgcn_cosf(float x) { return (float)cos(6.283185307179586 * (double)x); }
inline float __builtin_amdgcn_fractf(float x) { return x - floorf(x); }
// Buffer resources: the base address only (no range checks; callers stay in bounds).
typedef char* __amdgpu_buffer_rsrc_t;
inline __amdgpu_buffer_rsrc_t __builtin_amdgcn_make_buffer_rsrc(void* p, short, int, int) { return (char*)p; }
typedef unsigned emu_u32x4 __attribute__((ext_vector_type(4)));
inline emu_u32x4 __builtin_amdgcn_raw_buffer_load_b128(__amdgpu_buffer_rsrc_t r, int off, int soff, int) {
  emu_u32x4 v;
  memcpy(&v, r + off + soff, 16);
  return v;
}
inline void __builtin_amdgcn_raw_buffer_store_b128(emu_u32x4 v, __amdgpu_buffer_rsrc_t r, int off, int soff, int) {
  memcpy(r + off + soff, &v, 16);
}
#define __builtin_amdgcn_rcpf(x) (1.0f / (x))
#define hipLaunchKernelGGL(k, g, b, shm, st, ...) emu::launch(k, dim3(g), dim3(b), __VA_ARGS__)

inline float __uint_as_float(unsigned u) { float f; memcpy(&f, &u, 4); return f; }
inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }
inline unsigned max(unsigned a, unsigned b) { return a > b ? a : b; }
inline unsigned min(unsigned a, unsigned b) { return a < b ? a : b; }
inline int64_t min(int64_t a, int64_t b) { return a < b ? a : b; }
// Atomics on block-shared memory (emulated threads of one block run concurrently).
inline unsigned atomicAdd(unsigned* p, unsigned v) { return __atomic_fetch_add(p, v, __ATOMIC_RELAXED); }
inline int atomicMax(int* p, int v) { return __atomic_fetch_max(p, v, __ATOMIC_RELAXED); }
inline int atomicAdd(int* p, int v) { return __atomic_fetch_add(p, v, __ATOMIC_RELAXED); }
inline int atomicExch(int* p, int v) { return __atomic_exchange_n(p, v, __ATOMIC_RELAXED); }
inline int atomicOr(int* p, int v) { return __atomic_fetch_or(p, v, __ATOMIC_RELAXED); }
inline unsigned atomicMax(unsigned* p, unsigned v) { return __atomic_fetch_max(p, v, __ATOMIC_RELAXED); }
inline unsigned atomicMin(unsigned* p, unsigned v) { return __atomic_fetch_min(p, v, __ATOMIC_RELAXED); }
inline unsigned long long atomicAdd(unsigned long long* p, unsigned long long v) {
  return __atomic_fetch_add(p, v, __ATOMIC_RELAXED);
}
inline float rsqrtf(float x) { return 1.0f / sqrtf(x); }
inline unsigned __umulhi(unsigned a, unsigned b) { return (unsigned)(((unsigned long long)a * b) >> 32); }
