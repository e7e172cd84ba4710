// Host emulation of the small HIP subset the kernels in pie_amd/csrc use. TEST INFRASTRUCTURE:
// it lets the unchanged kernel sources run on the CPU (each lane an OS thread, one block at a
// time) so that indexing can be checked under AddressSanitizer with exact-size buffers.
//
// Emulated: thread/block indices, __shared__ (function-local statics: blocks run one after
// another), __syncthreads (block barrier), DPP row_ror / quad_perm, readlane, readfirstlane
// (wave barriers), the fp builtins used, hipLaunchKernelGGL and the few runtime calls made.
#pragma once

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
inline uint4 make_uint4(unsigned a, unsigned b, unsigned c, unsigned d) { return uint4{a, b, c, d}; }
inline float2 make_float2(float a, float b) { return float2{a, b}; }

typedef void* hipStream_t;
typedef int hipError_t;
enum { hipSuccess = 0 };
enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount = 1 };
inline hipError_t hipGetLastError() { return hipSuccess; }
inline const char* hipGetErrorString(hipError_t) { return "emulated"; }
inline hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
inline hipError_t hipDeviceGetAttribute(int* v, hipDeviceAttribute_t, int) {
  const char* e = getenv("EMU_CUS");
  *v = e ? atoi(e) : 1;  // few "CUs" so grid caps engage and grid-stride loops iterate
  return hipSuccess;
}

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(x)
#define __shared__ static

namespace emu {
struct Wave {
  std::barrier<> bar{64};
  uint32_t xchg[64];
  bool live[64] = {};
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
  (void)old;
  const int lane = ctx->lane;
  int from;
  if (ctrl < 0x100) {
    from = (lane & ~3) + ((ctrl >> (2 * (lane & 3))) & 3);
  } else if (ctrl > 0x120 && ctrl < 0x130) {
    const int n = ctrl - 0x120;
    from = (lane & ~15) + (((lane & 15) - n + 16) & 15);
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
        c.bid = dim3(b, 0, 0);
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
#define __builtin_amdgcn_update_dpp emu::update_dpp
#define __builtin_amdgcn_readlane emu::readlane
#define __builtin_amdgcn_readfirstlane emu::readfirstlane
#define __builtin_amdgcn_exp2f exp2f
#define __builtin_amdgcn_rcpf(x) (1.0f / (x))
#define hipLaunchKernelGGL(k, g, b, shm, st, ...) emu::launch(k, dim3(g), dim3(b), __VA_ARGS__)

inline float __uint_as_float(unsigned u) { float f; memcpy(&f, &u, 4); return f; }
inline float rsqrtf(float x) { return 1.0f / sqrtf(x); }
inline unsigned __umulhi(unsigned a, unsigned b) { return (unsigned)(((unsigned long long)a * b) >> 32); }
