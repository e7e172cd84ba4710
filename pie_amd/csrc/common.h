// Shared helpers for the gfx950 per-layer kernels: bf16 packing, wavefront reductions,
// alignment checks, launch-error reporting. Every kernel in this library is HBM-bound
// streaming work: 128-bit global loads/stores, fp32 math, no MFMA.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/pie_hip.h"

namespace pie {

constexpr int kWave = 64;  // CDNA wavefront width

// ---------------------------------------------------------------- error reporting (host)
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
int num_cus();  // compute units of the current device (cached per device)

// Device state that overlapping launches would race on (the allocation-free decode's static
// scratch, a prefill plan's work counters), keyed by its address. inflight_check refuses a
// launch (PIE_HIP_EBUSY) while the last launch that used `key` is still running on another
// stream; launches on the same stream are ordered by it and pass. inflight_mark records the
// launch just made. Launches recorded under stream capture are neither checked nor recorded:
// they run at replay, which the host does not see.
int inflight_check(const void* key, void* stream, const char* what);
void inflight_mark(const void* key, void* stream);

// ---------------------------------------------------------------- grouped launch (host)
// Between pie_hip_group_begin and pie_hip_group_end (group.hip) the groupable entry points
// validate their arguments, then hand them to group_add_* instead of launching; the group's
// end launches them together. The records hold the entry points' own arguments.
struct EmbedRec {
  const int32_t* ids;
  int64_t T;
  const uint16_t* W;
  int64_t V, H, w_rs;
  uint16_t* out;
  int64_t out_rs;
};
struct AddNormRec {
  const uint16_t* x;
  int64_t x_rs;
  const uint16_t* r;
  int64_t r_rs;
  uint16_t* s;
  int64_t s_rs;
  uint16_t* y;
  int64_t y_rs;
  const uint16_t* w;
  int64_t rows, cols;
  float eps;
};
struct ActRec {
  const uint16_t* in;
  int64_t in_rs;
  uint16_t* out;
  int64_t out_rs, rows, I;
  int gelu;  // 0 SiLU, 1 GELU(tanh)
};
struct QkRec {
  const uint16_t* q;
  int64_t q_ts, q_hs;
  const uint16_t* k;
  int64_t k_ts, k_hs;
  const uint16_t* v;
  int64_t v_ts, v_hs;
  uint16_t* q_out;
  int64_t qo_ts, qo_hs;
  uint16_t* k_out;
  int64_t ko_ts, ko_hs;
  const uint16_t* qw;
  const uint16_t* kw;
  float eps;
  const int32_t* pos;
  int64_t T, Hq, Hkv, D;
  const float* inv_freq;  // host array of D/2 values (copied when recorded)
  const int32_t* batch_indices;
  const int32_t* positions;
  const int32_t* kv_indices;
  const int32_t* kv_indptr;
  int64_t batch_size;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t num_pages, page_stride, slot_stride, head_stride, page_size;
};
bool group_is_open();
int group_add_embedding(const EmbedRec& r, void* stream);
int group_add_add_norm(const AddNormRec& r, void* stream);
int group_add_act(const ActRec& r, void* stream);
int group_add_qk(const QkRec& r, void* stream);

#define PIE_REQUIRE(cond, ...)                                 \
  do {                                                         \
    if (!(cond)) return ::pie::set_error(PIE_HIP_EINVAL, __VA_ARGS__); \
  } while (0)

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------- bf16 (device)
// A uint4 carries 8 bf16 values; word i holds elements 2i (low half) and 2i+1 (high half).
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf1(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Round two fp32 values to nearest-even bf16 (v_cvt_pk_bf16_f32 on gfx950) and pack them.
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint16_t to_bf1(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}
// Round an fp32 value to bf16 and return it widened back to fp32.
__device__ __forceinline__ float round_bf(float f) { return bf1(to_bf1(f)); }
// Round a finite fp64 value straight to bf16 (round to nearest even on the 8-bit significand,
// one rounding, no detour through fp32) and return it as fp32. Exact for results in fp32's
// normal range.
__device__ __forceinline__ float round_bf_d(double d) {
  unsigned long long u = __builtin_bit_cast(unsigned long long, d);
  u += ((1ull << 44) - 1) + ((u >> 45) & 1ull);
  return (float)__builtin_bit_cast(double, u & ~((1ull << 45) - 1));
}

__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
  f[0] = bf_lo(v.x); f[1] = bf_hi(v.x); f[2] = bf_lo(v.y); f[3] = bf_hi(v.y);
  f[4] = bf_lo(v.z); f[5] = bf_hi(v.z); f[6] = bf_lo(v.w); f[7] = bf_hi(v.w);
}
__device__ __forceinline__ uint4 pack8(const float* f) {
  uint4 v;
  v.x = pack_bf2(f[0], f[1]); v.y = pack_bf2(f[2], f[3]);
  v.z = pack_bf2(f[4], f[5]); v.w = pack_bf2(f[6], f[7]);
  return v;
}

// 128-bit accesses. ld_nt/st_nt take the non-temporal path (streamed data that must not
// evict reused lines); ld16/st16 the ordinary cached path. Each kernel picks per access what
// measured fastest on MI355X in steady state (back-to-back launches over buffers larger than
// the last-level cache, so a kernel pays for draining its own writes): non-temporal stores for
// every large streamed output (e.g. SiLU-and-mul 6.47 vs 6.13 TB/s, embedding 6.27 vs
// 5.23 TB/s), non-temporal loads and stores for large RMSNorm row lists (row_ld / row_st below).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_nt(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt(void* p, const uint4& v) {
  const u32x4_t w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(p));
}
__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void st16(void* p, const uint4& v) { *reinterpret_cast<uint4*>(p) = v; }
// 16-byte vector i of a row whose base address is the same in every lane of the wave, through a
// buffer resource: with NT the access carries the non-temporal cache policy as an operand of the
// instruction, where compiler passes cannot drop it (LLVM's loop-invariant code motion drops the
// !nontemporal metadata of plain stores in some loop shapes).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* row_base) {
  const uint64_t a = reinterpret_cast<uint64_t>(row_base);  // the same in every lane: say so
  const uint64_t u = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(a >> 32)) << 32) |
                     (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(u), 0, 0x7fffffff, 0x00020000);
}
template <bool NT>
__device__ __forceinline__ uint4 row_ld(const void* row_base, int i) {
  if constexpr (NT) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(row_rsrc(row_base), i * 16, 0, 2);
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return ld16(reinterpret_cast<const char*>(row_base) + (int64_t)i * 16);
  }
}
template <bool NT>
__device__ __forceinline__ void row_st(void* row_base, int i, const uint4& v) {
  if constexpr (NT) {
    const u32x4_t w = {v.x, v.y, v.z, v.w};
    __builtin_amdgcn_raw_buffer_store_b128(w, row_rsrc(row_base), i * 16, 0, 2);
  } else {
    st16(reinterpret_cast<char*>(row_base) + (int64_t)i * 16, v);
  }
}

// ---------------------------------------------------------------- reductions (device)
// Sum over each 16-lane DPP row, result broadcast to all 16 lanes (row_ror 8,4,2,1).
__device__ __forceinline__ float row16_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x122, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x121, 0xF, 0xF, false));
  return v;
}
// fp64 form: each step moves both 32-bit halves with the same DPP rotation.
template <int CTRL>
__device__ __forceinline__ double dpp_ror_d(double v) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)u, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(u >> 32), CTRL, 0xF, 0xF, false);
  return __builtin_bit_cast(double, ((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}
__device__ __forceinline__ double row16_sum(double v) {
  v += dpp_ror_d<0x128>(v);
  v += dpp_ror_d<0x124>(v);
  v += dpp_ror_d<0x122>(v);
  v += dpp_ror_d<0x121>(v);
  return v;
}
__device__ __forceinline__ double readlane_d(double v, int l) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = __builtin_amdgcn_readlane((int)(unsigned)u, l);
  const unsigned hi = __builtin_amdgcn_readlane((int)(unsigned)(u >> 32), l);
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ double wave_sum(double v) {
  v = row16_sum(v);
  return readlane_d(v, 0) + readlane_d(v, 16) + readlane_d(v, 32) + readlane_d(v, 48);
}
// Full-wavefront sum, uniform result (scalar register).
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  const int b = __builtin_bit_cast(int, v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Compiler-only fences on values (no instruction is emitted). keep_s: x is materialised in
// scalar registers here, so the loads it comes from are waited for at this point and not later.
// opaque_v: x passes through a vector register the compiler cannot see into, so what is computed
// from it cannot be hoisted above this point. The tests' CPU emulator of these kernels (which
// defines PIE_HOST_EMULATION) has no registers to name and gives the identity.
#ifdef PIE_HOST_EMULATION
__device__ __forceinline__ void keep_s(uint32_t) {}
__device__ __forceinline__ int opaque_v(int x) { return x; }
#else
__device__ __forceinline__ void keep_s(uint32_t x) { asm volatile("" ::"s"(x)); }
__device__ __forceinline__ int opaque_v(int x) {
  asm volatile("" : "+v"(x));
  return x;
}
#endif

// Kernel arguments sit in memory that the scalar cache fetches on first use, one 64-byte line at
// a time, and the compiler loads each field where it is first needed, often behind a branch that
// waits for an earlier field: for a large argument block that is a chain of cache-miss round
// trips before the first load of real data. Touching one dword of every line of the block at
// kernel entry requests all of its lines at once (one round trip); later field loads hit.
// Bytes: the leading part of the block that scalar loads read (large arrays read by vector loads
// go last in the argument structs and are left out).
template <int Bytes, typename T>
__device__ __forceinline__ void prefetch_kernarg(const T& args) {
  static_assert(Bytes > 0 && Bytes <= (int)sizeof(T), "prefetch within the argument block");
  constexpr int kLines = (Bytes + 63) / 64;
  const uint32_t* p = reinterpret_cast<const uint32_t*>(&args);
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < kLines; ++i) x ^= p[16 * i];
  keep_s(x);
}

// Unsigned 32-bit division by a runtime-constant divisor with a host-computed multiplier
// (round-up method: q = (mulhi(n, m) + n) >> l with l = ceil(log2 d),
// m = floor(2^32 (2^l - d) / d) + 1); exact for every 32-bit n.
struct FastDiv {
  uint32_t d, m, l;
  static FastDiv make(uint32_t d) {
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    const uint64_t m = ((((1ull << l) - d) << 32) / d) + 1;
    return FastDiv{d, (uint32_t)m, l};
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    return (uint32_t)(((uint64_t)__umulhi(n, m) + n) >> l);
  }
};

}  // namespace pie
