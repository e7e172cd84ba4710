// The sampling path after the LM head: Pie's safe_scaled_softmax
// (pie/src/pie_worker/model/common.py:38-59 torch form, :68-188 the Triton kernel it runs on GPUs)
// and flashinfer.sampling's five samplers as Pie calls them (common.py:316-344; API restated in
// pie/src/flashinfer_metal/sampling.py:19-79).
//
// One work group of 1024 threads per row; rows of 32k-256k vocabulary entries are streamed from
// HBM/L2 with 16-byte loads in every pass.
//
// Filters (flashinfer's semantics, exact): top_k keeps token i iff fewer than k tokens are
// strictly more probable (tokens tied with the k-th largest all stay); top_p keeps i iff the mass
// of strictly more probable tokens is below top_p times the row's mass; min_p keeps
// p_i >= min_p * max p; top_k_top_p applies top_p inside the top-k set. Thresholds come from a
// radix select over the fp32 bit patterns (monotone for p >= 0), 8 bits per pass, with token
// counts (top_k) or masses (top_p) per digit. Masses are fixed point (p * 2^40 rounded, summed in
// 64-bit integers), so every sum is exact and independent of thread order: the same row always
// gives the same kept set and the same sample.
// Draw: inverse CDF in index order over the kept tokens, target u * kept mass, with u from
// Philox4x32-10 (counter = (offset, row), key = seed) or caller-given uniforms.
#include <math.h>

#include "common.h"

namespace pie {

constexpr int kSampThreads = 1024;
constexpr int kSampWaves = kSampThreads / 64;
constexpr double kMassScale = 1099511627776.0;  // 2^40

__device__ __forceinline__ uint32_t prob_key(float p) {
  return p > 0.f ? __builtin_bit_cast(uint32_t, p) : 0u;  // NaN and p <= 0 -> 0 (never kept)
}
__device__ __forceinline__ uint64_t prob_mass(float p) {
  return p > 0.f ? (uint64_t)rint((double)p * kMassScale) : 0ull;
}

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3",
// SC 2011): ten rounds of two 32x32->64 multiplies with a Weyl-sequence key schedule.
__device__ __forceinline__ void philox4x32_10(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
  constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)M0 * c[0], p1 = (uint64_t)M1 * c[2];
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    const uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0; c[1] = lo1; c[2] = n2; c[3] = lo0;
    k0 += W0; k1 += W1;
  }
}

// Uniform double in [0, 1) with 53 random bits for (seed, offset, row).
__device__ __forceinline__ double philox_uniform(uint64_t seed, uint64_t offset, uint32_t row) {
  uint32_t c[4] = {(uint32_t)offset, (uint32_t)(offset >> 32), row, 0u};
  philox4x32_10(c, (uint32_t)seed, (uint32_t)(seed >> 32));
  const uint64_t bits = ((uint64_t)c[0] << 21) ^ (uint64_t)(c[1] >> 11);
  return (double)(bits & ((1ull << 53) - 1)) * (1.0 / 9007199254740992.0);
}

__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
  const int lo = __builtin_amdgcn_ds_bpermute(src << 2, (int)(uint32_t)v);
  const int hi = __builtin_amdgcn_ds_bpermute(src << 2, (int)(uint32_t)(v >> 32));
  return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

struct SampleShared {
  uint32_t cnt[256];
  uint64_t mass[256];
  uint64_t wsum[kSampWaves];
  uint64_t u64a, u64b;
  uint32_t u32a, u32b;
  int32_t pick;
};

// Block-wide sum (all threads get the result).
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, SampleShared& sh) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += shfl_u64(v, lane ^ o);
  __syncthreads();
  if (lane == 0) sh.wsum[w] = v;
  __syncthreads();
  uint64_t t = 0;
#pragma unroll
  for (int i = 0; i < kSampWaves; ++i) t += sh.wsum[i];
  return t;
}

__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, SampleShared& sh) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, (uint32_t)__builtin_amdgcn_ds_bpermute((lane ^ o) << 2, (int)v));
  __syncthreads();
  if (lane == 0) sh.wsum[w] = v;
  __syncthreads();
  uint32_t t = 0;
#pragma unroll
  for (int i = 0; i < kSampWaves; ++i) t = max(t, (uint32_t)sh.wsum[i]);
  return t;
}

// Visits every element of the row as (index, value); 16-byte loads where the row allows.
template <typename F>
__device__ __forceinline__ void for_row(const float* p, int V, bool vec, F&& f) {
  if (vec) {
    // four 16-byte loads in flight per thread before any is used
    const int nv = V >> 2;
    int i = threadIdx.x;
    for (; i + 3 * kSampThreads < nv; i += 4 * kSampThreads) {
      float4 x[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) x[k] = *reinterpret_cast<const float4*>(p + 4 * (i + k * kSampThreads));
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int j = 4 * (i + k * kSampThreads);
        f(j, x[k].x); f(j + 1, x[k].y); f(j + 2, x[k].z); f(j + 3, x[k].w);
      }
    }
    for (; i < nv; i += kSampThreads) {
      const float4 x = *reinterpret_cast<const float4*>(p + 4 * i);
      f(4 * i, x.x); f(4 * i + 1, x.y); f(4 * i + 2, x.z); f(4 * i + 3, x.w);
    }
    for (int i = 4 * nv + threadIdx.x; i < V; i += kSampThreads) f(i, p[i]);
  } else {
    for (int i = threadIdx.x; i < V; i += kSampThreads) f(i, p[i]);
  }
}

// Radix search over keys >= lo (8 bits per pass, most significant first). by_mass = false: the
// key of the need-th largest key (top-k threshold). by_mass = true: the smallest key v such that
// the mass of keys strictly above v is below thr (top-p threshold; the maximal key when thr <= 0);
// returns 0 if no key >= lo exists.
__device__ uint32_t radix_threshold(const float* p, int V, bool vec, uint32_t lo, bool by_mass,
                                    uint32_t need, double thr, SampleShared& sh) {
  uint32_t prefix = 0, pmask = 0;
  uint64_t above = 0;  // mass of keys above the current prefix bucket (by_mass)
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += kSampThreads) { sh.cnt[i] = 0; sh.mass[i] = 0; }
    __syncthreads();
    for_row(p, V, vec, [&](int, float x) {
      const uint32_t k = prob_key(x);
      if (k == 0 || k < lo || (k & pmask) != prefix) return;
      const uint32_t d = (k >> shift) & 255u;
      atomicAdd(&sh.cnt[d], 1u);
      if (by_mass) atomicAdd((unsigned long long*)&sh.mass[d], (unsigned long long)prob_mass(x));
    });
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t dsel = 0;
      bool found = false;
      if (!by_mass) {
        uint32_t c = 0;
        for (int d = 255; d >= 0; --d) {
          if (c + sh.cnt[d] >= need && sh.cnt[d] > 0) { dsel = (uint32_t)d; need -= c; found = true; break; }
          c += sh.cnt[d];
        }
      } else {
        uint64_t a = above, a_sel = above;
        int hi = -1;
        for (int d = 255; d >= 0; --d) {
          if (sh.cnt[d] > 0) {
            if (hi < 0) hi = d;
            if ((double)a < thr) { dsel = (uint32_t)d; a_sel = a; found = true; }
            else break;
          }
          a += sh.mass[d];
        }
        if (!found && hi >= 0) { dsel = (uint32_t)hi; a_sel = above; found = true; }  // thr <= 0: the maximum
        above = a_sel;
      }
      sh.u32a = found ? (prefix | (dsel << shift)) : 0xffffffffu;
      sh.u32b = need;
      sh.u64a = above;
    }
    __syncthreads();
    if (sh.u32a == 0xffffffffu) return 0u;
    prefix = sh.u32a;
    need = sh.u32b;
    above = sh.u64a;
    pmask |= 255u << shift;
    __syncthreads();
  }
  return prefix;
}

struct SampleArgs {
  const float* probs;
  int64_t stride;
  int32_t V, B;
  const int32_t* rows;  // optional: output row r samples probs row rows[r] (in [0, nrows))
  int32_t nrows;
  int32_t mode;         // 0 plain, 1 top_p, 2 top_k, 3 min_p, 4 top_k then top_p
  const int32_t* top_k;
  int32_t top_k_s;
  const float* top_p;
  float top_p_s;
  const float* min_p;
  float min_p_s;
  const double* uniforms;  // optional: u per output row
  uint64_t seed, offset;
  int32_t* out;
  int32_t vec;  // rows are 16-byte aligned: 16-byte loads
};

__global__ __launch_bounds__(kSampThreads) void sample_kernel(SampleArgs a) {
  __shared__ SampleShared sh;
  const int r = blockIdx.x;
  const int src = a.rows ? a.rows[r] : r;
  if (src < 0 || src >= a.nrows) {  // a row index outside probs: no draw
    if (threadIdx.x == 0) a.out[r] = -1;
    return;
  }
  const float* p = a.probs + (int64_t)src * a.stride;
  const int V = a.V;
  const bool vec = a.vec != 0;
  // lower bound on kept keys (1 = every p > 0)
  uint32_t lo = 1u;
  if (a.mode == 2 || a.mode == 4) {
    const int32_t k = a.top_k ? a.top_k[r] : a.top_k_s;
    if (k > 0 && k < V) {
      uint32_t npos = 0;
      for_row(p, V, vec, [&](int, float x) { npos += prob_key(x) != 0; });
      npos = (uint32_t)block_sum_u64(npos, sh);
      if ((uint32_t)k < npos) lo = max(1u, radix_threshold(p, V, vec, 1u, false, (uint32_t)k, 0.0, sh));
    }
  }
  if (a.mode == 1 || a.mode == 4) {
    const float tp = a.top_p ? a.top_p[r] : a.top_p_s;
    uint64_t tot = 0;
    for_row(p, V, vec, [&](int, float x) { if (prob_key(x) >= lo) tot += prob_mass(x); });
    tot = block_sum_u64(tot, sh);
    const uint32_t t = radix_threshold(p, V, vec, lo, true, 0u, (double)tp * (double)tot, sh);
    if (t > lo) lo = t;
  }
  double mthr = 0.0;
  if (a.mode == 3) {
    uint32_t mk = 0;
    for_row(p, V, vec, [&](int, float x) { mk = max(mk, prob_key(x)); });
    mk = block_max_u32(mk, sh);
    mthr = (double)(a.min_p ? a.min_p[r] : a.min_p_s) * (double)__builtin_bit_cast(float, mk);
  }
  auto kept_mass = [&](float x) -> uint64_t {
    const uint32_t k = prob_key(x);
    if (k < lo) return 0ull;  // also k == 0
    if (a.mode == 3 && !((double)x >= mthr)) return 0ull;
    return prob_mass(x);
  };
  uint64_t tot = 0;
  int last = -1;
  for_row(p, V, vec, [&](int i, float x) {
    const uint64_t m = kept_mass(x);
    tot += m;
    if (m) last = max(last, i);
  });
  tot = block_sum_u64(tot, sh);
  {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) last = max(last, __builtin_amdgcn_ds_bpermute((lane ^ o) << 2, last));
    __syncthreads();
    if (lane == 0) sh.wsum[threadIdx.x >> 6] = (uint64_t)(int64_t)last;
    __syncthreads();
    for (int i = 0; i < kSampWaves; ++i) last = max(last, (int)(int64_t)sh.wsum[i]);
  }
  const double u = a.uniforms ? a.uniforms[r] : philox_uniform(a.seed, a.offset, (uint32_t)r);
  const double target = u * (double)tot;
  // inverse CDF: tiles of 4 consecutive elements per thread, block-scanned in index order
  if (threadIdx.x == 0) sh.pick = -1;
  __syncthreads();
  uint64_t run = 0;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int base = 0; base < V; base += 4 * kSampThreads) {
    const int i0 = base + 4 * threadIdx.x;
    uint64_t m[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) m[e] = i0 + e < V ? kept_mass(p[i0 + e]) : 0ull;
    const uint64_t mine = m[0] + m[1] + m[2] + m[3];
    // inclusive scan of `mine` over the block
    uint64_t incl = mine;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint64_t y = shfl_u64(incl, lane >= o ? lane - o : lane);
      if (lane >= o) incl += y;
    }
    __syncthreads();
    if (lane == 63) sh.wsum[w] = incl;
    __syncthreads();
    uint64_t before = run, tile = 0;
    for (int i = 0; i < kSampWaves; ++i) {
      if (i < w) before += sh.wsum[i];
      tile += sh.wsum[i];
    }
    const uint64_t excl = before + incl - mine;
    if (mine && (double)(excl + mine) > target && !((double)excl > target)) {
      uint64_t c = excl;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        c += m[e];
        if (m[e] && (double)c > target) { sh.pick = i0 + e; break; }
      }
    }
    __syncthreads();
    if (sh.pick >= 0) break;
    run += tile;
  }
  if (threadIdx.x == 0) a.out[r] = sh.pick >= 0 ? sh.pick : last;
}

// safe_scaled_softmax: probs = softmax(logits / T) per row, or the one-hot of the first maximum
// when T < greedy_threshold. Two passes over the row: (max, first argmax, sum of exp2 relative to
// a running max) with 16-byte loads, then the normalised write; fp32 math in the exp2 domain,
// output in the logits' dtype.
template <bool BF16>
struct RowIO {
  static constexpr int E = BF16 ? 8 : 4;  // elements per 16-byte vector
  __device__ static void load(const void* base, int64_t i, float (&x)[E]) {
    const uint4 v = ld16(reinterpret_cast<const char*>(base) + i * (BF16 ? 2 : 4));
    if (BF16) unpack8(v, x);
    else { x[0] = __uint_as_float(v.x); x[1] = __uint_as_float(v.y); x[2] = __uint_as_float(v.z); x[3] = __uint_as_float(v.w); }
  }
  __device__ static void store(void* base, int64_t i, const float (&x)[E]) {
    uint4 v;
    if (BF16) v = pack8(x);
    else v = make_uint4(__builtin_bit_cast(uint32_t, x[0]), __builtin_bit_cast(uint32_t, x[1]),
                        __builtin_bit_cast(uint32_t, x[2]), __builtin_bit_cast(uint32_t, x[3]));
    st_nt(reinterpret_cast<char*>(base) + i * (BF16 ? 2 : 4), v);
  }
  __device__ static float get(const void* base, int64_t i) {
    return BF16 ? bf1(reinterpret_cast<const uint16_t*>(base)[i]) : reinterpret_cast<const float*>(base)[i];
  }
  __device__ static void put(void* base, int64_t i, float v) {
    if (BF16) reinterpret_cast<uint16_t*>(base)[i] = to_bf1(v);
    else reinterpret_cast<float*>(base)[i] = v;
  }
};

template <bool BF16>
__global__ __launch_bounds__(kSampThreads) void scaled_softmax_kernel(const void* __restrict__ logits,
                                                                      int64_t stride, int V,
                                                                      const float* __restrict__ temps,
                                                                      float greedy, void* __restrict__ out,
                                                                      int64_t out_stride, int vec) {
  using IO = RowIO<BF16>;
  constexpr int E = IO::E;
  __shared__ float sm[kSampWaves], ss[kSampWaves];
  __shared__ int si[kSampWaves];
  const int r = blockIdx.x;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const char* row = reinterpret_cast<const char*>(logits) + (int64_t)r * stride * (BF16 ? 2 : 4);
  char* orow = reinterpret_cast<char*>(out) + (int64_t)r * out_stride * (BF16 ? 2 : 4);
  const float T = temps[r];
  const bool greedy_row = T < greedy;
  const float c = greedy_row ? 1.f : 1.4426950408889634f / T;
  // pass 1: max, first argmax and sum of exp2(x*c - running max) (online rescaling)
  float mx = -INFINITY, s = 0.f;
  int am = 0x7fffffff;
  auto visit = [&](float x, int i) {
    if (x > mx) {
      s = s * __builtin_amdgcn_exp2f((mx - x) * c);  // mx = -inf first: exp2(-inf) = 0
      mx = x;
      am = i;
    }
    s += __builtin_amdgcn_exp2f((x - mx) * c);
  };
  const int nv = vec ? V / E : 0;
  int v = threadIdx.x;
  for (; v + 3 * kSampThreads < nv; v += 4 * kSampThreads) {  // four 16-byte loads in flight
    float x[4][E];
#pragma unroll
    for (int k = 0; k < 4; ++k) IO::load(row, (int64_t)(v + k * kSampThreads) * E, x[k]);
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int e = 0; e < E; ++e) visit(x[k][e], (v + k * kSampThreads) * E + e);
  }
  for (; v < nv; v += kSampThreads) {
    float x[E];
    IO::load(row, (int64_t)v * E, x);
#pragma unroll
    for (int e = 0; e < E; ++e) visit(x[e], v * E + e);
  }
  for (int i = nv * E + threadIdx.x; i < V; i += kSampThreads) visit(IO::get(row, i), i);
  // combine (max, argmax, sum) across the wave, then across waves
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float y = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ o) << 2, __builtin_bit_cast(int, mx)));
    const float ys = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ o) << 2, __builtin_bit_cast(int, s)));
    const int yi = __builtin_amdgcn_ds_bpermute((lane ^ o) << 2, am);
    const float m2 = fmaxf(mx, y);
    const float s2 = (mx == -INFINITY ? 0.f : s * __builtin_amdgcn_exp2f((mx - m2) * c)) +
                     (y == -INFINITY ? 0.f : ys * __builtin_amdgcn_exp2f((y - m2) * c));
    if (y > mx || (y == mx && yi < am)) am = yi;
    mx = m2;
    s = s2;
  }
  if (lane == 0) { sm[w] = mx; ss[w] = s; si[w] = am; }
  __syncthreads();
  float M = -INFINITY;
  int A = 0x7fffffff;
  for (int i = 0; i < kSampWaves; ++i)
    if (sm[i] > M || (sm[i] == M && si[i] < A)) { M = sm[i]; A = si[i]; }
  float S = 0.f;
  for (int i = 0; i < kSampWaves; ++i)
    if (sm[i] != -INFINITY) S += ss[i] * __builtin_amdgcn_exp2f((sm[i] - M) * c);
  // pass 2: write
  const float inv = 1.f / S;
  const float mc = M * c;
  for (int v = threadIdx.x; v < nv; v += kSampThreads) {
    float x[E];
    if (greedy_row) {
#pragma unroll
      for (int e = 0; e < E; ++e) x[e] = (v * E + e) == A ? 1.f : 0.f;
    } else {
      IO::load(row, (int64_t)v * E, x);
#pragma unroll
      for (int e = 0; e < E; ++e) x[e] = __builtin_amdgcn_exp2f(fmaf(x[e], c, -mc)) * inv;
    }
    IO::store(orow, (int64_t)v * E, x);
  }
  for (int i = nv * E + threadIdx.x; i < V; i += kSampThreads)
    IO::put(orow, i, greedy_row ? (i == A ? 1.f : 0.f) : __builtin_amdgcn_exp2f(fmaf(IO::get(row, i), c, -mc)) * inv);
}

}  // namespace pie

using namespace pie;

extern "C" int pie_hip_sample(const float* probs, int64_t prob_stride, int64_t prob_rows, int64_t vocab,
                              int64_t batch, const int32_t* row_indices, int32_t mode, const int32_t* top_k,
                              int32_t top_k_scalar, const float* top_p, float top_p_scalar,
                              const float* min_p, float min_p_scalar, const double* uniforms,
                              uint64_t seed, uint64_t offset, int32_t* out, void* stream) {
  PIE_REQUIRE(probs && out, "sample: null probs or out");
  PIE_REQUIRE(vocab > 0 && vocab < (1ll << 28) && batch >= 0 && batch < (1ll << 31) &&
                  prob_stride >= vocab && prob_rows >= 0 && prob_rows < (1ll << 31) &&
                  (row_indices || prob_rows >= batch),
              "sample: bad vocab %lld / batch %lld / stride %lld", (long long)vocab, (long long)batch,
              (long long)prob_stride);
  PIE_REQUIRE(mode >= 0 && mode <= 4, "sample: bad mode %d", mode);
  if (batch == 0) return PIE_HIP_OK;
  SampleArgs a{probs, prob_stride, (int32_t)vocab, (int32_t)batch, row_indices, (int32_t)prob_rows, mode, top_k,
               top_k_scalar, top_p, top_p_scalar, min_p, min_p_scalar, uniforms, seed, offset, out,
               (prob_stride % 4 == 0 && aligned16(probs)) ? 1 : 0};
  hipLaunchKernelGGL(sample_kernel, dim3((unsigned)batch), dim3(kSampThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("sample");
}

extern "C" int pie_hip_scaled_softmax(const void* logits, int32_t is_bf16, int64_t stride, int64_t batch,
                                      int64_t vocab, const float* temperatures, float greedy_threshold,
                                      void* out, int64_t out_stride, void* stream) {
  PIE_REQUIRE(logits && out && temperatures, "scaled_softmax: null pointer");
  PIE_REQUIRE(vocab > 0 && vocab < (1ll << 31) && batch >= 0 && batch < (1ll << 31) && stride >= vocab &&
                  out_stride >= vocab,
              "scaled_softmax: bad shape");
  if (batch == 0) return PIE_HIP_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t e = is_bf16 ? 8 : 4;  // elements per 16-byte vector
  const int vec = aligned16(logits) && aligned16(out) && stride % e == 0 && out_stride % e == 0;
  if (is_bf16)
    hipLaunchKernelGGL(scaled_softmax_kernel<true>, dim3((unsigned)batch), dim3(kSampThreads), 0, st, logits,
                       stride, (int)vocab, temperatures, greedy_threshold, out, out_stride, vec);
  else
    hipLaunchKernelGGL(scaled_softmax_kernel<false>, dim3((unsigned)batch), dim3(kSampThreads), 0, st, logits,
                       stride, (int)vocab, temperatures, greedy_threshold, out, out_stride, vec);
  return check_launch("scaled_softmax");
}
