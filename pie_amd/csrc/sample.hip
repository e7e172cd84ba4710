// The sampling path after the LM head: Pie's safe_scaled_softmax
// (pie/src/pie_worker/model/common.py:38-59 torch form, :68-188 the Triton kernel it runs on GPUs)
// and flashinfer.sampling's five samplers as Pie calls them (common.py:316-344; API restated in
// pie/src/flashinfer_metal/sampling.py:19-79).
//
// One work group of 1024 threads per row; rows of 32k-256k vocabulary entries are streamed from
// HBM/L2 with 16-byte loads.
//
// Filters (flashinfer's semantics, exact): top_k keeps token i iff fewer than k tokens are
// strictly more probable (tokens tied with the k-th largest all stay); top_p keeps i iff the mass
// of strictly more probable tokens is below top_p times the row's mass; min_p keeps
// p_i >= min_p * max p; top_k_top_p applies top_p inside the top-k set. Thresholds come from a
// radix select over the fp32 bit patterns (monotone for p >= 0), 8 bits per pass, with token
// counts (top_k) or masses (top_p) per digit. Masses are fixed point (p * 2^40 rounded, summed in
// 64-bit integers), so every sum is exact and independent of thread order: the same row always
// gives the same kept set and the same sample.
// Two row reads in the common case: pass A finds a floor under the threshold (from each thread's
// two largest keys, or the row maximum for min_p), pass B copies the elements above it into LDS
// in vocabulary order, and the radix selects and the draw run over that short list. top_k with a
// small k over a long row needs one read: the k-th largest of the row's first 8192 entries is
// already a floor, so the list is built in the same pass that counts the row's p > 0. Plain
// sampling, and rows whose list would not fit, take the direct passes over the row. top_p runs
// in its own kernel instantiation: a histogram pass (mass per eighth of a binade of the key)
// finds the bin holding the threshold, one gather collects every key from that bin up (or, for
// large kept sets, the bin's keys alone), and a radix search inside the bin gives the threshold.
// Draw: inverse CDF in index order over the kept tokens, target u * kept mass, with u from
// Philox4x32-10 (counter = (offset, row), key = seed) or caller-given uniforms; the kept-mass
// pass sums chunks of the row so that only the chunk holding the target is scanned.
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

// v of lane - n within the lane's 16-lane row (0 for the row's first n lanes): DPP row_shr:n.
template <int N>
__device__ __forceinline__ uint64_t row_shr_u64(uint64_t v) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, 0x110 + N, 0xf, 0xf, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), 0x110 + N, 0xf, 0xf, false);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
  return ((uint64_t)hi << 32) | lo;
}
// Inclusive scan over the wave's 64 lanes (all active): within 16-lane rows by DPP shifts, then
// the totals of the rows before each row.
__device__ __forceinline__ uint64_t row_incl_scan_u64(uint64_t v) {
  v += row_shr_u64<1>(v);
  v += row_shr_u64<2>(v);
  v += row_shr_u64<4>(v);
  v += row_shr_u64<8>(v);
  return v;
}
__device__ __forceinline__ uint64_t wave_incl_scan_u64(uint64_t v) {
  v = row_incl_scan_u64(v);
  const uint64_t r0 = readlane_u64(v, 15), r1 = readlane_u64(v, 31), r2 = readlane_u64(v, 47);
  const int row = (threadIdx.x & 63) >> 4;
  return v + (row > 0 ? r0 : 0ull) + (row > 1 ? r1 : 0ull) + (row > 2 ? r2 : 0ull);
}
// The wave's total (all lanes active), the same in every lane.
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
  v = row_incl_scan_u64(v);
  return readlane_u64(v, 15) + readlane_u64(v, 31) + readlane_u64(v, 47) + readlane_u64(v, 63);
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
  v = wave_sum_u64(v);
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

// Visits every element of the row as (index, value); 16-byte loads where the row allows. The row
// goes in batches of kRowU vectors per thread, two batches in flight: the next batch's loads are
// issued before the current one is used (two register buffers in turn, no copies, which would
// wait for the younger loads), so a thread keeps 2 kRowU 16-byte loads outstanding.
constexpr int kRowU = 2;  // 2 measured faster than 4 (more registers, slower passes)
template <typename F>
__device__ __forceinline__ void for_row(const float* p, int V, bool vec, F&& f) {
  if (vec) {
    const int nv = V >> 2;
    constexpr int S = kRowU * kSampThreads;  // vectors per batch
    const int nb = nv / S;                   // full batches (no bounds tests)
    auto load = [&](float4 (&d)[kRowU], int at) {
#pragma unroll
      for (int k = 0; k < kRowU; ++k) d[k] = *reinterpret_cast<const float4*>(p + 4 * (at + threadIdx.x + k * kSampThreads));
    };
    auto use = [&](const float4 (&d)[kRowU], int at) {
#pragma unroll
      for (int k = 0; k < kRowU; ++k) {
        const int j = 4 * (at + threadIdx.x + k * kSampThreads);
        f(j, d[k].x); f(j + 1, d[k].y); f(j + 2, d[k].z); f(j + 3, d[k].w);
      }
    };
    if (nb > 0) {
      float4 x[kRowU], y[kRowU];
      load(x, 0);
      if (nb > 1) load(y, S);
      for (int bi = 0;;) {
        use(x, bi * S);
        if (bi + 2 < nb) load(x, (bi + 2) * S);
        if (++bi >= nb) break;
        use(y, bi * S);
        if (bi + 2 < nb) load(y, (bi + 2) * S);
        if (++bi >= nb) break;
      }
    }
    // the last partial batch: every load issued before any is used
    {
      const int at = nb * S;
      float4 d[kRowU];
#pragma unroll
      for (int k = 0; k < kRowU; ++k) {
        const int v = min(at + (int)threadIdx.x + k * kSampThreads, nv - 1);
        if (nv > 0) d[k] = *reinterpret_cast<const float4*>(p + 4 * v);
      }
#pragma unroll
      for (int k = 0; k < kRowU; ++k) {
        const int v = at + threadIdx.x + k * kSampThreads;
        if (v < nv) { f(4 * v, d[k].x); f(4 * v + 1, d[k].y); f(4 * v + 2, d[k].z); f(4 * v + 3, d[k].w); }
      }
    }
    for (int i = 4 * nv + threadIdx.x; i < V; i += kSampThreads) f(i, p[i]);
  } else {
    for (int i = threadIdx.x; i < V; i += kSampThreads) f(i, p[i]);
  }
}

// Radix search over keys >= lo (8 bits per pass, most significant first). by_mass = false: the
// key of the need-th largest key (top-k threshold; 0 if fewer than need keys >= lo exist).
// by_mass = true: the smallest key v such that the mass of keys strictly above v is below thr
// (top-p threshold; the maximal key when thr <= 0); 0 if no key >= lo exists. Each pass counts
// the digits of the keys under the current prefix; wave 0 then scans the 256 digits from the top
// (4 per lane) to pick the next one. prefix0 / pmask0 / shift0: the search starts inside the
// bucket of keys k with (k & pmask0) == prefix0 (every key the caller passes lies in it), at the
// 8-bit digit that starts at bit shift0; the last digit (shift 0) may overlap bits already fixed.
__device__ __forceinline__ uint32_t radix_threshold(const float* p, int V, bool vec, uint32_t lo, bool by_mass,
                                    uint32_t need, double thr, SampleShared& sh, uint32_t prefix0 = 0u,
                                    uint32_t pmask0 = 0u, int shift0 = 24) {
  uint32_t prefix = prefix0, pmask = pmask0;
  uint64_t above = 0;  // mass of keys above the current prefix bucket (by_mass)
  for (int shift = shift0;; shift = shift > 8 ? shift - 8 : 0) {
    for (int i = threadIdx.x; i < 256; i += kSampThreads) { sh.cnt[i] = 0; sh.mass[i] = 0; }
    if (threadIdx.x == 0) sh.u32a = 0xffffffffu;
    __syncthreads();
    for_row(p, V, vec, [&](int, float x) {
      const uint32_t k = prob_key(x);
      if (k == 0 || k < lo || (k & pmask) != prefix) return;
      const uint32_t d = (k >> shift) & 255u;
      atomicAdd(&sh.cnt[d], 1u);
      if (by_mass) atomicAdd((unsigned long long*)&sh.mass[d], (unsigned long long)prob_mass(x));
    });
    __syncthreads();
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      uint32_t c[4];
      uint64_t m[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {  // this lane's digits, descending: 255 - 4 lane - e
        c[e] = sh.cnt[255 - 4 * lane - e];
        m[e] = by_mass ? sh.mass[255 - 4 * lane - e] : 0ull;
      }
      const uint32_t lc = c[0] + c[1] + c[2] + c[3];
      const uint64_t lm = m[0] + m[1] + m[2] + m[3];
      const uint32_t ic = (uint32_t)wave_incl_scan_u64(lc);
      const uint64_t im = by_mass ? wave_incl_scan_u64(lm) : 0ull;
      uint32_t cc = ic - lc;          // keys in the digits above this lane's first
      uint64_t ma = above + im - lm;  // their mass plus the mass above the prefix
      if (!by_mass) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (c[e] && cc < need && cc + c[e] >= need) {  // exactly one digit qualifies
            sh.u32a = prefix | ((uint32_t)(255 - 4 * lane - e) << shift);
            sh.u32b = need - cc;
          }
          cc += c[e];
        }
      } else {
        // the lowest non-empty digit whose mass above is below thr (masses above only grow
        // downwards, so the qualifying digits run from the top); the highest non-empty digit
        // when none qualifies
        int low = 256, high = -1;
        uint64_t a = ma;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d = 255 - 4 * lane - e;
          if (c[e]) {
            if ((double)a < thr) low = d;
            high = max(high, d);
          }
          a += m[e];
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
          low = min(low, __builtin_amdgcn_ds_bpermute((lane ^ o) << 2, low));
          high = max(high, __builtin_amdgcn_ds_bpermute((lane ^ o) << 2, high));
        }
        const int dsel = low < 256 ? low : high;
        if (dsel >= 0 && (255 - dsel) / 4 == lane) {  // the owner of dsel records the mass above it
          const int ei = (255 - dsel) % 4;
          uint64_t a2 = ma;
#pragma unroll
          for (int e = 0; e < 4; ++e) a2 += e < ei ? m[e] : 0ull;
          sh.u32a = prefix | ((uint32_t)dsel << shift);
          sh.u64a = low < 256 ? a2 : above;
        }
      }
    }
    __syncthreads();
    if (sh.u32a == 0xffffffffu) return 0u;
    prefix = sh.u32a;
    if (!by_mass) need = sh.u32b;
    if (by_mass) above = sh.u64a;
    pmask |= 255u << shift;
    __syncthreads();
    if (shift == 0) break;
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

// A row's sampling parameters, read once at the kernel's start (their loads then overlap the
// row's passes): top_k, top_p, min_p and the draw's uniform u.
struct RowParams {
  int32_t k;
  float tp, mp;
  double u;
};
__device__ __forceinline__ RowParams row_params(const SampleArgs& a, int r) {
  RowParams q;
  q.k = a.top_k ? a.top_k[r] : a.top_k_s;
  q.tp = a.top_p ? a.top_p[r] : a.top_p_s;
  q.mp = a.min_p ? a.min_p[r] : a.min_p_s;
  q.u = a.uniforms ? a.uniforms[r] : philox_uniform(a.seed, a.offset, (uint32_t)r);
  return q;
}

// min and max of v and the v of lane ^ j (j < 64), in registers: DPP within 16-lane rows
// (quad_perm for j = 1, 2; row_shl:4 / row_shr:4 for j = 4; row_ror:8 for j = 8), and across
// rows v_permlane16_swap / v_permlane32_swap, which leave {v, partner} in their two results.
__device__ __forceinline__ void lane_pair(uint32_t v, int j, uint32_t& lo, uint32_t& hi) {
  uint32_t a = v, b;
  if (j == 1) {
    b = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
  } else if (j == 2) {
    b = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
  } else if (j == 4) {
    const uint32_t up = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x104, 0xf, 0xf, false);  // lane + 4
    const uint32_t dn = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, false);  // lane - 4
    b = (threadIdx.x & 4) ? dn : up;
  } else if (j == 8) {
    b = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, false);  // row_ror:8
  } else if (j == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    a = r[0];
    b = r[1];
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    a = r[0];
    b = r[1];
  }
  lo = min(a, b);
  hi = max(a, b);
}

// Short candidate lists (at most kSampThreads elements, in LDS): the top_k / top_p thresholds from
// a bitonic sort of the keys (one per thread; compare-exchange partners within a wave in registers
// by lane_pair, across waves through LDS), a block scan of the sorted masses, and one thread
// that sees the cut. Radix passes over such lists serialise on LDS atomics: the keys of a row's
// largest probabilities share their top bits, so every count lands in one or two bins. Same
// kept sets as the radix selects: top_k keeps keys >= the k-th largest (ties stay), top_p keeps
// keys >= the smallest key whose strictly larger keys' mass is below top_p * mass (the maximal
// key when that product is <= 0).
// S (a power of two, 64..kSampThreads) keys, held by threads [0, S); every thread of the block
// calls it (the cross-wave steps are block barriers), the others idle.
template <int S = kSampThreads>
__device__ __forceinline__ uint32_t sort_desc_keys(uint32_t v, uint32_t* buf) {
  const int t = threadIdx.x;
  const bool act = t < S;  // wave-uniform
#pragma unroll
  for (int k = 2; k <= S; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const bool desc = (t & k) == 0;     // this k-block sorts descending (the whole array at the end)
      const bool first = (t & j) == 0;  // the lower position of the pair
      if (j >= 64) {
        __syncthreads();
        if (act) buf[t] = v;
        __syncthreads();
        if (act) {
          const uint32_t pv = buf[t ^ j];
          v = (first == desc) ? max(v, pv) : min(v, pv);
        }
      } else if (act) {
        uint32_t lo, hi;
        lane_pair(v, j, lo, hi);
        v = (first == desc) ? hi : lo;
      }
    }
  }
  return v;
}

// Returns lo for the list p[0, n) (n <= kSampThreads): the smallest kept key under the row's
// top_k / top_p (modes 1, 2, 4), as sample_row's radix selects would give it.
__device__ __forceinline__ uint32_t list_threshold(const float* p, int n, const SampleArgs& a, const RowParams& rp, int64_t npos,
                                   uint64_t row_tot, SampleShared& sh, uint32_t* buf) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  uint32_t v = t < n ? prob_key(p[t]) : 0u;
  // position t now holds the (t+1)-th largest key (the sort spans the smallest power of two
  // holding the list; the positions past it hold zero keys, as before)
  v = n <= 256 ? sort_desc_keys<256>(v, buf) : n <= 512 ? sort_desc_keys<512>(v, buf) : sort_desc_keys(v, buf);
  const uint64_t m = v ? prob_mass(__builtin_bit_cast(float, v)) : 0ull;
  // inclusive block scan of the masses in sorted order
  uint64_t incl = wave_incl_scan_u64(m);
  __syncthreads();
  if (lane == 63) sh.wsum[w] = incl;
  buf[t] = v;
  if (t == 0) { sh.u32a = 0u; sh.u32b = (uint32_t)n; sh.u64a = 0; }
  __syncthreads();
  for (int i = 0; i < w; ++i) incl += sh.wsum[i];
  const uint64_t excl = incl - m;
  uint32_t lo = 1u;
  int lim = n;  // positions [0, lim) hold the keys >= lo
  if (a.mode == 2 || a.mode == 4) {
    const int32_t k = rp.k;
    int64_t np = npos;
    if (np < 0) {  // the list's count of p > 0 (sorted: the first zero key's position)
      if (t == 0) sh.pick = 0;
      __syncthreads();
      if (v != 0u && (t + 1 == kSampThreads || buf[t + 1] == 0u)) sh.pick = t + 1;
      __syncthreads();
      np = sh.pick;
    }
    if (k > 0 && k < n && (int64_t)k < np) {
      lo = max(1u, buf[k - 1]);
      // the top-k set: every position whose key is >= the k-th largest
      if (v >= lo && (t + 1 == n || buf[t + 1] < lo)) { sh.u32b = (uint32_t)(t + 1); sh.u64a = incl; }
      __syncthreads();
      lim = (int)sh.u32b;
    } else {
      __syncthreads();
    }
  }
  if (a.mode == 1 || a.mode == 4) {
    const float tp = rp.tp;
    uint64_t tot;
    if (a.mode == 1 && row_tot) {
      tot = row_tot;
    } else if (lim < n) {
      tot = sh.u64a;
    } else {  // every key >= lo: the list's mass
      __syncthreads();
      if (t == kSampThreads - 1) sh.u64a = incl;
      __syncthreads();
      tot = sh.u64a;
    }
    const double thr = (double)tp * (double)tot;
    // the last position whose strictly-before mass is below thr (ties before it share its key)
    if (t < lim && v != 0u && (double)excl < thr && (t + 1 == lim || !((double)incl < thr))) sh.u32a = v;
    __syncthreads();
    uint32_t tkey = sh.u32a;
    if (tkey == 0u && lim > 0 && buf[0] != 0u) tkey = buf[0];  // thr <= 0: the maximal key
    if (tkey > lo) lo = tkey;
  }
  __syncthreads();  // buf is reused by the caller
  return lo;
}

// Draw for output row r from the values p[0, V): thresholds by radix select, then the inverse CDF
// in order. idx (optional) maps a position in p to the vocabulary index (p is then the row's
// candidate list, ascending in vocabulary index). npos: the row's count of p > 0 (-1: count it
// here over p). row_tot: the row's total mass for top_p (0: sum it here over p). Candidate lists
// hold every element at or above the threshold being searched, so the counts and masses that
// decide it are the same as over the whole row. lo_given > 0: the kept keys' lower bound is
// already known (top_p resolved from the row's histogram): no threshold search here.
__device__ __forceinline__ void sample_row(const float* p, const uint32_t* idx, int V, bool vec,
                                           const SampleArgs& a, int r, const RowParams& rp, int64_t npos,
                                           uint64_t row_tot, SampleShared& sh, uint32_t* list_buf = nullptr,
                                           uint32_t lo_given = 0u) {
  if (V == 0) {  // nothing to draw from (an empty candidate list)
    if (threadIdx.x == 0) a.out[r] = -1;
    return;
  }

  // lower bound on kept keys (1 = every p > 0)
  uint32_t lo = lo_given ? lo_given : 1u;
  const bool given = lo_given != 0u;
  const bool short_list = !given && list_buf && idx && V <= kSampThreads && a.mode != 3;
  if (given) {
  } else if (short_list) {
    lo = list_threshold(p, V, a, rp, npos, row_tot, sh, list_buf);
  } else if (a.mode == 2 || a.mode == 4) {
    const int32_t k = rp.k;
    if (k > 0 && k < V) {
      if (npos < 0) {
        uint32_t c = 0;
        for_row(p, V, vec, [&](int, float x) { c += prob_key(x) != 0; });
        npos = (int64_t)block_sum_u64(c, sh);
      }
      if ((int64_t)k < npos) lo = max(1u, radix_threshold(p, V, vec, 1u, false, (uint32_t)k, 0.0, sh));
    }
  }
  if (!given && !short_list && (a.mode == 1 || a.mode == 4)) {
    const float tp = rp.tp;
    uint64_t tot = 0;
    if (a.mode == 1 && row_tot) {
      tot = row_tot;
    } else {
      for_row(p, V, vec, [&](int, float x) { if (prob_key(x) >= lo) tot += prob_mass(x); });
      tot = block_sum_u64(tot, sh);
    }
    const uint32_t t = radix_threshold(p, V, vec, lo, true, 0u, (double)tp * (double)tot, sh);
    if (t > lo) lo = t;
  }
  double mthr = 0.0;
  if (a.mode == 3) {
    uint32_t mk = 0;
    for_row(p, V, vec, [&](int, float x) { mk = max(mk, prob_key(x)); });
    mk = block_max_u32(mk, sh);
    mthr = (double)rp.mp * (double)__builtin_bit_cast(float, mk);
  }
  auto kept_mass = [&](float x) -> uint64_t {
    const uint32_t k = prob_key(x);
    if (k < lo) return 0ull;  // also k == 0
    if (a.mode == 3 && !((double)x >= mthr)) return 0ull;
    return prob_mass(x);
  };
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (idx && V <= kSampThreads) {
    // a candidate list of at most one element per thread: one block scan of the kept masses in
    // list (= vocabulary) order; the draw is the first element whose inclusive mass exceeds
    // u * total (the same element the chunked search below finds)
    const int t = threadIdx.x;
    const uint64_t m = t < V ? kept_mass(p[t]) : 0ull;
    uint64_t incl = wave_incl_scan_u64(m);
    const uint64_t mb = __builtin_amdgcn_ballot_w64(m != 0ull);  // the wave's last kept element
    int last = mb ? (t & ~63) + 63 - __builtin_clzll(mb) : -1;
    __syncthreads();
    if (lane == 63) sh.wsum[w] = incl;
    if (lane == 0) sh.cnt[w] = (uint32_t)(last + 1);
    if (t == 0) sh.pick = -1;
    __syncthreads();
    uint64_t tot = 0, before = 0;
    for (int i = 0; i < kSampWaves; ++i) {
      if (i < w) before += sh.wsum[i];
      tot += sh.wsum[i];
      last = max(last, (int)sh.cnt[i] - 1);
    }
    const double target = rp.u * (double)tot;
    incl += before;
    const uint64_t excl = incl - m;
    if (m && (double)incl > target && !((double)excl > target)) sh.pick = t;
    __syncthreads();
    if (t == 0) {
      const int j = sh.pick >= 0 ? sh.pick : last;
      a.out[r] = j >= 0 ? (int32_t)idx[j] : j;
    }
    return;
  }
  // kept-mass pass: the sums of chunks of whole 4096-element tiles (at most 256 chunks), so that
  // the inverse CDF scans only the chunk where the target falls
  constexpr int kTile = 4 * kSampThreads;
  const int ntiles = (V + kTile - 1) / kTile;
  const int tpc = (ntiles + 255) / 256;  // tiles per chunk
  for (int i = threadIdx.x; i < 256; i += kSampThreads) sh.mass[i] = 0;
  __syncthreads();
  auto load4 = [&](int i0, float (&x)[4]) {
    if (vec && i0 + 3 < V) {
      const float4 v = *reinterpret_cast<const float4*>(p + i0);
      x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = i0 + e < V ? p[i0 + e] : 0.f;
    }
  };
  // The pass sums each lane's kept masses in fp64: the terms are integers below 2^41 (p <= 2)
  // and a lane sums at most 64 of them per tile, so every partial sum is exact (below 2^53) and
  // converts to the same integer the fixed-point sum gives, at half the per-element cost.
  double acc = 0.0;
  auto visit = [&](int, float x) {
    const uint32_t k = prob_key(x);
    const bool keep = k >= lo && (a.mode != 3 || (double)x >= mthr);  // lo >= 1: k == 0 never kept
    acc += keep ? rint((double)x * kMassScale) : 0.0;
  };
  auto chunk_done = [&](int t) {  // this wave's share of tile t is in acc
    const uint64_t m = wave_sum_u64((uint64_t)acc);
    if (lane == 0 && m) atomicAdd((unsigned long long*)&sh.mass[t / tpc], (unsigned long long)m);
    acc = 0.0;
  };
  if (vec) {
    // Wave w takes whole tiles w, w + 16, ...: a tile is 1024 16-byte vectors, 16 per lane, read
    // as four quarters of 4 loads with the next quarter's loads issued before the current quarter
    // is used, and its mass is reduced once per wave and tile.
    const int nv = V >> 2;
    constexpr int kQuarter = kTile / 16;  // vectors per quarter tile
    // (loads past the last vector re-read it, unused: every load is issued unconditionally)
    const int nh = w < ntiles && nv > 0 ? 4 * ((ntiles - w + kSampWaves - 1) / kSampWaves) : 0;
    auto hbase = [&](int h) { return (w + kSampWaves * (h >> 2)) * (kTile / 4) + (h & 3) * kQuarter; };
    auto load = [&](float4 (&d)[4], int h) {
      const int v0 = hbase(h) + lane;
#pragma unroll
      for (int k = 0; k < 4; ++k) d[k] = *reinterpret_cast<const float4*>(p + 4 * min(v0 + 64 * k, nv - 1));
    };
    auto use = [&](const float4 (&d)[4], int h) {
      const int v0 = hbase(h) + lane;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int v = v0 + 64 * k;
        if (v < nv) { visit(4 * v, d[k].x); visit(4 * v + 1, d[k].y); visit(4 * v + 2, d[k].z); visit(4 * v + 3, d[k].w); }
      }
      if ((h & 3) == 3) chunk_done(w + kSampWaves * (h >> 2));
    };
    if (nh > 0) {
      float4 x[4], y[4];
      load(x, 0);
      load(y, 1);
      for (int h = 0;;) {
        use(x, h);
        if (h + 2 < nh) load(x, h + 2);
        if (++h >= nh) break;
        use(y, h);
        if (h + 2 < nh) load(y, h + 2);
        if (++h >= nh) break;
      }
    }
    if (4 * nv < V && w == (ntiles - 1) % kSampWaves) {  // the last < 4 elements, in the last tile
      if (lane < V - 4 * nv) visit(4 * nv + lane, p[4 * nv + lane]);
      chunk_done(ntiles - 1);
    }
  } else {
    for (int t = 0; t < ntiles; ++t) {
      for (int e = 0; e < 4; ++e) {
        const int i = t * kTile + 4 * threadIdx.x + e;
        if (i < V) visit(i, p[i]);
      }
      if ((t + 1) % tpc == 0 || t == ntiles - 1) chunk_done(t);  // chunk t / tpc ends here
    }
  }
  if (threadIdx.x == 0) { sh.pick = -1; sh.u32b = 0u; }
  __syncthreads();
  // wave 0: the total, the target and the first chunk whose inclusive prefix exceeds it; when
  // none does (u * total reaches the total), the last chunk with kept mass, scanned for its last
  // kept element
  if (threadIdx.x < 64) {
    uint64_t c[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) c[e] = sh.mass[4 * lane + e];
    const uint64_t lm = c[0] + c[1] + c[2] + c[3];
    const uint64_t incl = wave_incl_scan_u64(lm);
    const uint64_t tot = readlane_u64(incl, 63);
    const double target = rp.u * (double)tot;
    uint64_t run = incl - lm;
    int first = 256, lastc = -1;
    uint64_t first_excl = 0, last_excl = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (first == 256 && c[e] && (double)(run + c[e]) > target) { first = 4 * lane + e; first_excl = run; }
      if (c[e]) { lastc = 4 * lane + e; last_excl = run; }
      run += c[e];
    }
    int f = first;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) f = min(f, __builtin_amdgcn_ds_bpermute((lane ^ o) << 2, f));
    const uint64_t lb = __builtin_amdgcn_ballot_w64(lastc >= 0);
    const int ll = lb ? 63 - __builtin_clzll(lb) : -1;  // the lane holding the last kept chunk
    if (first == f && f < 256) {
      sh.u32a = (uint32_t)f;
      sh.u64a = first_excl;
    }
    if (f == 256 && lane == ll) {
      sh.u32a = (uint32_t)lastc;
      sh.u64a = last_excl;
    }
    if (lane == 0) {
      if (f == 256 && ll < 0) sh.u32a = 0xffffffffu;  // nothing kept
      sh.u64b = __builtin_bit_cast(uint64_t, target);
    }
  }
  __syncthreads();
  // inverse CDF inside the chunk: tiles of 4 consecutive elements per thread, block-scanned in
  // index order
  if (sh.u32a != 0xffffffffu) {
    const int chunk = (int)sh.u32a;
    const double target = __builtin_bit_cast(double, sh.u64b);
    uint64_t run = sh.u64a;
    int last = -1;  // this thread's last kept element of the chunk
    const int end = min(V, (chunk + 1) * tpc * kTile);
    for (int base = chunk * tpc * kTile; base < end; base += kTile) {
      const int i0 = base + 4 * threadIdx.x;
      float x[4];
      load4(i0, x);
      uint64_t m[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) m[e] = kept_mass(x[e]);
      const uint64_t mine = m[0] + m[1] + m[2] + m[3];
      // inclusive scan of `mine` over the block
      uint64_t incl = wave_incl_scan_u64(mine);
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
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (m[e]) last = i0 + e;  // ascending within the thread and across tiles
      __syncthreads();
      if (sh.pick >= 0) break;
      run += tile;
    }
    if (sh.pick < 0 && last >= 0) atomicMax((unsigned*)&sh.u32b, (unsigned)(last + 1));
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const int j = sh.pick >= 0 ? sh.pick : (int)sh.u32b - 1;
    a.out[r] = (idx && j >= 0) ? (int32_t)idx[j] : j;
  }
}

// Candidate lists. Pass A keeps each thread's two largest keys (2048 elements of the row, its
// largest among them) with the row's count of p > 0 and, for top_p, its total mass. Any subset's
// k-th largest key is at most the row's, and any subset whose mass reaches the top-p threshold
// bounds the row's top-p threshold from below the same way (the subset's mass above a key is at
// most the row's), so the subset's own thresholds are floors for the row's. Pass B copies every
// element at or above the floor into LDS in vocabulary order (each wave owns a contiguous
// segment of the row and appends with ballots), and the exact selection and the draw then run
// over that list. No floor (k above the subset's count, a subset mass below the threshold), or
// more than kWaveCands candidates in some wave's segment, sends the row to the direct passes.
constexpr int kWaveCands = 512;
constexpr int kCands = kWaveCands * kSampWaves;
// The one-read top_k path: the floor comes from a sample of the row (the first three batches of
// every wave's segment, kSampleElems elements); it runs for k <= kOnePassMaxK (about
// k * V / kSampleElems candidates: for k = 50 at V = 128256 about 150, inside the short-list
// path's 1024 for every row) and rows of at least kOnePassMinV elements (shorter rows gain little
// from skipping a read).
constexpr int kSampleElems = 3 * 4 * 256 * kSampWaves;
constexpr int kOnePassMaxK = 256;
constexpr int kHeadMaxima = 256;  // the sample floor: the k-th largest of this many group maxima
static_assert(kOnePassMaxK <= kHeadMaxima, "the sample floor needs k <= kHeadMaxima");
constexpr int kOnePassMinV = 65536;

struct alignas(16) CandShared {
  float val[kCands];  // the per-thread tops (pass A), then the candidates
  uint32_t idx[kCands];
  int32_t wn[kSampWaves];
};

// Pass A of the candidate lists: each thread's two largest keys, stored as floats at
// tops[2 thread], tops[2 thread + 1]; count = the thread's count of p > 0, mass = its mass (when
// with_mass). Returns the mass of the two stored keys.
constexpr int kTops = 2 * kSampThreads;
__device__ __forceinline__ uint64_t thread_tops(const float* p, int V, bool vec, bool with_mass, float* tops,
                                                uint32_t& count, uint64_t& mass) {
  uint32_t t1 = 0u, t2 = 0u, c = 0;
  uint64_t m = 0;
  for_row(p, V, vec, [&](int, float x) {
    const uint32_t key = prob_key(x);
    c += key != 0;
    if (with_mass) m += prob_mass(x);
    t2 = max(t2, min(t1, key));
    t1 = max(t1, key);
  });
  count = c;
  mass = m;
  tops[2 * threadIdx.x] = __builtin_bit_cast(float, t1);
  tops[2 * threadIdx.x + 1] = __builtin_bit_cast(float, t2);
  return prob_mass(__builtin_bit_cast(float, t1)) + prob_mass(__builtin_bit_cast(float, t2));
}

// Appends this wave's candidates (pred(i, x)) to val/idx[w * kWaveCands ...] in index order and
// returns their count (which may exceed kWaveCands; only the first kWaveCands are stored).
// Which elements a candidate list keeps: kind 0 key >= lo; 1 p > 0 and x >= mthr (min_p);
// 2 keys in bin `bin` of the top_p histogram. count_pos: also count the p > 0 seen.
struct ListPred {
  int kind;
  uint32_t lo;
  uint32_t bin;
  double mthr;
  __device__ __forceinline__ bool operator()(int, float x) const {
    const uint32_t key = prob_key(x);
    return kind == 0 ? key >= lo : kind == 1 ? (key != 0u && (double)x >= mthr) : (key >> 20) == bin;
  }
};

template <typename P>
__device__ __forceinline__ int compact_segment(const float* p, int V, bool vec, P&& pred, CandShared& cs) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint64_t lt = (1ull << lane) - 1ull;
  float* val = cs.val + w * kWaveCands;
  uint32_t* idx = cs.idx + w * kWaveCands;
  int n = 0;
  auto emit = [&](uint32_t bits, int i0, const float* x, int stride) {
    const uint32_t c = __builtin_popcount(bits);
    if (__builtin_amdgcn_ballot_w64(c != 0) == 0) return;
    const uint64_t b0 = __builtin_amdgcn_ballot_w64(c & 1u), b1 = __builtin_amdgcn_ballot_w64(c & 2u),
                   b2 = __builtin_amdgcn_ballot_w64(c & 4u);
    int pos = n + __builtin_popcountll(b0 & lt) + 2 * __builtin_popcountll(b1 & lt) +
              4 * __builtin_popcountll(b2 & lt);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (bits >> e & 1u) {
        if (pos < kWaveCands) { val[pos] = x[e]; idx[pos] = (uint32_t)(i0 + e * stride); }
        ++pos;
      }
    n += __builtin_popcountll(b0) + 2 * __builtin_popcountll(b1) + 4 * __builtin_popcountll(b2);
  };
  if (vec) {
    const int nv = V >> 2;
    const int seg = (nv + kSampWaves - 1) / kSampWaves;
    const int v0 = w * seg, v1 = min(nv, v0 + seg);
    int vb = v0;  // wave-uniform position: every lane runs the same trips (ballots need them all)
    // batches of kU x 1 KiB per wave, the next batch's loads issued before the current one is
    // compacted (two batches in flight: one memory round trip per two batches)
    constexpr int kU = 4, kB = kU * 64;  // 4 measured best (2, 8 and 16 slower)
    if (vb + kB <= v1) {
      // two register buffers in turn (no copy between them, which would wait for the younger
      // batch's loads): while one batch is compacted the next one's loads are in flight
      float4 x[kU], y[kU];
      auto load = [&](float4 (&d)[kU], int at) {
#pragma unroll
        for (int k = 0; k < kU; ++k) d[k] = *reinterpret_cast<const float4*>(p + 4 * (at + lane + 64 * k));
      };
      auto scan = [&](const float4 (&d)[kU], int at) {
#pragma unroll
        for (int k = 0; k < kU; ++k) {
          const float xe[4] = {d[k].x, d[k].y, d[k].z, d[k].w};
          const int i0 = 4 * (at + lane + 64 * k);
          uint32_t bits = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) bits |= (uint32_t)pred(i0 + e, xe[e]) << e;
          emit(bits, i0, xe, 1);
        }
      };
      load(x, vb);
      if (vb + 2 * kB <= v1) load(y, vb + kB);
      for (;;) {
        // x holds batch vb, y (if vb + 2 kB <= v1) batch vb + kB
        const bool has_y = vb + 2 * kB <= v1;
        scan(x, vb);
        if (has_y && vb + 3 * kB <= v1) load(x, vb + 2 * kB);
        vb += kB;
        if (!has_y) break;
        const bool has_x = vb + 2 * kB <= v1;
        scan(y, vb);
        if (has_x && vb + 3 * kB <= v1) load(y, vb + 2 * kB);
        vb += kB;
        if (!has_x) break;
      }
    }
    if (vb < v1) {  // the last partial batch: one round trip, loads past the segment clamped
      float4 x[kU];
#pragma unroll
      for (int k = 0; k < kU; ++k) x[k] = *reinterpret_cast<const float4*>(p + 4 * min(vb + lane + 64 * k, v1 - 1));
#pragma unroll
      for (int k = 0; k < kU; ++k) {
        const int v = vb + lane + 64 * k;
        const float xe[4] = {x[k].x, x[k].y, x[k].z, x[k].w};
        uint32_t bits = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) bits |= (uint32_t)(v < v1 && pred(4 * v + e, xe[e])) << e;
        emit(bits, 4 * v, xe, 1);
      }
    }
    if (w == kSampWaves - 1) {  // the last < 4 elements belong to the last segment
      const int i = 4 * nv + lane;
      float xe[4] = {i < V ? p[i] : 0.f, 0.f, 0.f, 0.f};
      emit(i < V ? (uint32_t)pred(i, xe[0]) : 0u, i, xe, 0);
    }
  } else {
    const int seg = (V + kSampWaves - 1) / kSampWaves;
    const int i1 = min(V, w * seg + seg);
    for (int i = w * seg + lane; i - lane < i1; i += 64) {
      float xe[4] = {i < i1 ? p[i] : 0.f, 0.f, 0.f, 0.f};
      emit(i < i1 ? (uint32_t)pred(i, xe[0]) : 0u, i, xe, 0);
    }
  }
  return n;
}

// top_p over rows whose kept set is too large for the two-read candidate path: a histogram of the
// row's mass by the top 11 bits of the key (sign 0, exponent, 3 mantissa bits: 2048 bins, each an
// eighth of a binade) locates the bin holding the threshold in one pass; then either every key
// from that bin up is gathered (when they fit), or only that bin's keys, whose radix search over
// the 20 remaining bits gives the exact threshold. Bins spread the LDS atomics over many
// addresses (an 8-bit first radix digit puts nearly every key of a row in a handful of bins).
constexpr int kBinShift = 20, kBins = 2048;
struct HistShared {
  uint32_t cnt[kBins];
  uint64_t mass[kBins];
  uint64_t above;    // mass of the keys in bins above the selected one
  uint32_t bin;      // the selected bin (0xffffffff: the row has no p > 0)
  uint32_t n_ge;     // keys in bins >= the selected one
  uint32_t n_bin;    // keys in the selected bin
};

// The bin holding the top_p threshold for thr = top_p * row mass: the lowest non-empty bin whose
// mass above it (the bins above) is below thr, or the highest non-empty bin when none is (thr <=
// 0: the threshold is the maximal key). Wave 0 scans 32 bins per lane from the top.
__device__ __forceinline__ void select_bin(double thr, HistShared& hs) {
  if (threadIdx.x >= 64) return;
  const int lane = threadIdx.x;
  uint64_t lm = 0;
  uint32_t lc = 0;
#pragma unroll 4
  for (int e = 0; e < 32; ++e) {
    const int d = kBins - 1 - 32 * lane - e;
    lm += hs.mass[d];
    lc += hs.cnt[d];
  }
  const uint64_t im = wave_incl_scan_u64(lm);
  const uint32_t ic = (uint32_t)wave_incl_scan_u64(lc);
  // this lane's lowest qualifying bin and its highest non-empty bin
  uint64_t a = im - lm;
  int low = kBins, high = -1;
#pragma unroll 4
  for (int e = 0; e < 32; ++e) {
    const int d = kBins - 1 - 32 * lane - e;
    if (hs.cnt[d]) {
      if ((double)a < thr) low = d;
      high = max(high, d);
    }
    a += hs.mass[d];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    low = min(low, __builtin_amdgcn_ds_bpermute((lane ^ o) << 2, low));
    high = max(high, __builtin_amdgcn_ds_bpermute((lane ^ o) << 2, high));
  }
  const int dsel = low < kBins ? low : high;
  if (dsel < 0) {
    if (lane == 0) hs.bin = 0xffffffffu;
    return;
  }
  if ((kBins - 1 - dsel) / 32 == lane) {  // the owner records the mass and counts above dsel
    uint64_t ma = im - lm;
    uint32_t ca = ic - lc;
  #pragma unroll 4
  for (int e = 0; e < 32; ++e) {
      const int d = kBins - 1 - 32 * lane - e;
      if (d == dsel) break;
      ma += hs.mass[d];
      ca += hs.cnt[d];
    }
    hs.bin = (uint32_t)dsel;
    hs.above = ma;
    hs.n_ge = ca + hs.cnt[dsel];
    hs.n_bin = hs.cnt[dsel];
  }
}

// The k-th largest of a wave's keys (KPL per lane; 0 for no key): the largest v with at least k
// keys >= v, found bit by bit from the top with ballots (keys of p > 0 have bit 31 clear); 0 when
// fewer than k keys are positive.
template <int KPL>
__device__ __forceinline__ uint32_t wave_kth_largest(const uint32_t (&key)[KPL], int k) {
  uint32_t prefix = 0u;
  for (int b = 30; b >= 0; --b) {
    const uint32_t cand = prefix | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < KPL; ++j) cnt += __builtin_popcountll(__builtin_amdgcn_ballot_w64(key[j] >= cand));
    if (cnt >= k) prefix = cand;
  }
  return prefix;
}

// Raises a wave's floor to the k-th largest key of its candidate list (n entries at val / idx)
// when that is higher and keeps, in order, the entries at or above the floor; returns the new
// count. Every read of the list precedes every write (entries only move to lower positions).
__device__ __forceinline__ int wave_shrink(float* val, uint32_t* idx, int n, int k, uint32_t& f) {
  constexpr int J = kWaveCands / 64;
  const int lane = threadIdx.x & 63;
  const uint64_t lt = (1ull << lane) - 1ull;
  float v[J];
  uint32_t ix[J], key[J];
  __builtin_amdgcn_wave_barrier();  // the list's last appends (other lanes' writes) come first
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int i = 64 * j + lane;
    v[j] = i < n ? val[i] : 0.f;
    ix[j] = i < n ? idx[i] : 0u;
    key[j] = i < n ? prob_key(v[j]) : 0u;
  }
  f = max(f, wave_kth_largest<J>(key, k));
  int base = 0;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const bool keep = key[j] >= f && key[j] != 0u;
    const uint64_t b = __builtin_amdgcn_ballot_w64(keep);
    if (keep) {
      const int pos = base + (int)__builtin_popcountll(b & lt);
      val[pos] = v[j];
      idx[pos] = ix[j];
    }
    base += (int)__builtin_popcountll(b);
  }
  return base;
}

// The wave's largest of v (all lanes active), in every lane.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = max(v, (uint32_t)__builtin_amdgcn_ds_bpermute(((threadIdx.x & 63) ^ o) << 2, (int)v));
  return v;
}
// The largest float at or below min_p * mx (computed in fp64, as the kept test (double)x >=
// min_p * max does), and at least the smallest positive float: x >= it for every x kept under
// any maximum >= mx.
__device__ __forceinline__ float minp_floor(double min_p, float mx) {
  const double t = min_p * (double)mx;
  float fl = (float)t;
  if ((double)fl > t) fl = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, fl) - 1u);
  return fmaxf(fl, __builtin_bit_cast(float, 1u));
}
// min_p's shrink of a wave's candidate list: raises the floor ff to minp_floor of the list's
// largest key and keeps, in order, the entries at or above it (entries only move to lower
// positions; every read precedes every write).
__device__ __forceinline__ int minp_shrink(float* val, uint32_t* idx, int n, double min_p, float& ff) {
  constexpr int J = kWaveCands / 64;
  const int lane = threadIdx.x & 63;
  const uint64_t lt = (1ull << lane) - 1ull;
  float v[J];
  uint32_t ix[J];
  __builtin_amdgcn_wave_barrier();  // the list's last appends (other lanes' writes) come first
  uint32_t mk = 0u;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int i = 64 * j + lane;
    v[j] = i < n ? val[i] : 0.f;
    ix[j] = i < n ? idx[i] : 0u;
    mk = max(mk, prob_key(v[j]));
  }
  ff = fmaxf(ff, minp_floor(min_p, __builtin_bit_cast(float, wave_max_u32(mk))));
  int base = 0;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const bool keep = 64 * j + lane < n && v[j] >= ff;
    const uint64_t b = __builtin_amdgcn_ballot_w64(keep);
    if (keep) {
      const int pos = base + (int)__builtin_popcountll(b & lt);
      val[pos] = v[j];
      idx[pos] = ix[j];
    }
    base += (int)__builtin_popcountll(b);
  }
  return base;
}

// One read of the row for top_k (k <= kOnePassMaxK), as wave segments: each wave keeps, in
// vocabulary order, the candidates at or above its own floor, which starts at the sample floor (a
// floor under the row's k-th largest key: the k-th largest of the maxima of kHeadMaxima disjoint
// groups of kSampleElems / kHeadMaxima sampled elements, a subset of the row; the sample's
// largest keys mostly fall in different groups, so it is nearly as tight as the sample's k-th
// largest) and rises to the k-th largest key of the wave's list whenever the list would overflow
// (wave_shrink; rows whose largest keys cluster in one segment). A subset's k-th largest never
// exceeds the row's, so every key at or above the row's k-th largest stays listed; a wave with
// more than kSampThreads / kSampWaves entries at the end keeps its own top k (ties included), so
// the lists together usually fit the short-list path. Returns the wave's count, more than
// kWaveCands when a list of ties would not shrink (unusable).
template <bool kMinP>
__device__ __forceinline__ int one_read_segment(const float* p, int V, int k, double min_p, CandShared& cs) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint64_t lt = (1ull << lane) - 1ull;
  float* val = cs.val + w * kWaveCands;
  uint32_t* idx = cs.idx + w * kWaveCands;
  int n = 0;
  bool over = false;
  uint32_t f = 1u;
  float ff = 0.f;  // the floor as a float: for f >= 1, x >= ff iff prob_key(x) >= f (NaN fails)
  // the list's shrink when it would overflow: top_k keeps the wave's own top k, min_p the keys at
  // or above min_p times the wave's largest key (the row's is at least as large)
  auto shrink = [&]() {
    if constexpr (kMinP) {
      n = minp_shrink(val, idx, n, min_p, ff);
    } else {
      n = wave_shrink(val, idx, n, k, f);
      ff = __builtin_bit_cast(float, f);
    }
  };
  // appends the keys >= f of four consecutive elements per lane (up to 256 per call); most calls
  // find none and leave after one ballot
  auto add4 = [&](const float (&x)[4], int i0, bool live) {
    if (over) return;
    uint32_t bits = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) bits |= (uint32_t)(live && x[e] >= ff) << e;
    if (__builtin_amdgcn_ballot_w64(bits != 0u) == 0) return;
    if (n + 256 > kWaveCands) {
      shrink();
      if (n + 256 > kWaveCands) {  // keys that do not shrink: the list is unusable
        over = true;
        return;
      }
      bits = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) bits |= (uint32_t)(live && x[e] >= ff) << e;
    }
    const uint32_t cnt = __builtin_popcount(bits);
    const uint64_t b0 = __builtin_amdgcn_ballot_w64(cnt & 1u), b1 = __builtin_amdgcn_ballot_w64(cnt & 2u),
                   b2 = __builtin_amdgcn_ballot_w64(cnt & 4u);
    int pos = n + __builtin_popcountll(b0 & lt) + 2 * __builtin_popcountll(b1 & lt) +
              4 * __builtin_popcountll(b2 & lt);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (bits >> e & 1u) {
        val[pos] = x[e];
        idx[pos] = (uint32_t)(i0 + e);
        ++pos;
      }
    n += __builtin_popcountll(b0) + 2 * __builtin_popcountll(b1) + 4 * __builtin_popcountll(b2);
  };
  const int nv = V >> 2;
  const int seg = (nv + kSampWaves - 1) / kSampWaves;
  const int v0 = w * seg, v1 = min(nv, v0 + seg);
  // the segment in batches of kB vectors; the last batch's loads past the segment are clamped to
  // its last vector and their keys dropped
  constexpr int kU = 4, kB = kU * 64;
  const int nb = v1 > v0 ? (v1 - v0 + kB - 1) / kB : 0;
  auto scan = [&](const float4 (&d)[kU], int at) {
#pragma unroll
    for (int q = 0; q < kU; ++q) {
      const int v = at + lane + 64 * q;
      const float xe[4] = {d[q].x, d[q].y, d[q].z, d[q].w};
      add4(xe, 4 * v, v < v1);
    }
  };
  float4 x[kU], y[kU], z[kU];
  auto load = [&](float4 (&d)[kU], int at) {
#pragma unroll
    for (int q = 0; q < kU; ++q)
      d[q] = *reinterpret_cast<const float4*>(p + 4 * min(at + lane + 64 * q, v1 - 1));
  };
  auto dmax = [](const float4 (&d)[kU]) {
    uint32_t m = 0u;
#pragma unroll
    for (int q = 0; q < kU; ++q)
      m = max(m, max(max(prob_key(d[q].x), prob_key(d[q].y)), max(prob_key(d[q].z), prob_key(d[q].w))));
    return m;
  };
  // The floor comes from the segments' first three batches (the start of every wave's segment,
  // 3 kB vectors per wave): the maxima of kHeadMaxima disjoint groups of them (a lane's 48
  // elements, then threads t, t + kHeadMaxima, ...), bitonic-sorted (no LDS atomics, which
  // serialise on keys sharing their top bits) in the candidates' memory, which is dead until the
  // floor is known. (The loads are unconditional: rows of at least kOnePassMinV elements give
  // every segment more than three batches.)
  load(x, v0);
  load(y, v0 + kB);
  load(z, v0 + 2 * kB);
  if constexpr (kMinP) {
    // min_p: min_p times the sample's largest key, rounded down to a float
    uint32_t hm = max(dmax(x), max(dmax(y), dmax(z)));
    hm = (uint32_t)wave_max_u32(hm);
    __shared__ uint32_t wmx[kSampWaves];
    if (lane == 0) wmx[w] = hm;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kSampWaves; ++i) hm = max(hm, wmx[i]);
    ff = minp_floor(min_p, __builtin_bit_cast(float, hm));
  } else {
    uint32_t hm = max(dmax(x), max(dmax(y), dmax(z)));
    uint32_t* buf = reinterpret_cast<uint32_t*>(cs.val);
    buf[threadIdx.x] = hm;
    __syncthreads();
    if (threadIdx.x < kHeadMaxima) {
#pragma unroll
      for (int i = 1; i < kSampThreads / kHeadMaxima; ++i) hm = max(hm, buf[threadIdx.x + i * kHeadMaxima]);
    }
    __shared__ uint32_t f0;
    hm = sort_desc_keys<kHeadMaxima>(hm, buf);
    if (threadIdx.x == k - 1) f0 = hm;
    __syncthreads();
    f = max(f0, 1u);
    ff = __builtin_bit_cast(float, f);
    __syncthreads();  // the sort buffer is dead from here: its memory holds the candidates
  }
  // three register buffers in turn (no copies between them, which would wait for the loads in
  // flight)
  for (int b = 0; b < nb; b += 3) {
    scan(x, v0 + b * kB);
    if (b + 3 < nb) load(x, v0 + (b + 3) * kB);
    if (b + 1 >= nb) break;
    scan(y, v0 + (b + 1) * kB);
    if (b + 4 < nb) load(y, v0 + (b + 4) * kB);
    if (b + 2 >= nb) break;
    scan(z, v0 + (b + 2) * kB);
    if (b + 5 < nb) load(z, v0 + (b + 5) * kB);
  }
  if (w == kSampWaves - 1) {  // the last < 4 elements belong to the last segment
    const int i = 4 * nv + lane;
    float xe[4] = {i < V ? p[i] : 0.f, 0.f, 0.f, 0.f};
    add4(xe, i, i < V);  // elements 1-3 of xe are 0: no key
  }
  if (over) return kWaveCands + 1;
  if (n > kSampThreads / kSampWaves) shrink();
  return n;
}

// Copies the elements that satisfy pred into cs.val / cs.idx in vocabulary order (each wave its
// own segment, then the gaps between the segments' lists closed); *total = the list's length.
// npos (optional): the row's count of p > 0, counted on the way (a top_k list's length stands in
// for it, below). False when some segment overflowed (the list is then unusable). topk > 0: the
// candidates of a top_k (one_read_segment, vec rows only) instead of pred's; minp > 0: those of a
// min_p the same way.
__device__ __forceinline__ bool gather_list(const float* p, int V, bool vec, const ListPred& pred, CandShared& cs,
                                         int* total_out, uint32_t* npos, int topk = 0, double minp = 0.0) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint32_t c = 0;
  const int n = topk > 0 ? one_read_segment<false>(p, V, topk, 0.0, cs)
              : minp > 0.0 ? one_read_segment<true>(p, V, 0, minp, cs)
                           : compact_segment(p, V, vec, [&](int i, float x) {
    c += prob_key(x) != 0u;
    return pred(i, x);
  }, cs);
  if (lane == 0) cs.wn[w] = n;
  __syncthreads();
  if (npos && topk == 0 && !(minp > 0.0)) {
    c = (uint32_t)wave_sum_u64(c);
    __shared__ uint32_t wc[kSampWaves];
    if (lane == 0) wc[w] = c;
    __syncthreads();
    uint32_t t = 0;
    for (int i = 0; i < kSampWaves; ++i) t += wc[i];
    *npos = t;
  }
  int total = 0;
  bool over = false;
  for (int i = 0; i < kSampWaves; ++i) {
    over |= cs.wn[i] > kWaveCands;
    total += cs.wn[i];
  }
  if (over) return false;
  // A top_k list stands in for the row's count of p > 0: it holds every key at or above the
  // row's k-th largest, so it has at least k entries when the row has k positive keys and
  // every positive key otherwise; its length then decides k < count and k >= count alike.
  if (npos && (topk > 0 || minp > 0.0)) *npos = (uint32_t)total;  // (min_p does not use it)
  // close the gaps between the segments' lists: list position d takes its entry from the wave
  // whose prefix range holds it (moves go to lower slots: read, then write); positions past the
  // total are skipped, so a short list costs one read and one write per thread
  constexpr int J = kCands / kSampThreads;
  float mv[J];
  uint32_t mi[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int d = threadIdx.x + j * kSampThreads;
    if (d < total) {
      int base = 0, sw = 0;
      for (; sw < kSampWaves - 1 && d >= base + cs.wn[sw]; ++sw) base += cs.wn[sw];
      const int s = sw * kWaveCands + (d - base);
      mv[j] = cs.val[s];
      mi[j] = cs.idx[s];
    }
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int d = threadIdx.x + j * kSampThreads;
    if (d < total) { cs.val[d] = mv[j]; cs.idx[d] = mi[j]; }
  }
  *total_out = total;
  return true;
}

// The histogram pass: every bin's count and mass, the row's count of p > 0 and its mass.
__device__ __forceinline__ void hist_pass(const float* p, int V, bool vec, HistShared& hs, SampleShared& sh,
                                       int64_t* npos, uint64_t* row_tot) {
  for (int i = threadIdx.x; i < kBins; i += kSampThreads) { hs.cnt[i] = 0u; hs.mass[i] = 0ull; }
  __syncthreads();
  uint32_t c = 0;
  uint64_t m = 0;
  for_row(p, V, vec, [&](int, float x) {
    const uint32_t key = prob_key(x);
    if (key) {
      const uint64_t pm = prob_mass(x);
      ++c;
      m += pm;
      atomicAdd(&hs.cnt[key >> kBinShift], 1u);
      atomicAdd((unsigned long long*)&hs.mass[key >> kBinShift], (unsigned long long)pm);
    }
  });
  *npos = (int64_t)block_sum_u64(c, sh);
  *row_tot = block_sum_u64(m, sh);
}

// kTopP: the top_p instantiation (mode 1 only, the histogram path); the other serves modes 0, 2-4.
// Two kernels, so each gets the registers its own paths need.
template <bool kTopP>
__global__ __launch_bounds__(kSampThreads) void sample_kernel(SampleArgs a) {
  prefetch_kernarg<(int)sizeof(SampleArgs)>(a);
  __shared__ SampleShared sh;
  __shared__ CandShared cs;
  const int r = blockIdx.x;
  const int src = a.rows ? a.rows[r] : r;
  if (src < 0 || src >= a.nrows) {  // a row index outside probs: no draw
    if (threadIdx.x == 0) a.out[r] = -1;
    return;
  }
  const float* p = a.probs + (int64_t)src * a.stride;
  const int V = a.V;
  const bool vec = a.vec != 0;
  const int mode = kTopP ? 1 : a.mode;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const RowParams rp = row_params(a, r);
  const int32_t k = (mode == 2 || mode == 4) ? rp.k : 0;
  // what the selection runs over: the row (direct passes) or its candidate list
  const float* sp = p;
  const uint32_t* sidx = nullptr;
  int sV = V;
  bool svec = vec;
  int64_t npos = -1;
  uint64_t row_tot = 0;
  // Copies the elements that satisfy pred into the candidate list (gather_list) and points the
  // selection at it; false (and the list unused) when some segment overflowed.
  auto gather = [&](const ListPred& pred, uint32_t* npos_out = nullptr, int topk = 0, double minp = 0.0) -> bool {
    int total;
    if (!gather_list(p, V, vec, pred, cs, &total, npos_out, topk, minp)) return false;
    sp = cs.val;
    sidx = cs.idx;
    sV = total;
    svec = true;
    return true;
  };
  bool listed = false;
  uint32_t lo_given = 0u;
  if constexpr (kTopP) {
    __shared__ HistShared hs;
    // top_p: the histogram pass (with the row's count of p > 0 and its mass), then one gather
    hist_pass(p, V, vec, hs, sh, &npos, &row_tot);
    const double thr = (double)rp.tp * (double)row_tot;
    select_bin(thr, hs);
    __syncthreads();
    const uint32_t bin = hs.bin;
    if (bin != 0xffffffffu) {
      const uint32_t bin_lo = bin << kBinShift;
      // one gather: every key from the threshold's bin up when they fit (the draw then runs over
      // the list), else the bin's keys alone (their radix search gives the threshold); one call
      // site, so the list code is inlined once
      bool got = false;
      int attempt = hs.n_ge <= (uint32_t)kCands ? 0 : 1;
      for (; attempt < 2 && !got; ++attempt) {
        if (attempt == 1 && hs.n_bin > (uint32_t)kCands) break;
        __syncthreads();
        got = gather(attempt == 0 ? ListPred{0, bin_lo, 0u, 0.0} : ListPred{2, 0u, bin, 0.0});
      }
      listed = got && attempt == 1;  // the loop's increment ran once after the first success
      // the threshold: a radix search inside the bin (keys of other bins are skipped), over the
      // list (every key from the bin up, or the bin's keys) or, when neither fit, over the row
      const double thr_in = thr - (double)hs.above;  // the bin's share of the threshold
      __syncthreads();
      lo_given = radix_threshold(got ? cs.val : p, got ? sV : V, got || vec, 1u, true, 0u, thr_in, sh, bin_lo,
                                 ~((1u << kBinShift) - 1u), kBinShift - 8);
      lo_given = max(lo_given, 1u);
      if (!listed) {  // the draw runs over the row
        sp = p;
        sidx = nullptr;
        sV = V;
        svec = vec;
      }
    }
    __syncthreads();
  }
  // One read for top_k (alone or before top_p) with k <= kOnePassMaxK over a long row: the k-th
  // largest of a sample of the row is a floor under the row's k-th largest, so one pass collects
  // every element at or above it (about k * V / kSampleElems of them for exchangeable rows; each
  // wave raises its own floor when its list fills, so rows whose largest keys cluster stay on this
  // path). A list of ties that will not shrink falls back to the passes below.
  if (!kTopP && (mode == 2 || mode == 4) && vec && k > 0 && k <= kOnePassMaxK && V >= kOnePassMinV) {
    uint32_t c = 0;
    listed = gather(ListPred{0, 0u, 0u, 0.0}, &c, k);  // the floor comes from the sample
    npos = (int64_t)c;
    __syncthreads();
  }
  // One read for min_p (0 < min_p <= 1) over a long row: min_p times the largest key of the same
  // sample is a floor under min_p times the row's largest key, each wave raising its own floor to
  // min_p times its list's largest key when the list fills; the list holds the row's largest key
  // and every kept one, and the draw below takes the row's maximum from it.
  if (!kTopP && mode == 3 && vec && V >= kOnePassMinV && rp.mp > 0.f && rp.mp <= 1.f) {
    listed = gather(ListPred{0, 0u, 0u, 0.0}, nullptr, 0, (double)rp.mp);
    __syncthreads();
  }
  // plain sampling, and top_k with k outside (0, V), keep every p > 0: no candidate list; top_p
  // went through the histogram above
  if (!kTopP && !listed && !(mode == 0 || ((mode == 2 || mode == 4) && !(k > 0 && k < V)))) {
    // pass A
    bool lists = true;
    uint32_t cand_lo = 1u;  // candidates: key >= cand_lo (top_k, top_p) or x >= mthr (min_p)
    double mthr = 0.0;
    if (mode == 3) {
      uint32_t mk = 0;
      for_row(p, V, vec, [&](int, float x) { mk = max(mk, prob_key(x)); });
      mk = block_max_u32(mk, sh);
      mthr = (double)rp.mp * (double)__builtin_bit_cast(float, mk);
    } else {
      const bool by_mass = mode == 1;
      uint32_t c = 0;
      uint64_t m = 0;
      uint64_t tm = thread_tops(p, V, vec, by_mass, cs.val, c, m);
      npos = (int64_t)block_sum_u64(c, sh);
      if (by_mass) {
        row_tot = block_sum_u64(m, sh);
        tm = block_sum_u64(tm, sh);
        const double thr = (double)rp.tp * (double)row_tot;
        // a floor needs the subset's mass to reach the threshold
        cand_lo = (double)tm < thr ? 0u : radix_threshold(cs.val, kTops, true, 1u, true, 0u, thr, sh);
      } else if ((int64_t)k < npos) {
        cand_lo = radix_threshold(cs.val, kTops, true, 1u, false, (uint32_t)k, 0.0, sh);
      } else {
        cand_lo = 1u;  // k >= the count of p > 0: top_k keeps everything
      }
      lists = cand_lo > 1u;
      __syncthreads();  // the tops are dead from here: their memory holds the candidates
    }
    if (lists) {
      // pass B (with too many candidates in some segment, the direct passes run over the row)
      gather(mode == 3 ? ListPred{1, 0u, 0u, mthr} : ListPred{0, cand_lo, 0u, 0.0});
    }
    __syncthreads();
  }
  sample_row(sp, sidx, sV, svec, a, r, rp, npos, row_tot, sh,
             sidx ? reinterpret_cast<uint32_t*>(cs.val + kSampThreads) : nullptr, lo_given);
}

// safe_scaled_softmax: probs = softmax(logits / T) per row, or the one-hot of the first maximum
// when T < greedy_threshold; fp32 math in the exp2 domain, output in the logits' dtype. This
// streaming kernel serves rows too long (or not aligned) for the register-resident one below:
// two passes over the row, (max, first argmax, sum of exp2 relative to a running max) with
// 16-byte loads, then the normalised write.
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
    // a masked (-inf) logit adds 0; with mx still -inf, (x - mx) would be NaN
    s += x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((x - mx) * c);
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
  for (int v = threadIdx.x; v < nv; v += kSampThreads) {
    float x[E];
    if (greedy_row) {
#pragma unroll
      for (int e = 0; e < E; ++e) x[e] = (v * E + e) == A ? 1.f : 0.f;
    } else {
      IO::load(row, (int64_t)v * E, x);
#pragma unroll
      for (int e = 0; e < E; ++e) x[e] = __builtin_amdgcn_exp2f((x[e] - M) * c) * inv;
    }
    IO::store(orow, (int64_t)v * E, x);
  }
  for (int i = nv * E + threadIdx.x; i < V; i += kSampThreads)
    IO::put(orow, i, greedy_row ? (i == A ? 1.f : 0.f) : __builtin_amdgcn_exp2f((IO::get(row, i) - M) * c) * inv);
}

// safe_scaled_softmax with the row held in registers (NV 16-byte vectors per thread, the row's
// last V % E elements one per thread): one read and one write of the row. The maximum first (and,
// for greedy rows, its first index), then the sum of exp2((x - max)*c), then the write from
// registers.
__device__ __forceinline__ float block_max_f(float v, float* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1)
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ o) << 2, __builtin_bit_cast(int, v))));
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < kSampWaves; ++i) t = fmaxf(t, red[i]);
  return t;
}
__device__ __forceinline__ float block_sum_f(float v, float* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1)
    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ o) << 2, __builtin_bit_cast(int, v)));
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < kSampWaves; ++i) t += red[i];
  return t;
}
__device__ __forceinline__ int block_min_i(int v, float* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = min(v, __builtin_amdgcn_ds_bpermute((lane ^ o) << 2, v));
  __syncthreads();
  if (lane == 0) red[w] = __builtin_bit_cast(float, v);
  __syncthreads();
  int t = __builtin_bit_cast(int, red[0]);
#pragma unroll
  for (int i = 1; i < kSampWaves; ++i) t = min(t, __builtin_bit_cast(int, red[i]));
  return t;
}

// Wave-wide max / sum: DPP within each 16-lane row (row_ror 8, 4; quad_perm), after which every
// lane of a row holds the row's value, then the four rows' values read from lanes 0, 16, 32, 48
// and combined in that order, so every lane gets the same result.
template <bool kMax>
__device__ __forceinline__ float wave_reduce_dpp(float v) {
  auto op = [](float x, float y) { return kMax ? fmaxf(x, y) : x + y; };
  auto dpp = [](float x, auto ctrl) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), decltype(ctrl)::value, 0xF, 0xF, false));
  };
  v = op(v, dpp(v, std::integral_constant<int, 0x128>{}));  // row_ror:8
  v = op(v, dpp(v, std::integral_constant<int, 0x124>{}));  // row_ror:4
  v = op(v, dpp(v, std::integral_constant<int, 0x4E>{}));   // quad_perm [2,3,0,1]
  v = op(v, dpp(v, std::integral_constant<int, 0xB1>{}));   // quad_perm [1,0,3,2]
  auto rd = [&](int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l)); };
  return op(op(rd(0), rd(16)), op(rd(32), rd(48)));
}
// Block-wide max / sum with one barrier: red holds kSampWaves floats used by this call alone.
template <bool kMax>
__device__ __forceinline__ float block_reduce_once(float v, float* red) {
  v = wave_reduce_dpp<kMax>(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < kSampWaves; ++i) t = kMax ? fmaxf(t, red[i]) : t + red[i];
  return t;
}

template <bool BF16, int NV>
__global__ __launch_bounds__(kSampThreads) void scaled_softmax_resident_kernel(
    const void* __restrict__ logits, int64_t stride, int V, const float* __restrict__ temps, float greedy,
    void* __restrict__ out, int64_t out_stride) {
  using IO = RowIO<BF16>;
  constexpr int E = IO::E;
  __shared__ float red[kSampWaves];
  __shared__ float red_max[kSampWaves], red_sum[kSampWaves];
  const int r = blockIdx.x;
  const char* row = reinterpret_cast<const char*>(logits) + (int64_t)r * stride * (BF16 ? 2 : 4);
  char* orow = reinterpret_cast<char*>(out) + (int64_t)r * out_stride * (BF16 ? 2 : 4);
  const int nv = V / E;
  // Every load is issued unconditionally (indices clamped into the row; the values past it are
  // never used) and the tail element's first, so the loads complete in the order the online
  // pass below consumes them and each vector is waited for alone. (Loads under conditions made
  // the compiler wait for all of them before the first use.)
  const int it = nv * E + threadIdx.x;  // this thread's tail element, if any
  const float xt_raw = IO::get(row, min(it, V - 1));
  uint4 d[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int v = min((int)threadIdx.x + j * kSampThreads, max(nv - 1, 0));
    d[j] = ld16(row + (int64_t)v * 16);
  }
  const float xt = it < V ? xt_raw : -INFINITY;
  const float T = temps[r];
  const bool greedy_row = T < greedy;
  const float c = greedy_row ? 1.f : 1.4426950408889634f / T;
  auto unpack = [&](const uint4& q, float (&x)[E]) {
    if (BF16) {
      unpack8(q, x);
    } else {
      x[0] = __uint_as_float(q.x); x[1] = __uint_as_float(q.y); x[2] = __uint_as_float(q.z); x[3] = __uint_as_float(q.w);
    }
  };
  // Online pass over this thread's elements in load order (loads complete in order, so each
  // vector is consumed as it lands and the exponentials overlap the loads still in flight):
  // running maximum m and s = sum of exp2((x - m) c), rescaled when m grows. Each vector's
  // exponentials replace its logits in registers (bf16 rows: rounded to bf16, which with the
  // final rounding stays within 2^-8 relative; fp32 rows: exact), with the reference maximum
  // mref[j] they were taken against, so the output pass needs one exponential per vector
  // (exp2((mref[j] - M) c)) instead of one per element. Rows of more than 16 vectors per thread
  // keep their logits (no registers to spare for mref) and recompute the exponentials. Greedy
  // rows need the maximum only.
  constexpr bool kKeep = NV <= 16;
  float m = -INFINITY, s = 0.f, mref[kKeep ? NV : 1];
  float et = 0.f, mt = -INFINITY;  // the tail element's exponential and its reference
  if constexpr (!kKeep) {  // the maximum first, the sum after the block maximum is known
    m = xt;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (threadIdx.x + j * kSampThreads >= nv) break;
      float x[E];
      unpack(d[j], x);
#pragma unroll
      for (int e = 0; e < E; ++e) m = fmaxf(m, x[e]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      mref[j] = -INFINITY;
      if (threadIdx.x + j * kSampThreads >= nv) break;
      float x[E];
      unpack(d[j], x);
      float mj = x[0];
#pragma unroll
      for (int e = 1; e < E; ++e) mj = fmaxf(mj, x[e]);
      if (mj > m) {
        s *= __builtin_amdgcn_exp2f((m - mj) * c);  // m = -inf: s is still 0
        m = mj;
      }
      if (!greedy_row) {
        // while every logit so far is -inf (masked), m is -inf: the reference 0 keeps
        // fmaf(-inf, c, -mc) at -inf (exponential 0) instead of NaN
        const float mc = m == -INFINITY ? 0.f : m * c;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          x[e] = __builtin_amdgcn_exp2f(fmaf(x[e], c, -mc));
          s += x[e];
        }
        mref[j] = m;
        if (BF16) d[j] = pack8(x);
        else d[j] = make_uint4(__builtin_bit_cast(uint32_t, x[0]), __builtin_bit_cast(uint32_t, x[1]),
                               __builtin_bit_cast(uint32_t, x[2]), __builtin_bit_cast(uint32_t, x[3]));
      }
    }
    if (it < V) {
      if (xt > m) {
        s *= __builtin_amdgcn_exp2f((m - xt) * c);
        m = xt;
      }
      mt = m;
      if (!greedy_row) {
        et = __builtin_amdgcn_exp2f(fmaf(xt, c, m == -INFINITY ? 0.f : -m * c));
        s += et;
      }
    }
  }
  float S;
  const float M = kKeep ? block_reduce_once<true>(m, red_max) : block_max_f(m, red);
  if (greedy_row) {
    int am = 0x7fffffff;  // first index holding the maximum
#pragma unroll
    for (int j = NV - 1; j >= 0; --j) {
      const int v = threadIdx.x + j * kSampThreads;
      if (v >= nv) continue;
      float x[E];
      unpack(d[j], x);
#pragma unroll
      for (int e = E - 1; e >= 0; --e)
        if (x[e] == M) am = v * E + e;
    }
    if (it < V && xt == M) am = min(am, it);
    const int A = block_min_i(am, red);
    float one[E];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int v = threadIdx.x + j * kSampThreads;
      if (v >= nv) break;
#pragma unroll
      for (int e = 0; e < E; ++e) one[e] = v * E + e == A ? 1.f : 0.f;
      IO::store(orow, (int64_t)v * E, one);
    }
    if (it < V) IO::put(orow, it, it == A ? 1.f : 0.f);
    return;
  }
  if constexpr (kKeep) {
    s = m == -INFINITY ? 0.f : s * __builtin_amdgcn_exp2f((m - M) * c);
    S = block_reduce_once<false>(s, red_sum);
  } else {
    s = it < V ? __builtin_amdgcn_exp2f((xt - M) * c) : 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (threadIdx.x + j * kSampThreads >= nv) break;
      float x[E];
      unpack(d[j], x);
#pragma unroll
      for (int e = 0; e < E; ++e) s += __builtin_amdgcn_exp2f((x[e] - M) * c);
    }
    S = block_sum_f(s, red);
  }
  const float inv = 1.f / S;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int v = threadIdx.x + j * kSampThreads;
    if (v >= nv) break;
    float x[E];
    unpack(d[j], x);
    if constexpr (kKeep) {
      const float f = __builtin_amdgcn_exp2f((mref[j] - M) * c) * inv;
#pragma unroll
      for (int e = 0; e < E; ++e) x[e] *= f;
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) x[e] = __builtin_amdgcn_exp2f((x[e] - M) * c) * inv;
    }
    IO::store(orow, (int64_t)v * E, x);
  }
  if (it < V)
    IO::put(orow, it, kKeep ? et * (__builtin_amdgcn_exp2f((mt - M) * c) * inv)
                            : __builtin_amdgcn_exp2f((xt - M) * c) * inv);
}

}  // namespace pie

using namespace pie;

extern "C" int pie_hip_sample(const float* probs, int64_t prob_stride, int64_t prob_rows, int64_t vocab,
                              int64_t batch, const int32_t* row_indices, int32_t mode, const int32_t* top_k,
                              int32_t top_k_scalar, const float* top_p, float top_p_scalar,
                              const float* min_p, float min_p_scalar, const double* uniforms,
                              uint64_t seed, uint64_t offset, int32_t* out, void* stream) {
  if (batch == 0) return PIE_HIP_OK;  // an empty batch (whose tensors may have null data)
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
  hipLaunchKernelGGL(mode == 1 ? sample_kernel<true> : sample_kernel<false>, dim3((unsigned)batch), dim3(kSampThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("sample");
}

extern "C" int pie_hip_scaled_softmax(const void* logits, int32_t is_bf16, int64_t stride, int64_t batch,
                                      int64_t vocab, const float* temperatures, float greedy_threshold,
                                      void* out, int64_t out_stride, void* stream) {
  if (batch == 0) return PIE_HIP_OK;  // an empty batch (whose tensors may have null data)
  PIE_REQUIRE(logits && out && temperatures, "scaled_softmax: null pointer");
  PIE_REQUIRE(vocab > 0 && vocab < (1ll << 31) && batch >= 0 && batch < (1ll << 31) && stride >= vocab &&
                  out_stride >= vocab,
              "scaled_softmax: bad shape");
  if (batch == 0) return PIE_HIP_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t e = is_bf16 ? 8 : 4;  // elements per 16-byte vector
  const int vec = aligned16(logits) && aligned16(out) && stride % e == 0 && out_stride % e == 0;
  // rows of up to 20 vectors per thread stay in registers for bf16 (163,840 entries), 16 for fp32
  // (65,536 entries: at 20 the fp32 kernel's registers spill)
  const int64_t per_thread = (vocab / e + kSampThreads - 1) / kSampThreads;
  const dim3 grid((unsigned)batch), block(kSampThreads);
#define PIE_SOFTMAX_RESIDENT(BF, NV)                                                                      \
  hipLaunchKernelGGL((scaled_softmax_resident_kernel<BF, NV>), grid, block, 0, st, logits, stride, (int)vocab, \
                     temperatures, greedy_threshold, out, out_stride)
  // (rows shorter than one 16-byte vector take the streaming kernel: the resident one reads
  // whole vectors)
  if (vec && vocab >= e && per_thread <= (is_bf16 ? 20 : 16)) {
    if (is_bf16) {
      if (per_thread <= 8) PIE_SOFTMAX_RESIDENT(true, 8);
      else if (per_thread <= 16) PIE_SOFTMAX_RESIDENT(true, 16);
      else PIE_SOFTMAX_RESIDENT(true, 20);
    } else {
      if (per_thread <= 8) PIE_SOFTMAX_RESIDENT(false, 8);
      else PIE_SOFTMAX_RESIDENT(false, 16);
    }
  } else if (is_bf16) {
    hipLaunchKernelGGL(scaled_softmax_kernel<true>, grid, block, 0, st, logits, stride, (int)vocab, temperatures,
                       greedy_threshold, out, out_stride, vec);
  } else {
    hipLaunchKernelGGL(scaled_softmax_kernel<false>, grid, block, 0, st, logits, stride, (int)vocab, temperatures,
                       greedy_threshold, out, out_stride, vec);
  }
#undef PIE_SOFTMAX_RESIDENT
  return check_launch("scaled_softmax");
}
