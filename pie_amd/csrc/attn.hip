// Paged attention over the KV cache the append kernels write: flashinfer's
// BatchDecodeWithPagedKVCacheWrapper.run and BatchPrefillWithPagedKVCacheWrapper.run as Pie
// calls them (pie/src/pie_worker/model/llama3.py:293-313, :689, :765-790; semantics restated in
// pie/src/flashinfer_metal/ops.py:163-282 and kernels/metal_attention_simdgroup_opt.metal).
//
// For request b with kv_len = (npages-1)*P + last_len[b] cached tokens and qo_len query tokens,
// query token i attends kv positions t <= kv_len - qo_len + i (or where the custom mask is set),
// head h reads kv head h / (Hq/Hkv), scores are q.k * sm_scale, output is softmax(scores) @ v.
//
// MI355X mapping. Both kernels run the matrix products on MFMA v_mfma_f32_16x16x32_bf16:
//   S^T = K Q^T   A = 16 kv tokens x 32 head dims (straight from HBM into registers: lane
//                 (n, g) holds token n's dims 8(4s+g)..+8 at step s, one 64-byte run per token
//                 per step), B = 16 query rows (the same dims permutation), C = S^T tile with
//                 lane (n, g) holding tokens 4g..4g+3 of query row n;
//   O  = P V      A = the probabilities in exactly that C layout read as 8 tokens per lane
//                 (two 16-token subtiles: tokens 4g+i and 16+4g+i), B = V staged row-major in
//                 LDS and read with ds_read_b64_tr_b16, whose 16-lane transpose turns 4 rows x
//                 4 dims into the 8-tokens-of-one-dim operand the MFMA wants.
// The query rows of one MFMA tile are (token, head) pairs of one kv-head group (GQA packing),
// so a decode step with 4 heads per kv head shares every K/V byte between its 4 heads.
// Softmax is online in the exp2 domain (scores pre-multiplied by sm_scale*log2 e); P is
// rounded to bf16 for the second product as flashinfer does; everything else is fp32.
#include <math.h>

#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "common.h"

namespace pie {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma_16x16x32(const u32x4_t& a, const u32x4_t& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// ds_read_b64_tr_b16: within each 16-lane group, output lane r element j is element r%4 of
// the 8 bytes addressed by lane 4j + r/4 (measured on gfx950).
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* p) {
  typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
  const i16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p));
  return __builtin_bit_cast(uint2, v);
}

__device__ __forceinline__ float lane_read(float v, int src_lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src_lane << 2, __builtin_bit_cast(int, v)));
}

__device__ __forceinline__ u32x4_t ld16v(const uint16_t* p) {
  return *reinterpret_cast<const u32x4_t*>(p);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
// Attention sinks (gpt_oss.py:693-697): a per-head logit in the units of the scaled scores that
// joins each row's softmax denominator and no value: the row's mass gains exp2(sink log2(e) - m)
// relative to the row's running maximum m (0 when the row saw nothing).
__device__ __forceinline__ float sink_mass(const float* sinks, int head, float m) {
  return sinks ? fast_exp2(sinks[head] * 1.4426950408889634f - (m == -INFINITY ? 0.f : m)) : 0.f;
}

// Online softmax with a lazy maximum: a row's reference maximum (and with it the rescale of its
// output accumulators and sum) moves only when a tile's scores exceed it by more than kLazyMax
// (log2 units), so every exponent stays <= 2^kLazyMax. Numerator and denominator share the
// reference, so the softmax is the same; the rescale runs a few times per row, not per tile.
constexpr float kLazyMax = 8.f;

// Kernel argument: the paged KV cache and its page table.
struct PagedKV {
  const uint16_t* k;       // k of page 0, slot 0, head 0
  const uint16_t* v;       // v of page 0, slot 0, head 0
  int64_t page_stride, slot_stride, head_stride;  // elements
  const int32_t* indptr;   // [B+1] pages per request
  const int32_t* indices;  // [sum pages] physical page ids
  const int32_t* last_len; // [B]
  int32_t num_pages;       // pages in the pool (ids outside [0, num_pages) are masked out)
  int32_t page_size;
  FastDiv pdiv;
};

__device__ __forceinline__ int kv_length(const PagedKV& kv, int b) {
  const int np = kv.indptr[b + 1] - kv.indptr[b];
  return np > 0 ? (np - 1) * kv.page_size + kv.last_len[b] : 0;
}

// Element offset of (token t of the request whose pages start at indices[page0], kv head h);
// -1 if its page id is out of range.
__device__ __forceinline__ int64_t kv_offset(const PagedKV& kv, int page0, int t, int h) {
  const uint32_t lp = kv.pdiv.div((uint32_t)t);
  const int slot = t - (int)lp * kv.page_size;
  const int page = kv.indices[page0 + (int)lp];
  if ((unsigned)page >= (unsigned)kv.num_pages) return -1;
  return (int64_t)page * kv.page_stride + (int64_t)slot * kv.slot_stride + (int64_t)h * kv.head_stride;
}

constexpr int kTileTokens = 32;  // kv tokens per wave iteration (two 16-token MFMA subtiles)

// XOR swizzle of the 16-byte chunks of LDS row r (rows of D bf16, no padding): the 16 rows one
// transpose read touches land on distinct chunks, so its 64 lanes hit every bank at most twice.
template <int D>
__device__ __forceinline__ int chunk_swizzle(int r) {
  return D == 64 ? (r >> 1) & 7 : r & 15;
}

// Swizzle of V rows, read by ds_read_b64_tr_b16: a transpose read takes two 16-byte chunks
// (one pair) from each of 16 rows, and every 8 consecutive rows must hit different 32-byte bank
// groups, so the pair index is XORed with r mod 8 (D = 64 keeps the row-pair scheme above).
template <int D>
__device__ __forceinline__ int v_swizzle(int r) {
  return D == 64 ? chunk_swizzle<64>(r) : (r & 7) << 1;
}

// Wait until this wave's LDS reads have returned (a transpose read must finish before a load
// into the same LDS tile is issued).
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt((63 << 14) | (0 << 8) | (7 << 4) | 15);
}

// Wait until at most n vector-memory operations of this wave are outstanding (loads into LDS
// included); exp and lgkm counters are not waited on.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(((N >> 4) << 14) | (15 << 8) | (7 << 4) | (N & 15));
}

// One wave's running state for 16 query rows over a stream of 32-token kv tiles.
template <int D>
struct WaveAttn {
  static constexpr int NS = D / 32;  // MFMA k-steps over the head dim
  static constexpr int NB = D / 16;  // 16-dim output blocks
  u32x4_t qb[NS];     // B operand: query row n, dims 8(4s+g)..+8
  f32x4_t o[NB];      // C layout: rows 4g+i, dim 16nb+n
  float m;            // running max (exp2 domain) of row n, same in all four lane groups
  float l;            // this lane's partial sum of row n's probabilities

  __device__ __forceinline__ void init() {
    #pragma unroll
    for (int nb = 0; nb < NB; ++nb) o[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    m = -INFINITY;
    l = 0.f;
  }

  // The PV B-operands of a 32-token tile from the wave's LDS tile vt ([32][D], chunk-swizzled):
  // for each 16-dim block, lane 16g + 4j + q of two transpose reads addresses row (16h + 4g + j),
  // dims 16nb + 4q..+3, which sit in logical chunk 2nb + q/2 of that row.
  __device__ __forceinline__ void read_v(const uint16_t* vt, int lane, u32x4_t (&vb)[NB]) const {
    const int g = lane >> 4, j = (lane >> 2) & 3, q = lane & 3;
    const int r0 = 4 * g + j, r1 = r0 + 16;
    const uint16_t* b0 = vt + r0 * D + 4 * (q & 1);
    const uint16_t* b1 = vt + r1 * D + 4 * (q & 1);
    const int z0 = v_swizzle<D>(r0), z1 = v_swizzle<D>(r1);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int lc = 2 * nb + (q >> 1);
      const uint2 lo = lds_read_tr16(b0 + 8 * (lc ^ z0));
      const uint2 hi = lds_read_tr16(b1 + 8 * (lc ^ z1));
      vb[nb] = u32x4_t{lo.x, lo.y, hi.x, hi.y};
    }
  }

  // Scores of a 32-token tile in the exp2 domain: s[u][i] = row n . token 16u+4g+i, -inf where
  // bit 4u+i of vmask is clear.
  __device__ __forceinline__ void scores(const u32x4_t (&ka)[2][NS], uint32_t vmask, float scale_log2,
                                         float (&s)[2][4]) const {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < NS; ++st) acc = mfma_16x16x32(ka[u][st], qb[st], acc);
      if (vmask == 0xFFu) {  // wave-uniform fast path for fully visible tiles
#pragma unroll
        for (int i = 0; i < 4; ++i) s[u][i] = acc[i] * scale_log2;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) s[u][i] = ((vmask >> (4 * u + i)) & 1u) ? acc[i] * scale_log2 : -INFINITY;
      }
    }
  }

  // Online-softmax step: updates m and l, returns the tile's probabilities as the PV A-operand
  // (bf16) and in a[i] the factor by which O row 4g+i must be rescaled; rescale = false (a
  // unset) when no row of the wave changed its maximum, so O needs no rescaling (wave-uniform).
  __device__ __forceinline__ u32x4_t softmax(const float (&s)[2][4], int lane, float (&a)[4],
                                             bool& rescale) {
    const int g = lane >> 4;
    float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                     fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
    mx = fmaxf(mx, lane_read(mx, lane ^ 16));
    mx = fmaxf(mx, lane_read(mx, lane ^ 32));
    const bool grow = mx > m + kLazyMax;  // lazy maximum
    const float m_new = grow ? mx : m;
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = grow ? fast_exp2(m - mx) : 1.f;
    float p[2][4], psum = 0.f;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) { p[u][i] = fast_exp2(s[u][i] - m_use); psum += p[u][i]; }
    l = l * alpha + psum;
    m = m_new;
    rescale = __builtin_amdgcn_ballot_w64(alpha != 1.f) != 0;
    if (rescale) {
      // O rows 4g+i take the factor of row 4g+i (held by lane 4g+i of every group)
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = lane_read(alpha, 4 * g + i);
    }
    return u32x4_t{pack_bf2(p[0][0], p[0][1]), pack_bf2(p[0][2], p[0][3]),
                   pack_bf2(p[1][0], p[1][1]), pack_bf2(p[1][2], p[1][3])};
  }

  // O block nb = O block nb * a + P V_nb (no rescaling when softmax() reported none).
  __device__ __forceinline__ void pv(const u32x4_t& pa, const u32x4_t& vb, const float (&a)[4], bool rescale,
                                     int nb) {
    f32x4_t c = o[nb];
    if (rescale) {
#pragma unroll
      for (int i = 0; i < 4; ++i) c[i] *= a[i];
    }
    o[nb] = mfma_16x16x32(pa, vb, c);
  }

  // One 32-token tile: ka = K A-operands of the two subtiles, vb = the V B-operands (read_v),
  // bit 4u+i of vmask says whether this lane's row n sees token 16u+4g+i.
  __device__ __forceinline__ void tile(const u32x4_t (&ka)[2][NS], uint32_t vmask,
                                       const u32x4_t (&vb)[NB], float scale_log2, int lane) {
    float s[2][4], a[4];
    bool rescale;
    scores(ka, vmask, scale_log2, s);
    const u32x4_t pa = softmax(s, lane, a, rescale);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) pv(pa, vb[nb], a, rescale, nb);
  }

  // Row n's total probability mass (sum of the four lane groups' partials).
  __device__ __forceinline__ float row_sum(int lane) const {
    float t = l + lane_read(l, lane ^ 16);
    return t + lane_read(t, lane ^ 32);
  }
};

// Page ids of a window of logical pages, staged in LDS once per work group.
constexpr int kPageWin = 512;

// Element offset of token t (its logical page lp = t / P lies in the staged window starting at
// lp0) for kv head h, branch-free; ok = false (and page 0 addressed) if the page id is out of
// range.
__device__ __forceinline__ uint64_t kv_offset_lds(const PagedKV& kv, const int32_t* ptab, int lp0,
                                                  int t, int h, bool& ok) {
  const int lp = (int)kv.pdiv.div((uint32_t)t);
  const int slot = t - lp * kv.page_size;
  const int page = ptab[lp - lp0];
  ok = (unsigned)page < (unsigned)kv.num_pages;
  const uint32_t pg = ok ? (uint32_t)page : 0u;
  return (uint64_t)pg * (uint32_t)kv.page_stride + (uint64_t)(uint32_t)slot * (uint32_t)kv.slot_stride +
         (uint64_t)(uint32_t)h * (uint32_t)kv.head_stride;
}

// One wave's loads for a 32-token tile: the K MFMA operands of both subtiles with their
// visibility ballots (registers), and the V rows, which go from HBM straight into the wave's
// LDS tile ([32][D], chunk-swizzled) without passing through registers. Tokens at or past `end`
// and tokens on out-of-range pages are invisible; their loads are clamped to valid addresses
// (an invisible row gets probability 0).
template <int D>
struct KVTile {
  static constexpr int NS = D / 32, CH = D / 8, RPI = 64 / CH, NVL = kTileTokens / RPI;
  u32x4_t ka[2][NS];
  uint64_t vis[2];

  // Row-independent visibility in tile()'s vmask form: bit 4u+i = token 16u+4g+i.
  __device__ __forceinline__ uint32_t vmask(int lane) const {
    const int g = lane >> 4;
    return (uint32_t)((vis[0] >> (4 * g)) & 15u) | ((uint32_t)((vis[1] >> (4 * g)) & 15u) << 4);
  }

  __device__ __forceinline__ void load(const PagedKV& kv, const int32_t* ptab, int lp0, int t0,
                                       int end, int kvh, int lane, uint16_t* vt) {
    const int n = lane & 15, g = lane >> 4;
#pragma unroll
    for (int i = 0; i < NVL; ++i) {
      const int r = RPI * i + lane / CH;
      bool ok;
      const uint64_t off = kv_offset_lds(kv, ptab, lp0, min(t0 + r, end - 1), kvh, ok);
      const int lc = (lane % CH) ^ v_swizzle<D>(r);
      __builtin_amdgcn_global_load_lds(kv.v + off + 8 * lc,
                                       (__attribute__((address_space(3))) void*)(vt + RPI * i * D),
                                       16, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int tok = t0 + 16 * u + n;
      bool ok;
      const uint16_t* kp = kv.k + kv_offset_lds(kv, ptab, lp0, min(tok, end - 1), kvh, ok);
#pragma unroll
      for (int s = 0; s < NS; ++s) ka[u][s] = ld16v(kp + 8 * (4 * s + g));
      vis[u] = __builtin_amdgcn_ballot_w64(tok < end && ok);
    }
  }
};

// ------------------------------------------------------------------------------ decode
// Grid (batch * splits * kv heads), one dimension: work group x takes the request of rank
// x / (splits * kv heads), split (x / kv heads) % splits, kv head x % kv heads. For batches of
// at most kRankMax requests the rank orders requests by attended length, longest first (ties
// by request index), so the longest requests' work groups are dispatched first and the short
// ones fill the tail; larger batches keep request order (rank = request). The split is derived
// on the device from the request's current kv length (chunks of ceil(kv_len / splits) rounded
// up to whole 32-token tiles, at least kMinChunk), and so is the rank, so a launch depends only
// on (batch, splits) and a captured graph replays correctly for any lengths.
// With one split the work group writes the output; otherwise it writes an fp32 partial output
// and its log2-sum-exp to slot x, and attn_merge_kernel combines the splits.
constexpr int kMinChunk = 128;
constexpr int kRankMax = 256;  // one request per thread of the work group

// The request of rank r (B <= kRankMax), with its kv length and first page-table entry. Every
// work group of the launch ranks the same lengths the same way, so together they cover each
// (request, split, kv head) once. lens: kRankMax ints of LDS.
__device__ __forceinline__ int request_of_rank(const PagedKV& kv, int B, int window_left, int r,
                                               int32_t* lens, int32_t* pick, int& kv_len, int& page0) {
  const int i = threadIdx.x;
  int kl = 0, li = -1;  // padding: below every length
  if (i < B) {
    kl = kv_length(kv, i);
    li = window_left >= 0 ? min(kl, window_left + 1) : kl;
  }
  lens[i] = li;
  __syncthreads();
  if (i < B) {
    int before = 0;  // requests ordered before i
    for (int k = 0; k < B; k += 4) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(lens + k);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int le = (int)v[e];
        before += le > li || (le == li && k + e < i);
      }
    }
    if (before == r) { pick[0] = i; pick[1] = kl; }
  }
  __syncthreads();
  const int b = uniform(pick[0]);
  kv_len = uniform(pick[1]);
  page0 = kv.indptr[b];
  return b;
}

__device__ __forceinline__ void split_range(int kv_len, int splits, int j, int& kv0, int& kv1) {
  int chunk = (kv_len + splits - 1) / splits;
  chunk = max(kMinChunk, (chunk + kTileTokens - 1) / kTileTokens * kTileTokens);
  kv0 = min(kv_len, j * chunk);
  kv1 = min(kv_len, kv0 + chunk);
}

template <int D>
__global__ __launch_bounds__(256) void attn_decode_kernel(
    const uint16_t* __restrict__ q, int64_t q_ts, int64_t q_hs, PagedKV kv, int B, int G, int Hq,
    float scale_log2, int splits, int window_left, uint16_t* __restrict__ out, int64_t o_ts,
    int64_t o_hs, float* __restrict__ part_o, float* __restrict__ part_lse,
    const float* __restrict__ sinks) {
  using W = WaveAttn<D>;
  constexpr int kVtile = kTileTokens * D;  // elements of one wave's V tile
  constexpr int kSmem = (4 * kVtile * 2 > 4 * 16 * (D + 2) * 4) ? 4 * kVtile * 2 : 4 * 16 * (D + 2) * 4;
  static_assert(kSmem >= kRankMax * 4, "the ranked lengths fit in the V tiles' LDS");
  __shared__ __attribute__((aligned(16))) char smem[kSmem];
  __shared__ int32_t rank_pick[2];

  const int Hkv = Hq / G;
  const int per = splits * Hkv;
  const int r = blockIdx.x / per, rem = blockIdx.x - r * per;
  const int j = rem / Hkv, kvh = rem - j * Hkv;
  int b = r, kv_len, page0;
  if (B <= kRankMax) {
    // the LDS holds the lengths until the first page window's barrier
    b = request_of_rank(kv, B, window_left, r, reinterpret_cast<int32_t*>(smem), rank_pick, kv_len, page0);
  } else {
    kv_len = kv_length(kv, b);
    page0 = kv.indptr[b];
  }
  const int slot = b * splits + j;
  const int lane = threadIdx.x & 63, w = uniform(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  // sliding window: the query (position kv_len - 1) sees positions >= kv_len - 1 - window_left
  const int ws = window_left >= 0 ? max(0, kv_len - 1 - window_left) : 0;
  int kv0, kv1;
  split_range(kv_len - ws, splits, j, kv0, kv1);
  kv0 += ws;
  kv1 += ws;

  W st;
  st.init();
  // query rows of this kv head: heads kvh*G + n (rows n >= G are zero)
  {
    const bool valid = n < G;
    const uint16_t* qp = q + (int64_t)b * q_ts + (int64_t)(kvh * G + (valid ? n : 0)) * q_hs;
    #pragma unroll
    for (int s = 0; s < W::NS; ++s) {
      const u32x4_t z = {0u, 0u, 0u, 0u};
      st.qb[s] = valid ? ld16v(qp + 8 * (4 * s + g)) : z;
    }
  }
  uint16_t* vt = reinterpret_cast<uint16_t*>(smem) + w * kVtile;
  __shared__ int32_t ptab[kPageWin];
  // kv tokens per page window: the pages any such run spans fit in kPageWin
  const int win = max(kTileTokens, (kPageWin - 2) * kv.page_size / kTileTokens * kTileTokens);
  for (int wt0 = kv0; wt0 < kv1; wt0 += win) {
    const int wt1 = min(kv1, wt0 + win);
    const int lp0 = (int)kv.pdiv.div((uint32_t)wt0);
    const int npg = (int)kv.pdiv.div((uint32_t)(wt1 - 1)) - lp0 + 1;
    __syncthreads();  // the previous window's lookups are done
    for (int i = threadIdx.x; i < npg; i += 256) ptab[i] = kv.indices[page0 + lp0 + i];
    __syncthreads();
    // each wave takes every fourth tile; the next tile's loads are issued before the current
    // tile's MFMA/softmax work so HBM latency overlaps compute
    // Each wave takes every fourth tile. Two tile slots alternate (no register copies, which
    // would force a wait on the in-flight loads): the next tile's loads are issued before the
    // current tile's MFMA/softmax work, so HBM latency overlaps compute.
    int t0 = wt0 + kTileTokens * w;
    if (t0 < wt1) {
      // Two K register slots alternate (no copies, which would force waits on loads in
      // flight); V has one LDS tile. Each step: wait for the current tile's loads, move its V
      // from LDS into registers, issue the next tile's loads (V into the now free LDS tile),
      // then run the current tile's MFMA/softmax work while they stream in.
      KVTile<D> ta, tb;
      u32x4_t vb[W::NB];
      ta.load(kv, ptab, lp0, t0, wt1, kvh, lane, vt);
      for (;;) {
        wait_vmcnt<0>();
        st.read_v(vt, lane, vb);
        wait_lgkmcnt0();
        const bool more_b = t0 + 4 * kTileTokens < wt1;
        if (more_b) tb.load(kv, ptab, lp0, t0 + 4 * kTileTokens, wt1, kvh, lane, vt);
        st.tile(ta.ka, ta.vmask(lane), vb, scale_log2, lane);
        if (!more_b) break;
        t0 += 4 * kTileTokens;
        wait_vmcnt<0>();
        st.read_v(vt, lane, vb);
        wait_lgkmcnt0();
        const bool more_a = t0 + 4 * kTileTokens < wt1;
        if (more_a) ta.load(kv, ptab, lp0, t0 + 4 * kTileTokens, wt1, kvh, lane, vt);
        st.tile(tb.ka, tb.vmask(lane), vb, scale_log2, lane);
        if (!more_a) break;
        t0 += 4 * kTileTokens;
      }
    }
  }
  const float lsum = st.row_sum(lane);

  // merge the four waves through LDS: m[4][16], l[4][16], o[4][16][D] (fp32)
  __syncthreads();
  float* ms = reinterpret_cast<float*>(smem);
  float* ls = ms + 4 * 16;
  float* os = ls + 4 * 16;
  if (g == 0) { ms[w * 16 + n] = st.m; ls[w * 16 + n] = lsum; }
  #pragma unroll
  for (int nb = 0; nb < W::NB; ++nb)
    #pragma unroll
    for (int i = 0; i < 4; ++i) os[(w * 16 + 4 * g + i) * D + 16 * nb + n] = st.o[nb][i];
  __syncthreads();
  constexpr int CH = D / 8;
  for (int u = threadIdx.x; u < G * CH; u += 256) {
    const int row = u / CH, c = u % CH;
    float M = -INFINITY;
    #pragma unroll
    for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, ms[ww * 16 + row]);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float L = 0.f;
    if (M != -INFINITY) {
      #pragma unroll
      for (int ww = 0; ww < 4; ++ww) {
        const float f = fast_exp2(ms[ww * 16 + row] - M);
        L += ls[ww * 16 + row] * f;
        const float* src = os + (ww * 16 + row) * D + 8 * c;
        #pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += src[e] * f;
      }
    }
    const int hq = kvh * G + row;
    // the sink joins the denominator once, after the splits are merged
    if (splits == 1 && M != -INFINITY) L += sink_mass(sinks, hq, M);
    const float inv = L > 0.f ? 1.f / L : 0.f;
    #pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= inv;
    if (splits == 1) {
      st16(out + (int64_t)b * o_ts + (int64_t)hq * o_hs + 8 * c, pack8(acc));
    } else {
      float* dst = part_o + ((int64_t)slot * Hq + hq) * D + 8 * c;
      #pragma unroll
      for (int e = 0; e < 8; ++e) dst[e] = acc[e];
      if (c == 0) part_lse[(int64_t)slot * Hq + hq] = L > 0.f ? M + log2f(L) : -INFINITY;
    }
  }
}

// Combines the `splits` partial results of each (request, head).
template <int D>
__global__ __launch_bounds__(64) void attn_merge_kernel(int B, int Hq, int splits,
                                                        const float* __restrict__ part_o,
                                                        const float* __restrict__ part_lse,
                                                        uint16_t* __restrict__ out, int64_t o_ts,
                                                        int64_t o_hs, const float* __restrict__ sinks) {
  constexpr int CH = D / 8;
  const int b = blockIdx.x;
  const int hq = blockIdx.y * (64 / CH) + threadIdx.x / CH;
  const int c = threadIdx.x % CH;
  if (b >= B || hq >= Hq) return;
  const int s0 = b * splits, ns = splits;
  float M = -INFINITY;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, part_lse[(int64_t)(s0 + s) * Hq + hq]);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float L = 0.f;
  if (M != -INFINITY) {
    for (int s = 0; s < ns; ++s) {
      const float f = fast_exp2(part_lse[(int64_t)(s0 + s) * Hq + hq] - M);
      L += f;
      const float* src = part_o + ((int64_t)(s0 + s) * Hq + hq) * D + 8 * c;
      #pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += src[e] * f;
    }
  }
  if (M != -INFINITY) L += sink_mass(sinks, hq, M);
  const float inv = L > 0.f ? 1.f / L : 0.f;
  #pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] *= inv;
  st16(out + (int64_t)b * o_ts + (int64_t)hq * o_hs + 8 * c, pack8(acc));
}


// ------------------------------------------------------------------------------ prefill
// Work item: request b, first packed query row row0 (row R = query token R / G, head R % G of
// the kv head's group). A work group of prefill_waves<D> waves owns prefill_rows<D> rows
// (prefill_row_tiles<D> 16-row MFMA row tiles per wave) and streams the request's kv tokens in 32-token tiles: the four waves load each K
// and V tile cooperatively (three tiles ahead through registers, then into LDS, chunk-swizzled,
// double-buffered),
// then every wave reads the K and V MFMA operands it needs into registers before the next
// tile's loads are issued, and runs both row tiles against them.
// Visibility: mode 0 every cached position, 1 causal (t <= kv_len - qo_len + i), 2 the custom
// mask, bit-packed by attn_pack_mask_kernel: query token i of request b reads 32-bit word
// w (kv positions 32w..32w+31) at packed + word_off[b] + i * ceil(kv_len / 32) + w.
// Work-group shape of attn_prefill_kernel: 4 waves of two 16-row MFMA row tiles (one for D = 256,
// whose accumulators would not fit twice). Head dim 128 runs attn_prefill32_kernel (32 rows per
// wave, same 128-row work items).
template <int D>
constexpr int prefill_waves() { return 4; }
template <int D>
constexpr int prefill_row_tiles() { return D == 256 ? 1 : 2; }
template <int D>
constexpr int prefill_min_waves() { return D == 256 ? 1 : 2; }
template <int D>
constexpr int prefill_rows() { return 16 * prefill_waves<D>() * prefill_row_tiles<D>(); }
constexpr int kPlanHeader = 16;  // plan words before the items: [0] items, [1] batch, [2] rows per item
// Plan words the head-dim-128 kernel uses as counters: the next unit of each XCD's queue, and
// the work groups that have finished (the last one sets all nine back to zero).
constexpr int kPlanQueueWord = 8, kPlanDoneWord = 7;
// words per work item: request b, first packed row, and the request's q0 (first query token),
// qo_len, kv_len and first page-table slot, so the kernels' prologue reads one 32-byte item
// instead of chasing b through qo_indptr / kv_indptr / kv_last_page_len; two pad words
constexpr int kPlanItemWords = 8;

// XCD-aware order of the prefill grid: work groups are dispatched round-robin over the 8 XCDs
// (id mod 8), each with its own L2, so XCD x takes the contiguous run [x * per, (x + 1) * per) of
// the (kv head, item) units. The plan lists each request's items together, so the work groups an
// XCD runs at one time mostly read the same request's K/V prefix through one L2. Returns the
// unit's plan item and sets kvh, or nullptr for the padding work groups past the last unit.
__device__ __forceinline__ const int32_t* prefill_unit(const int32_t* plan, int n_items, int n_kv_heads,
                                                       int& kvh) {
  const int units = n_items * n_kv_heads, per = (units + 7) / 8;
  const int u = (int)(blockIdx.x & 7u) * per + (int)(blockIdx.x >> 3);
  if (u >= units) return nullptr;
  kvh = u / n_items;
  return plan + kPlanHeader + kPlanItemWords * (u - kvh * n_items);
}

// attn_mask_extent_kernel marks a query token whose mask row is exactly causal (positions
// 0..kv_len - qo_len + i, nothing else) with this bit of its extent.
constexpr int kExtentCausal = 1 << 30;

// Custom-mask prologue: the furthest position any of the work group's nrows rows (from row0) can
// see, and whether every one of those rows' masks is exactly causal (then the causal path serves
// them without reading mask words). Every thread of the work group calls it.
__device__ __forceinline__ void mask_rows_extent(const int32_t* __restrict__ extent, int q0, int row0, int rows,
                                                 int G, int nrows, int& ext, bool& causal) {
  __shared__ int s_ext, s_mixed;
  if (threadIdx.x == 0) { s_ext = 0; s_mixed = 0; }
  __syncthreads();
  const int r = row0 + (int)threadIdx.x;
  if ((int)threadIdx.x < nrows && r < rows) {
    const int e = extent[q0 + r / G];
    atomicMax(&s_ext, e & ~kExtentCausal);
    if (!(e & kExtentCausal)) atomicOr(&s_mixed, 1);
  }
  __syncthreads();
  ext = s_ext;
  causal = s_mixed == 0;
}

// A plan made for another head_dim (its rows per item differ) cannot drive this kernel: every
// work group fills the whole output (the plan's tokens, all q heads) with NaN instead, so the
// mistake shows in the result rather than leaving the output unwritten.
template <int D>
__device__ void prefill_plan_mismatch(const int32_t* __restrict__ plan, const int32_t* __restrict__ qo_indptr,
                                      int Hq, uint16_t* __restrict__ out, int64_t o_ts, int64_t o_hs) {
  const int t0 = qo_indptr[0], T = qo_indptr[plan[1]] - t0;
  constexpr int CH = D / 8;  // 16-byte chunks per head row
  const int64_t n = (int64_t)T * Hq * CH;
  const uint4 nan4 = make_uint4(0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u);
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / (Hq * CH);
    const int h = (int)(i / CH % Hq), c = (int)(i % CH);
    *reinterpret_cast<uint4*>(out + (t0 + t) * o_ts + (int64_t)h * o_hs + 8 * c) = nan4;
  }
}

template <int D>
__global__ __launch_bounds__(64 * prefill_waves<D>(), prefill_min_waves<D>()) void attn_prefill_kernel(
    const uint16_t* __restrict__ q, int64_t q_ts, int64_t q_hs, PagedKV kv,
    const int32_t* __restrict__ qo_indptr, int G, float scale_log2, const int32_t* __restrict__ plan,
    int n_items, int n_kv_heads,
    int mode_in, int window_left, const uint32_t* __restrict__ packed,
    const int64_t* __restrict__ word_off, const int32_t* __restrict__ extent,
    uint16_t* __restrict__ out, int64_t o_ts, int64_t o_hs, const float* __restrict__ sinks) {
  using W = WaveAttn<D>;
  constexpr int NS = W::NS, NB = W::NB, CH = D / 8, RPI = 64 / CH;
  constexpr int RT = prefill_row_tiles<D>(), kPrefillRows = prefill_rows<D>();
  constexpr int NW = prefill_waves<D>(), NT = 64 * NW;  // waves, threads
  constexpr int TILE = kTileTokens * D;  // elements of one K or V tile
  constexpr int kSmemLoop = 2 * 2 * TILE * 2;
  constexpr int kSmemOut = kPrefillRows * D * 2;
  constexpr int kSmem = kSmemLoop > kSmemOut ? kSmemLoop : kSmemOut;
  __shared__ __attribute__((aligned(16))) char smem[kSmem];
  __shared__ int32_t ptab[kPageWin];

  if (plan[2] != kPrefillRows) {
    prefill_plan_mismatch<D>(plan, qo_indptr, G * n_kv_heads, out, o_ts, o_hs);
    return;
  }
  int kvh;
  const int32_t* item = prefill_unit(plan, n_items, n_kv_heads, kvh);
  if (!item) return;  // padding work group
  const int b = item[0], row0 = item[1], q0 = item[2], qo_len = item[3], kv_len = item[4];
  const int page0 = item[5];
  const int lane = threadIdx.x & 63, w = uniform(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int rows = qo_len * G;
  int mode = mode_in, mext = 0;  // a custom mask that is causal for all the rows: the causal path
  if (mode_in == 2) {
    bool causal;
    mask_rows_extent(extent, q0, row0, rows, G, kPrefillRows, mext, causal);
    mode = uniform(causal ? 1 : 2);  // wave-uniform (a scalar register), like the argument
  }

  // this lane's query rows (row n of each of the wave's row tiles)
  W st[RT];
  int lim[RT], tok[RT], lo[RT];  // visible positions of the row: lo..lim (and the mask)
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    st[rt].init();
    const int R = row0 + 16 * RT * w + 16 * rt + n;
    const bool valid = R < rows;
    const int i = valid ? R / G : 0, hg = valid ? R - i * G : 0;
    tok[rt] = i;
    lim[rt] = !valid ? -1 : mode == 1 ? min(kv_len - qo_len + i, kv_len - 1) : kv_len - 1;
    lo[rt] = window_left >= 0 ? kv_len - qo_len + i - window_left : 0;
    const uint16_t* qp = q + (int64_t)(q0 + i) * q_ts + (int64_t)(kvh * G + hg) * q_hs;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const u32x4_t z = {0u, 0u, 0u, 0u};
      st[rt].qb[s] = valid ? ld16v(qp + 8 * (4 * s + g)) : z;
    }
  }
  // kv positions any row of this work group can see (mode 2: the furthest set mask bit of its
  // rows' query tokens, from attn_mask_extent_kernel)
  const int last_row = min(rows, row0 + kPrefillRows) - 1;
  int kv_end = mode == 1 ? min(kv_len, kv_len - qo_len + last_row / G + 1) : kv_len;
  if (mode == 2) kv_end = min(kv_len, mext);
  // sliding window: no row of the work group sees positions before its first row's window
  // (tiles start 32-aligned so mask words line up)
  const int kv_begin = window_left >= 0 ? max(0, kv_len - qo_len + row0 / G - window_left) & ~31 : 0;
  int wave_lo = 0;  // the largest window start of the wave's rows (uniform)
  if (window_left >= 0) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) wave_lo = max(wave_lo, lim[rt] < 0 ? 0 : lo[rt]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) wave_lo = max(wave_lo, __builtin_amdgcn_ds_bpermute((lane ^ o) << 2, wave_lo));
    wave_lo = uniform(wave_lo);
  }
  // mode 2: this lane's rows' mask words; modes 0/1: the last kv position every row of the wave
  // sees (tiles ending at or before it need no per-element visibility test)
  const uint32_t* mword[RT];
  const int nw = (kv_len + 31) / 32;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) mword[rt] = mode == 2 ? packed + word_off[b] + (int64_t)tok[rt] * nw : nullptr;
  int wave_lim = 0x7fffffff;
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) wave_lim = min(wave_lim, lim[rt] < 0 ? 0x7fffffff : lim[rt]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) wave_lim = min(wave_lim, __builtin_amdgcn_ds_bpermute((lane ^ o) << 2, wave_lim));
  wave_lim = uniform(wave_lim);
  __shared__ int window_bad;
  __shared__ uint32_t mwt[2][RT][NT];  // mode 2: mask words of the tiles in LDS, per lane

  uint16_t* kt = reinterpret_cast<uint16_t*>(smem);  // [2 buffers][K, V][32][D]
  constexpr int WR = kTileTokens / NW;  // rows of each K / V tile one wave loads
  constexpr int NL = WR / RPI;          // load instructions per wave for them
  static_assert(NL >= 1 && WR % RPI == 0, "tile rows per wave");
  // A tile in flight in registers: this wave's rows 8w..8w+7 of K and V (chunk-swizzled as they
  // will sit in LDS).
  struct Slot { u32x4_t k[NL], v[NL]; uint32_t mw[RT]; };
  const int win = max(kTileTokens, (kPageWin - 2) * kv.page_size / kTileTokens * kTileTokens);
  for (int wt0 = kv_begin; wt0 < kv_end; wt0 += win) {
    const int wt1 = min(kv_end, wt0 + win);
    const int lp0 = (int)kv.pdiv.div((uint32_t)wt0);
    const int npg = (int)kv.pdiv.div((uint32_t)(wt1 - 1)) - lp0 + 1;
    const int ntiles = (wt1 - wt0 + kTileTokens - 1) / kTileTokens;
    if (threadIdx.x == 0) window_bad = 0;
    __syncthreads();  // the previous window's lookups and LDS tiles are done
    for (int i = threadIdx.x; i < npg; i += NT) {
      const int pg = kv.indices[page0 + lp0 + i];
      ptab[i] = pg;
      if ((unsigned)pg >= (unsigned)kv.num_pages) window_bad = 1;
    }
    __syncthreads();
    const bool all_pages_ok = window_bad == 0;
    auto gload = [&](Slot& sl, int tile) {
      const int t0 = wt0 + tile * kTileTokens;
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        const int r = WR * w + RPI * i + lane / CH;
        bool ok;
        const uint64_t off = kv_offset_lds(kv, ptab, lp0, min(t0 + r, wt1 - 1), kvh, ok);
        sl.k[i] = ld16v(kv.k + off + 8 * ((lane % CH) ^ chunk_swizzle<D>(r)));
        sl.v[i] = ld16v(kv.v + off + 8 * ((lane % CH) ^ v_swizzle<D>(r)));
      }
      if (mode == 2) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) sl.mw[rt] = mword[rt][t0 >> 5];
      }
    };
    auto lwrite = [&](const Slot& sl, int tile) {
      uint16_t* kd = kt + (tile & 1) * 2 * TILE;
      if (mode == 2) {  // each lane keeps its own rows' mask words with the tile (no sharing)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) mwt[tile & 1][rt][threadIdx.x] = sl.mw[rt];
      }
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        *reinterpret_cast<u32x4_t*>(kd + (WR * w + RPI * i) * D + 8 * lane) = sl.k[i];
        *reinterpret_cast<u32x4_t*>(kd + TILE + (WR * w + RPI * i) * D + 8 * lane) = sl.v[i];
      }
    };
    auto compute = [&](int tile) {
      const int t0 = wt0 + tile * kTileTokens;
      const uint16_t* kd = kt + (tile & 1) * 2 * TILE;
      // tokens of this tile on valid pages (bit r = token t0 + r); tested only in windows that
      // hold an out-of-range page id
      uint64_t tv = 0xffffffffull;
      if (!all_pages_ok) {
        bool pok = false;
        if (lane < kTileTokens && t0 + lane < wt1) kv_offset_lds(kv, ptab, lp0, t0 + lane, kvh, pok);
        tv = __builtin_amdgcn_ballot_w64(pok);
      }
      const bool full = mode != 2 && all_pages_ok && t0 + kTileTokens - 1 <= wave_lim && t0 >= wave_lo;
      u32x4_t ka[2][NS];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int r = 16 * u + n;
        const int z = chunk_swizzle<D>(r);
#pragma unroll
        for (int s = 0; s < NS; ++s)
          ka[u][s] = *reinterpret_cast<const u32x4_t*>(kd + r * D + 8 * ((4 * s + g) ^ z));
      }
      u32x4_t pa[RT];
      float a[RT][4];
      bool rs[RT];
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        uint32_t vm = 0xFFu;
        if (mode == 2) {
          // bit 16u+4g+i of the row's word is token t0+16u+4g+i
          const uint32_t mw = mwt[tile & 1][rt][threadIdx.x] & (uint32_t)tv;
          vm = ((mw >> (4 * g)) & 15u) | (((mw >> (16 + 4 * g)) & 15u) << 4);
          if (lim[rt] < 0) vm = 0;
        } else if (!full) {
          vm = 0;
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int r = 16 * u + 4 * g + i;
              vm |= (uint32_t)(t0 + r <= lim[rt] && ((tv >> r) & 1ull)) << (4 * u + i);
            }
        }
        if (t0 < wave_lo) {  // the tile crosses some row's window start
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (t0 + 16 * u + 4 * g + i < lo[rt]) vm &= ~(1u << (4 * u + i));
        }
        if (__builtin_amdgcn_ballot_w64(vm != 0xFFu) == 0) vm = 0xFFu;  // keep the fast path visible
        float sc[2][4];
        st[rt].scores(ka, vm, scale_log2, sc);
        pa[rt] = st[rt].softmax(sc, lane, a[rt], rs[rt]);
      }
      // PV: the V operand of each 16-dim block comes straight from LDS (transpose reads)
      const int j = (lane >> 2) & 3, qq = lane & 3;
      const int r0 = 4 * g + j, r1 = r0 + 16;
      const uint16_t* b0 = kd + TILE + r0 * D + 4 * (qq & 1);
      const uint16_t* b1 = kd + TILE + r1 * D + 4 * (qq & 1);
      const int z0 = v_swizzle<D>(r0), z1 = v_swizzle<D>(r1);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int lc = 2 * nb + (qq >> 1);
        const uint2 lo = lds_read_tr16(b0 + 8 * (lc ^ z0));
        const uint2 hi = lds_read_tr16(b1 + 8 * (lc ^ z1));
        const u32x4_t vb = {lo.x, lo.y, hi.x, hi.y};
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) st[rt].pv(pa[rt], vb, a[rt], rs[rt], nb);
      }
    };
    // Two register slots alternate (no copies, which would force waits on loads in flight):
    // tile k+3's loads are issued while tile k is computed and land in LDS two steps later.
    Slot sa, sb;
    gload(sa, 0);
    if (ntiles > 1) gload(sb, 1);
    lwrite(sa, 0);
    if (ntiles > 2) gload(sa, 2);
    __syncthreads();
    for (int k = 0;;) {
      compute(k);
      if (k + 1 < ntiles) {
        lwrite(sb, k + 1);
        if (k + 3 < ntiles) gload(sb, k + 3);
      }
      __syncthreads();
      if (++k >= ntiles) break;
      compute(k);
      if (k + 1 < ntiles) {
        lwrite(sa, k + 1);
        if (k + 3 < ntiles) gload(sa, k + 3);
      }
      __syncthreads();
      if (++k >= ntiles) break;
    }
  }

  // normalise and stage the bf16 rows in LDS ([kPrefillRows][D]), then write 16-byte chunks
  float inv[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    float L = st[rt].row_sum(lane);
    const int R = row0 + 16 * RT * w + 16 * rt + n;
    if (sinks && R < rows) L += sink_mass(sinks, kvh * G + R % G, st[rt].m);
    inv[rt] = L > 0.f ? 1.f / L : 0.f;
  }
  __syncthreads();
  uint16_t* ot = reinterpret_cast<uint16_t*>(smem);
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float f = lane_read(inv[rt], 4 * g + i);
      const int row = 16 * RT * w + 16 * rt + 4 * g + i;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) ot[row * D + 16 * nb + n] = to_bf1(st[rt].o[nb][i] * f);
    }
  __syncthreads();
  for (int u = threadIdx.x; u < kPrefillRows * CH; u += NT) {
    const int row = u / CH, c = u % CH;
    const int R = row0 + row;
    if (R >= rows) continue;
    const int i = R / G, hg = R - i * G;
    st16(out + (int64_t)(q0 + i) * o_ts + (int64_t)(kvh * G + hg) * o_hs + 8 * c,
         *reinterpret_cast<const uint4*>(ot + row * D + 8 * c));
  }
}


// ------------------------------------------------------------------------------ prefill, D = 128
// The same work items, visibility rules, K/V tile pipeline and masks as attn_prefill_kernel, with
// the products on v_mfma_f32_32x32x16_bf16 and the output computed transposed:
//   S^T = K Q^T    A = 32 kv tokens x 16 dims (lane (t, kg): token t's dims 8(2s+kg)..+8 at
//                  step s, from LDS), B = 32 query rows (lane (r, kg): row r, the same dims)
//   O^T = V^T P^T  A = 32 dims x 16 tokens (two transpose reads of 4 V rows each),
//                  B = P^T: lane (r, kg) holds row r's probabilities of tokens
//                  16j + 8(e/4) + 4kg + e%4, exactly 8 consecutive registers of S^T's C layout
// so every lane owns one query row r = lane % 32 in both products: its running max, sum and
// rescale factor are its own (one exchange with lane ^ 32 for the max), and no factor has to be
// broadcast to other lanes. Each wave owns 32 rows; a work group of 4 waves, 128 rows.
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16_t mfma_32x32x16(const u32x4_t& a, const u32x4_t& b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Scheduling group: the next `n` instructions of class `mask` (0x8 MFMA, 0x100 LDS read).
#define sched_group(mask, n) __builtin_amdgcn_sched_group_barrier((mask), (n), 0)

// V-row swizzle for this kernel's transpose reads: one read takes 4 consecutive rows x 4 chunks
// per half-wave, so rows r..r+3 XOR chunk bits 2-3 with r mod 4.
__device__ __forceinline__ int v32_swizzle(int r) { return (r & 3) << 2; }


template <int D>
__global__ __launch_bounds__(256, 2) void attn_prefill32_kernel(
    const uint16_t* __restrict__ q, int64_t q_ts, int64_t q_hs, PagedKV kv,
    const int32_t* __restrict__ qo_indptr, int G, float scale_log2, const int32_t* __restrict__ plan,
    int n_items, int n_kv_heads,
    int mode_in, int window_left, const uint32_t* __restrict__ packed,
    const int64_t* __restrict__ word_off, const int32_t* __restrict__ extent,
    uint16_t* __restrict__ out, int64_t o_ts, int64_t o_hs, const float* __restrict__ sinks) {
  static_assert(D == 128, "32x32 prefill is built for head_dim 128");
  constexpr int NS = D / 16;  // QK k-steps
  constexpr int NB = D / 32;  // 32-dim output blocks
  constexpr int CH = D / 8, RPI = 64 / CH;
  constexpr int kRows = 128, NT = 256;
  constexpr int TILE = kTileTokens * D;
  __shared__ __attribute__((aligned(16))) char smem[2 * 2 * TILE * 2];
  __shared__ int32_t ptab[kPageWin];
  __shared__ int window_bad;
  __shared__ uint32_t mwt[2][NT];

  // Persistent: each work group takes (kv head, item) units from its XCD's queue until every
  // queue is empty. XCD x's queue is the contiguous run [x * per, (x + 1) * per) of the units, in
  // plan order (each request's items together), so the work groups of one XCD share the K/V
  // prefix they read through its L2; a work group whose queue is empty takes from the others.
  if (plan[2] != kRows) {
    prefill_plan_mismatch<D>(plan, qo_indptr, G * n_kv_heads, out, o_ts, o_hs);
    return;
  }
  int32_t* counters = const_cast<int32_t*>(plan);
  __shared__ int s_unit;
  const int units = n_items * n_kv_heads, per = (units + 7) / 8;
  const int xcd = (int)(__builtin_amdgcn_s_getreg((20) | (0 << 6) | ((4 - 1) << 11)) & 7);  // HW_REG_XCC_ID
  int queue = 0;
  for (;;) {
  __syncthreads();  // the previous unit's LDS use (and s_unit) is done
  if (threadIdx.x == 0) {
    int u = -1;
    for (; queue < 8 && u < 0; ) {
      const int x = (xcd + queue) & 7;
      const int n = min(per, units - x * per);
      const int i = atomicAdd(&counters[kPlanQueueWord + x], 1);
      if (i < n) u = x * per + i; else ++queue;
    }
    s_unit = u;
  }
  __syncthreads();
  const int u = s_unit;
  if (u < 0) break;
  const int kvh = u / n_items;
  const int32_t* item = plan + kPlanHeader + kPlanItemWords * (u - kvh * n_items);
  const int b = item[0], row0 = item[1], q0 = item[2], qo_len = item[3], kv_len = item[4];
  const int page0 = item[5];
  const int lane = threadIdx.x & 63, w = uniform(threadIdx.x >> 6);
  const int r32 = lane & 31, kg = lane >> 5;
  const int rows = qo_len * G;
  int mode = mode_in, mext = 0;  // a custom mask that is causal for all the rows: the causal path
  if (mode_in == 2) {
    bool causal;
    mask_rows_extent(extent, q0, row0, rows, G, kRows, mext, causal);
    mode = uniform(causal ? 1 : 2);  // wave-uniform (a scalar register), like the argument
  }

  // this lane's query row
  const int R = row0 + 32 * w + r32;
  const bool valid = R < rows;
  const int tok = valid ? R / G : 0, hg = valid ? R - tok * G : 0;
  const int lim = !valid ? -1 : mode == 1 ? min(kv_len - qo_len + tok, kv_len - 1) : kv_len - 1;
  const int lo = window_left >= 0 ? kv_len - qo_len + tok - window_left : 0;
  u32x4_t qb[NS];
  {
    const uint16_t* qp = q + (int64_t)(q0 + tok) * q_ts + (int64_t)(kvh * G + hg) * q_hs;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const u32x4_t z = {0u, 0u, 0u, 0u};
      qb[s] = valid ? ld16v(qp + 8 * (2 * s + kg)) : z;
    }
  }
  f32x16_t o[NB];
#pragma unroll
  for (int bb = 0; bb < NB; ++bb)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[bb][i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  const int last_row = min(rows, row0 + kRows) - 1;
  int kv_end = mode == 1 ? min(kv_len, kv_len - qo_len + last_row / G + 1) : kv_len;
  if (mode == 2) kv_end = min(kv_len, mext);
  const int kv_begin = window_left >= 0 ? max(0, kv_len - qo_len + row0 / G - window_left) & ~31 : 0;
  const int nw = (kv_len + 31) / 32;
  const uint32_t* mword = mode == 2 ? packed + word_off[b] + (int64_t)tok * nw : nullptr;
  // uniform bounds of the wave's rows: tiles inside [wave_lo, wave_lim] need no per-element test
  int wave_lim = valid ? lim : 0x7fffffff, wave_lo = valid ? lo : 0;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    wave_lim = min(wave_lim, __builtin_amdgcn_ds_bpermute((lane ^ off) << 2, wave_lim));
    wave_lo = max(wave_lo, __builtin_amdgcn_ds_bpermute((lane ^ off) << 2, wave_lo));
  }
  wave_lim = uniform(wave_lim);
  wave_lo = uniform(wave_lo);

  uint16_t* kt = reinterpret_cast<uint16_t*>(smem);  // [2 buffers][K, V][32][D]
  constexpr int WR = kTileTokens / 4;  // rows of each K / V tile one wave loads
  constexpr int NL = WR / RPI;
  struct Slot { u32x4_t k[NL], v[NL]; uint32_t mw; };
  const int win = max(kTileTokens, (kPageWin - 2) * kv.page_size / kTileTokens * kTileTokens);
  for (int wt0 = kv_begin; wt0 < kv_end; wt0 += win) {
    const int wt1 = min(kv_end, wt0 + win);
    const int lp0 = (int)kv.pdiv.div((uint32_t)wt0);
    const int npg = (int)kv.pdiv.div((uint32_t)(wt1 - 1)) - lp0 + 1;
    const int ntiles = (wt1 - wt0 + kTileTokens - 1) / kTileTokens;
    if (threadIdx.x == 0) window_bad = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < npg; i += NT) {
      const int pg = kv.indices[page0 + lp0 + i];
      ptab[i] = pg;
      if ((unsigned)pg >= (unsigned)kv.num_pages) window_bad = 1;
    }
    __syncthreads();
    const bool all_pages_ok = window_bad == 0;
    auto gload = [&](Slot& sl, int tile) {
      const int t0 = wt0 + tile * kTileTokens;
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        const int r = WR * w + RPI * i + lane / CH;
        bool ok;
        const uint64_t off = kv_offset_lds(kv, ptab, lp0, min(t0 + r, wt1 - 1), kvh, ok);
        sl.k[i] = ld16v(kv.k + off + 8 * ((lane % CH) ^ chunk_swizzle<D>(r)));
        sl.v[i] = ld16v(kv.v + off + 8 * ((lane % CH) ^ v32_swizzle(r)));
      }
      if (mode == 2) sl.mw = mword[t0 >> 5];
    };
    auto lwrite = [&](const Slot& sl, int tile) {
      uint16_t* kd = kt + (tile & 1) * 2 * TILE;
      if (mode == 2) mwt[tile & 1][threadIdx.x] = sl.mw;
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        *reinterpret_cast<u32x4_t*>(kd + (WR * w + RPI * i) * D + 8 * lane) = sl.k[i];
        *reinterpret_cast<u32x4_t*>(kd + TILE + (WR * w + RPI * i) * D + 8 * lane) = sl.v[i];
      }
    };
    auto compute = [&](int tile) {
      const int t0 = wt0 + tile * kTileTokens;
      const uint16_t* kd = kt + (tile & 1) * 2 * TILE;
      // S^T: token r32 of the tile against this lane group's 32 rows
      f32x16_t sacc;
#pragma unroll
      for (int i = 0; i < 16; ++i) sacc[i] = 0.f;
      {
        const int z = chunk_swizzle<D>(r32);
        // K operands read four k-steps ahead of the MFMA chain. The schedule is pinned: left to
        // itself the compiler reads two ahead and exposes the LDS latency four times per tile.
        u32x4_t kr[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) kr[s] = *reinterpret_cast<const u32x4_t*>(kd + r32 * D + 8 * ((2 * s + kg) ^ z));
#pragma unroll
        for (int s = 0; s < NS; ++s) sacc = mfma_32x32x16(kr[s], qb[s], sacc);
        sched_group(0x100, 4);
#pragma unroll
        for (int s = 0; s < NS - 4; ++s) { sched_group(0x008, 1); sched_group(0x100, 1); }
        sched_group(0x008, 4);
      }
      // visibility of token tt(i) = 8(i/4) + 4kg + i%4 for this lane's row: mask bits by shifts,
      // then the per-element bounds only in tiles that cross a row's limit or window start
      uint32_t vis = 0xffffu;
      if (mode == 2) {
        const uint32_t mw = mwt[tile & 1][threadIdx.x];
        vis = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) vis |= ((mw >> (8 * c + 4 * kg)) & 15u) << (4 * c);
      }
      if (!all_pages_ok || t0 + kTileTokens - 1 > wave_lim || t0 < wave_lo) {
        uint64_t tv = 0xffffffffull;
        if (!all_pages_ok) {
          bool pok = false;
          if (lane < kTileTokens && t0 + lane < wt1) kv_offset_lds(kv, ptab, lp0, t0 + lane, kvh, pok);
          tv = __builtin_amdgcn_ballot_w64(pok);
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int tt = 8 * (i >> 2) + 4 * kg + (i & 3), t = t0 + tt;
          if (!(t <= lim && t >= lo && ((tv >> tt) & 1ull))) vis &= ~(1u << i);
        }
      }
      // Scores stay raw (q.k) until the exponent, where one fma applies the scale: the row maximum
      // is taken over raw scores, negated when the scale is negative (a uniform branch), with
      // hidden entries set to the raw value that scales to -inf (the scale is never 0 here).
      const bool neg = scale_log2 < 0.f;
      const bool masked = __builtin_amdgcn_ballot_w64(vis != 0xffffu) != 0;
      if (masked) {
        const float hidden = neg ? INFINITY : -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) sacc[i] = ((vis >> i) & 1u) ? sacc[i] : hidden;
      }
      float mx = -INFINITY;
      if (!neg) {
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sacc[i]);
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, -sacc[i]);
      }
      mx = fmaxf(mx, lane_read(mx, lane ^ 32)) * fabsf(scale_log2);
      // lazy maximum (kLazyMax)
      if (__builtin_amdgcn_ballot_w64(mx > m_run + kLazyMax) != 0) {
        const bool grow = mx > m_run + kLazyMax;
        const float alpha = grow ? fast_exp2(m_run - mx) : 1.f;
        if (grow) m_run = mx;
        l_run *= alpha;
#pragma unroll
        for (int bb = 0; bb < NB; ++bb)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[bb][i] *= alpha;
      }
      const float m_use = m_run == -INFINITY ? 0.f : m_run;
      float sc[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) sc[i] = fast_exp2(fmaf(sacc[i], scale_log2, -m_use));
      // the row's partial sum as a tree (a chain of 16 dependent adds sat on the critical path)
      float ps[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) ps[i] = (sc[4 * i] + sc[4 * i + 1]) + (sc[4 * i + 2] + sc[4 * i + 3]);
      l_run += (ps[0] + ps[1]) + (ps[2] + ps[3]);
      u32x4_t pb[2];
#pragma unroll
      for (int j = 0; j < 2; ++j)
        pb[j] = u32x4_t{pack_bf2(sc[8 * j], sc[8 * j + 1]), pack_bf2(sc[8 * j + 2], sc[8 * j + 3]),
                        pack_bf2(sc[8 * j + 4], sc[8 * j + 5]), pack_bf2(sc[8 * j + 6], sc[8 * j + 7])};
      // O^T += V^T P^T. Transpose-read source lanes: group G16 = lane / 16 reads rows
      // 16j + 8h + 4kg + (lane%16)/4 (h: first or second 4 tokens), dims 32bb + 16(G16%2) + 4(lane%4)
      const int g16 = lane >> 4, jj = (lane >> 2) & 3, qq = lane & 3;
      const uint16_t* vbase = kd + TILE;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) {
          uint2 hv[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int r = 16 * j + 8 * h + 4 * kg + jj;
            const int dim = 32 * bb + 16 * (g16 & 1) + 4 * qq;
            const int c = (dim >> 3) ^ v32_swizzle(r);
            hv[h] = lds_read_tr16(vbase + r * D + 8 * c + (dim & 7));
          }
          const u32x4_t va = {hv[0].x, hv[0].y, hv[1].x, hv[1].y};
          o[bb] = mfma_32x32x16(va, pb[j], o[bb]);
        }
    };
    Slot sa, sb;
    gload(sa, 0);
    if (ntiles > 1) gload(sb, 1);
    lwrite(sa, 0);
    if (ntiles > 2) gload(sa, 2);
    __syncthreads();
    for (int k = 0;;) {
      compute(k);
      if (k + 1 < ntiles) {
        lwrite(sb, k + 1);
        if (k + 3 < ntiles) gload(sb, k + 3);
      }
      __syncthreads();
      if (++k >= ntiles) break;
      compute(k);
      if (k + 1 < ntiles) {
        lwrite(sa, k + 1);
        if (k + 3 < ntiles) gload(sa, k + 3);
      }
      __syncthreads();
      if (++k >= ntiles) break;
    }
  }
  // normalise and write: o[bb][i] is dim 32bb + 8(i/4) + 4kg + i%4 of row R; lanes r and r^32
  // together cover 8 consecutive dims
  float L = l_run + lane_read(l_run, lane ^ 32);
  if (valid) L += sink_mass(sinks, kvh * G + hg, m_run);
  const float inv = L > 0.f ? 1.f / L : 0.f;
  if (valid) {
    uint16_t* op = out + (int64_t)(q0 + tok) * o_ts + (int64_t)(kvh * G + hg) * o_hs;
#pragma unroll
    for (int bb = 0; bb < NB; ++bb)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint2 v = {pack_bf2(o[bb][4 * c] * inv, o[bb][4 * c + 1] * inv),
                         pack_bf2(o[bb][4 * c + 2] * inv, o[bb][4 * c + 3] * inv)};
        *reinterpret_cast<uint2*>(op + 32 * bb + 8 * c + 4 * kg) = v;
      }
  }
  }
  // the last work group out resets the counters for the next launch with this plan; the fence
  // orders this group's queue atomics before its done count
  __threadfence();
  if (threadIdx.x == 0 && atomicAdd(&counters[kPlanDoneWord], 1) == (int)gridDim.x - 1) {
    for (int x = 0; x < 8; ++x) atomicExch(&counters[kPlanQueueWord + x], 0);
    atomicExch(&counters[kPlanDoneWord], 0);
  }
}

}  // namespace pie

using namespace pie;

// Host: how many splits per request. Aims at ~4 work groups per CU over all (request, kv head,
// split) triples when the launch takes requests longest first (batches of at most kRankMax), at
// ~16 otherwise (smaller pieces even out the tail that request order leaves); when the longest
// context is known (max_kv_len >= 0) no split is shorter than kMinChunk tokens. The result
// depends on the batch only, so one plan serves a captured graph.
extern "C" int pie_hip_attention_decode_plan(int64_t batch, int64_t num_kv_heads, int64_t max_kv_len,
                                             int64_t num_cus, int64_t* splits) {
  PIE_REQUIRE(splits && batch >= 0 && num_kv_heads > 0, "decode_plan: bad batch %lld / num_kv_heads %lld",
              (long long)batch, (long long)num_kv_heads);
  const int64_t cus = num_cus > 0 ? num_cus : 256;
  const int64_t per = std::max<int64_t>(1, batch * num_kv_heads);
  const int64_t groups = (batch <= kRankMax ? 4 : 16) * cus;
  int64_t s = (groups + per - 1) / per;
  if (max_kv_len >= 0) s = std::min<int64_t>(s, std::max<int64_t>(1, (max_kv_len + kMinChunk - 1) / kMinChunk));
  *splits = std::max<int64_t>(1, std::min<int64_t>(s, 64));
  return PIE_HIP_OK;
}

static int paged_kv_desc(PagedKV* kv, const uint16_t* k_cache, const uint16_t* v_cache,
                         int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                         int64_t num_pages, const int32_t* kv_indptr, const int32_t* kv_indices,
                         const int32_t* kv_last_page_len, int64_t page_size, int64_t D,
                         const char* what) {
  PIE_REQUIRE(k_cache && v_cache && kv_indptr && kv_indices && kv_last_page_len, "%s: null cache or page table", what);
  PIE_REQUIRE(page_size > 0 && page_size <= 65536 && num_pages > 0 && num_pages < (1ll << 31),
              "%s: bad page_size %lld / num_pages %lld", what, (long long)page_size, (long long)num_pages);
  PIE_REQUIRE(aligned16(k_cache) && aligned16(v_cache) && page_stride % 8 == 0 && slot_stride % 8 == 0 &&
                  head_stride % 8 == 0,
              "%s: cache pointers and strides must be 16-byte aligned", what);
  (void)D;
  kv->k = k_cache;
  kv->v = v_cache;
  kv->page_stride = page_stride;
  kv->slot_stride = slot_stride;
  kv->head_stride = head_stride;
  kv->indptr = kv_indptr;
  kv->indices = kv_indices;
  kv->last_len = kv_last_page_len;
  kv->num_pages = (int32_t)num_pages;
  kv->page_size = (int32_t)page_size;
  kv->pdiv = FastDiv::make((uint32_t)page_size);
  return PIE_HIP_OK;
}

template <int D>
static void launch_decode(hipStream_t st, const uint16_t* q, int64_t q_ts, int64_t q_hs,
                          const PagedKV& kv, int G, int Hq, int Hkv, float sl2, int B, int splits,
                          int window_left, uint16_t* out, int64_t o_ts, int64_t o_hs, float* po,
                          float* pl, const float* sinks) {
  hipLaunchKernelGGL(attn_decode_kernel<D>, dim3(B * splits * Hkv), dim3(256), 0, st, q, q_ts, q_hs, kv,
                     B, G, Hq, sl2, splits, window_left, out, o_ts, o_hs, po, pl, sinks);
  if (splits > 1)
    hipLaunchKernelGGL(attn_merge_kernel<D>, dim3(B, (Hq + 64 / (D / 8) - 1) / (64 / (D / 8))), dim3(64), 0,
                       st, B, Hq, splits, po, pl, out, o_ts, o_hs, sinks);
}

static int attention_decode_impl(
    const pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride, const pie_bf16* k_cache,
    const pie_bf16* v_cache, int64_t page_stride, int64_t slot_stride, int64_t head_stride,
    int64_t num_pages, const int32_t* kv_indptr, const int32_t* kv_indices,
    const int32_t* kv_last_page_len, int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads,
    int64_t head_dim, int64_t page_size, float sm_scale, int64_t window_left, const float* sinks, int64_t splits,
    void* workspace, int64_t workspace_bytes, pie_bf16* out, int64_t o_tok_stride,
    int64_t o_head_stride, void* stream, const char* what) {
  PagedKV kv;
  int rc = paged_kv_desc(&kv, k_cache, v_cache, page_stride, slot_stride, head_stride, num_pages,
                         kv_indptr, kv_indices, kv_last_page_len, page_size, head_dim,
                         what);
  if (rc) return rc;
  PIE_REQUIRE(q && out, "attention_decode: null q or out");
  PIE_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256,
              "attention_decode: head_dim %lld not in {64, 128, 256}", (long long)head_dim);
  PIE_REQUIRE(num_kv_heads > 0 && num_qo_heads % num_kv_heads == 0 && num_qo_heads / num_kv_heads <= 16 &&
                  num_kv_heads <= 65535,
              "attention_decode: need num_qo_heads = G * num_kv_heads with G <= 16 (got %lld / %lld)",
              (long long)num_qo_heads, (long long)num_kv_heads);
  PIE_REQUIRE(batch >= 0 && splits >= 1 && splits <= 64 && batch * splits * num_kv_heads < (1ll << 31),
              "attention_decode: bad batch %lld / splits %lld", (long long)batch, (long long)splits);
  PIE_REQUIRE(aligned16(q) && aligned16(out) && q_tok_stride % 8 == 0 && q_head_stride % 8 == 0 &&
                  o_tok_stride % 8 == 0 && o_head_stride % 8 == 0,
              "attention_decode: q/out pointers and strides must be 16-byte aligned");
  const int64_t slots = splits > 1 ? batch * splits : 0;
  const int64_t need = slots * num_qo_heads * (head_dim + 1) * 4;
  PIE_REQUIRE(slots == 0 || (workspace && workspace_bytes >= need && aligned16(workspace)),
              "%s: workspace of %lld bytes < %lld needed for %lld splits", what,
              (long long)workspace_bytes, (long long)need, (long long)splits);
  if (batch == 0) return PIE_HIP_OK;
  float* po = static_cast<float*>(workspace);
  float* pl = po ? po + slots * num_qo_heads * head_dim : nullptr;
  const int G = (int)(num_qo_heads / num_kv_heads);
  const float sl2 = sm_scale * 1.4426950408889634f;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int B = (int)batch, S = (int)splits, Hq = (int)num_qo_heads, Hkv = (int)num_kv_heads;
  const int W = window_left < 0 ? -1 : (int)std::min<int64_t>(window_left, 1 << 30);
  switch (head_dim) {
    case 64: launch_decode<64>(st, q, q_tok_stride, q_head_stride, kv, G, Hq, Hkv, sl2, B, S, W, out,
                               o_tok_stride, o_head_stride, po, pl, sinks); break;
    case 128: launch_decode<128>(st, q, q_tok_stride, q_head_stride, kv, G, Hq, Hkv, sl2, B, S, W, out,
                                 o_tok_stride, o_head_stride, po, pl, sinks); break;
    default: launch_decode<256>(st, q, q_tok_stride, q_head_stride, kv, G, Hq, Hkv, sl2, B, S, W, out,
                                o_tok_stride, o_head_stride, po, pl, sinks); break;
  }
  return check_launch(what);
}

extern "C" int pie_hip_attention_decode(
    const pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride, const pie_bf16* k_cache,
    const pie_bf16* v_cache, int64_t page_stride, int64_t slot_stride, int64_t head_stride,
    int64_t num_pages, const int32_t* kv_indptr, const int32_t* kv_indices,
    const int32_t* kv_last_page_len, int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads,
    int64_t head_dim, int64_t page_size, float sm_scale, int64_t window_left, const float* sinks, int64_t splits,
    void* workspace, int64_t workspace_bytes, pie_bf16* out, int64_t o_tok_stride,
    int64_t o_head_stride, void* stream) {
  return attention_decode_impl(q, q_tok_stride, q_head_stride, k_cache, v_cache, page_stride,
                               slot_stride, head_stride, num_pages, kv_indptr, kv_indices,
                               kv_last_page_len, batch, num_qo_heads, num_kv_heads, head_dim,
                               page_size, sm_scale, window_left, sinks, splits, workspace, workspace_bytes,
                               out, o_tok_stride, o_head_stride, stream, "attention_decode");
}

// ---------------------------------------------------------------- decode without allocation
// The split partials (fp32 outputs + log2-sum-exp per (slot, head)) live in a file-scope device
// array instead of a caller workspace, for callers that cannot allocate. Each device holds its
// own copy; host code uses only the address hipGetSymbolAddress returns for the current device
// (the array's name is a host-side stand-in, never a device address). Every partial a run
// reads is written earlier in the same run (empty splits write zeros and -inf), so the array
// needs no clearing between calls; calls that overlap on one device race on it.
constexpr int64_t kDecodeScratchBytes = 32ll << 20;
static __device__ __align__(256) char scratch[kDecodeScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_dev[64] = {nullptr};

static int decode_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= 64)
    return set_error(PIE_HIP_ELAUNCH, "attention_decode_noalloc: no current device (%s)", hipGetErrorString(e));
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(PIE_HIP_ELAUNCH, "attention_decode_noalloc: hipGetSymbolAddress failed on device %d: %s",
                       dev, hipGetErrorString(e));
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return PIE_HIP_OK;
}

extern "C" int pie_hip_attention_decode_noalloc(
    const pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride, const pie_bf16* k_cache,
    const pie_bf16* v_cache, int64_t page_stride, int64_t slot_stride, int64_t head_stride,
    int64_t num_pages, const int32_t* kv_indptr, const int32_t* kv_indices,
    const int32_t* kv_last_page_len, int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads,
    int64_t head_dim, int64_t page_size, float sm_scale, int64_t window_left, const float* sinks, int64_t splits,
    pie_bf16* out, int64_t o_tok_stride, int64_t o_head_stride, void* stream) {
  const char* what = "attention_decode_noalloc";
  PIE_REQUIRE(batch >= 0 && splits >= 1 && splits <= 64 && num_qo_heads > 0 && head_dim > 0,
              "%s: bad batch %lld / splits %lld", what, (long long)batch, (long long)splits);
  const int64_t need = splits > 1 ? batch * splits * num_qo_heads * (head_dim + 1) * 4 : 0;
  PIE_REQUIRE(need <= kDecodeScratchBytes,
              "%s: %lld bytes of split partials exceed the %lld-byte static scratch (use fewer splits "
              "or pie_hip_attention_decode with a workspace)",
              what, (long long)need, (long long)kDecodeScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    int rc = decode_scratch(&ws);
    if (rc) return rc;
    rc = inflight_check(ws, stream, what);
    if (rc) return rc;
  }
  const int rc = attention_decode_impl(q, q_tok_stride, q_head_stride, k_cache, v_cache, page_stride,
                               slot_stride, head_stride, num_pages, kv_indptr, kv_indices,
                               kv_last_page_len, batch, num_qo_heads, num_kv_heads, head_dim,
                               page_size, sm_scale, window_left, sinks, splits, ws, kDecodeScratchBytes,
                               out, o_tok_stride, o_head_stride, stream, what);
  if (rc == PIE_HIP_OK && need > 0) inflight_mark(ws, stream);
  return rc;
}

// Host: the prefill work list. Reads host copies of qo_indptr, kv_indptr and kv_last_page_len
// (as flashinfer's plan does); lists (request, first row) items of prefill_rows<D> packed rows,
// those that see the most kv positions first, and for mode 2 the byte offset of every
// request's [qo_len, kv_len] mask block (int64, 8-byte aligned in the plan).
extern "C" int pie_hip_attention_prefill_plan(const int32_t* qo_indptr, const int32_t* kv_indptr,
                                              const int32_t* kv_last_page_len, int64_t batch,
                                              int64_t page_size, int64_t num_qo_heads,
                                              int64_t num_kv_heads, int64_t head_dim, int32_t mode,
                                              int32_t* plan,
                                              int64_t plan_capacity, int64_t* plan_words,
                                              int64_t* num_items, int64_t* mask_bytes,
                                              int64_t* mask_words) {
  PIE_REQUIRE(qo_indptr && kv_indptr && kv_last_page_len && plan && plan_words && num_items && mask_bytes &&
                  mask_words,
              "prefill_plan: null argument");
  PIE_REQUIRE(batch >= 0 && batch < (1 << 24) && page_size > 0 && num_kv_heads > 0 &&
                  num_qo_heads % num_kv_heads == 0 && mode >= 0 && mode <= 2,
              "prefill_plan: bad batch %lld / page_size %lld / heads %lld,%lld / mode %d",
              (long long)batch, (long long)page_size, (long long)num_qo_heads,
              (long long)num_kv_heads, mode);
  PIE_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256,
              "prefill_plan: head_dim %lld not in {64, 128, 256}", (long long)head_dim);
  const int64_t G = num_qo_heads / num_kv_heads;
  const int64_t kPrefillRows = head_dim == 256 ? prefill_rows<256>() : prefill_rows<128>();
  struct Item { int32_t b, row0, q0, qo, kv, page0; int64_t work, req_work; };
  std::vector<Item> items;
  std::vector<int64_t> moff((size_t)batch + 1, 0), woff((size_t)batch + 1, 0);
  int64_t mtotal = 0, wtotal = 0;
  for (int64_t b = 0; b < batch; ++b) {
    const int64_t qo = (int64_t)qo_indptr[b + 1] - qo_indptr[b];
    const int64_t np = (int64_t)kv_indptr[b + 1] - kv_indptr[b];
    PIE_REQUIRE(qo >= 0 && np >= 0, "prefill_plan: indptr decreases at request %lld", (long long)b);
    const int64_t kv = np > 0 ? (np - 1) * page_size + kv_last_page_len[b] : 0;
    PIE_REQUIRE(kv >= 0 && kv < (mode == 2 ? kExtentCausal : (1ll << 31)) && qo * G < (1ll << 31),
                "prefill_plan: request %lld too long", (long long)b);
    moff[(size_t)b] = mtotal;
    woff[(size_t)b] = wtotal;
    mtotal += qo * kv;
    wtotal += qo * ((kv + 31) / 32);
    for (int64_t r0 = 0; r0 < qo * G; r0 += kPrefillRows) {
      const int64_t last = std::min(qo * G, r0 + kPrefillRows) - 1;
      const int64_t seen = mode == 1 ? std::max<int64_t>(0, std::min(kv, kv - qo + last / G + 1)) : kv;
      items.push_back(Item{(int32_t)b, (int32_t)r0, qo_indptr[b], (int32_t)qo, (int32_t)kv, kv_indptr[b],
                           seen, kv * qo});
    }
  }
  // Each request's items stay together (they share its K/V prefix, which the kernels' XCD-aware
  // order keeps in one L2): longest requests first, and in each request the items that see the
  // most K/V first, so the shortest work comes last.
  std::stable_sort(items.begin(), items.end(), [](const Item& x, const Item& y) {
    if (x.req_work != y.req_work) return x.req_work > y.req_work;
    if (x.b != y.b) return x.b < y.b;
    return x.work > y.work;
  });
  int64_t words = kPlanHeader + kPlanItemWords * (int64_t)items.size();
  words = (words + 1) / 2 * 2;  // int64 mask offsets start 8-byte aligned
  moff[(size_t)batch] = mtotal;
  woff[(size_t)batch] = wtotal;
  const int64_t moff_word = words, woff_word = words + 2 * (batch + 1);
  if (mode == 2) words += 4 * (batch + 1);
  *plan_words = words;
  *num_items = (int64_t)items.size();
  *mask_bytes = mtotal;
  *mask_words = wtotal;
  PIE_REQUIRE(words <= plan_capacity, "prefill_plan: needs %lld words, capacity %lld",
              (long long)words, (long long)plan_capacity);
  for (int i = 0; i < kPlanHeader; ++i) plan[i] = 0;
  plan[0] = (int32_t)items.size();
  plan[1] = (int32_t)batch;
  plan[2] = (int32_t)kPrefillRows;
  plan[3] = (int32_t)moff_word;  // mode 2: int64 byte offsets of the mask blocks [batch + 1]
  plan[4] = (int32_t)woff_word;  // mode 2: int64 offsets of the packed mask words [batch + 1]
  // [7] and [8, 16): the persistent kernel's work counters (zero between launches)
  int32_t* p = plan + kPlanHeader;
  for (const Item& it : items) {
    const int32_t w8[kPlanItemWords] = {it.b, it.row0, it.q0, it.qo, it.kv, it.page0, 0, 0};
    for (int i = 0; i < kPlanItemWords; ++i) *p++ = w8[i];
  }
  if (mode == 2) {
    memcpy(plan + moff_word, moff.data(), sizeof(int64_t) * (size_t)(batch + 1));
    memcpy(plan + woff_word, woff.data(), sizeof(int64_t) * (size_t)(batch + 1));
  }
  return PIE_HIP_OK;
}

template <int D>
static void launch_prefill(hipStream_t st, dim3 grid, const uint16_t* q, int64_t q_ts, int64_t q_hs,
                           const PagedKV& kv, const int32_t* qo_indptr, int G, float sl2,
                           const int32_t* plan, int mode, int window_left, const uint32_t* packed,
                           const int64_t* woff, const int32_t* extent, uint16_t* out, int64_t o_ts,
                           int64_t o_hs, const float* sinks) {
  // attn_prefill32_kernel scales raw scores inside the exponent, where a zero scale would turn a
  // hidden (-inf) score into NaN; 1e-30 gives the same result (every exponent rounds to 2^0).
  const dim3 xgrid(8 * ((grid.x * grid.y + 7) / 8));  // (kv head, item) units, padded to 8 XCDs
  if constexpr (D == 128)
    hipLaunchKernelGGL(attn_prefill32_kernel<128>, dim3(8 * ((2 * num_cus() + 7) / 8)), dim3(256), 0, st, q, q_ts,
                       q_hs, kv, qo_indptr, G,
                       sl2 == 0.f ? 1e-30f : sl2, plan, (int)grid.x, (int)grid.y, mode, window_left, packed,
                       woff, extent, out, o_ts, o_hs, sinks);
  else
    hipLaunchKernelGGL(attn_prefill_kernel<D>, xgrid, dim3(64 * prefill_waves<D>()), 0, st, q, q_ts, q_hs, kv,
                       qo_indptr, G, sl2, plan, (int)grid.x, (int)grid.y, mode, window_left, packed, woff,
                       extent, out, o_ts, o_hs, sinks);
}

// Visible extent of every query token under the packed mask: 1 + the last kv position whose bit
// is set (0 if none), with kExtentCausal set when the row is exactly causal. One thread per query
// token, scanning its words from the end (and, for the causal test, from the start).
__global__ __launch_bounds__(256) void attn_mask_extent_kernel(const uint32_t* __restrict__ packed,
                                                               const int32_t* __restrict__ plan,
                                                               const int32_t* __restrict__ qo_indptr,
                                                               PagedKV kv, int B, int T,
                                                               int32_t* __restrict__ extent) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= T) return;
  const int64_t* woff = reinterpret_cast<const int64_t*>(plan + plan[4]);
  int lo = 0, hi = B - 1;  // the request holding query token j
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (qo_indptr[mid] <= j) lo = mid; else hi = mid - 1;
  }
  const int b = lo, i = j - qo_indptr[b];
  const int kv_len = kv_length(kv, b);
  const int nw = (kv_len + 31) / 32;
  const uint32_t* row = packed + woff[b] + (int64_t)i * nw;
  int e = 0;
  for (int w = nw - 1; w >= 0; --w)
    if (row[w]) { e = 32 * w + 32 - __builtin_clz(row[w]); break; }
  // exactly causal: the extent is the causal one and every bit below it is set
  bool causal = e > 0 && e == kv_len - (qo_indptr[b + 1] - qo_indptr[b]) + i + 1;
  for (int w = 0; causal && 32 * w < e; ++w) {
    const int n = min(32, e - 32 * w);
    causal = row[w] == (n == 32 ? 0xffffffffu : (1u << n) - 1u);
  }
  extent[j] = e | (causal ? kExtentCausal : 0);
}

// Bit-packs the custom mask: one thread per 32-bit word (query token i of request b, kv
// positions 32w..32w+31; bit j = mask byte of position 32w+j, 0 past kv_len).
__global__ __launch_bounds__(256) void attn_pack_mask_kernel(const uint8_t* __restrict__ mask,
                                                             const int32_t* __restrict__ plan,
                                                             const int32_t* __restrict__ qo_indptr,
                                                             PagedKV kv, int B, int64_t total,
                                                             uint32_t* __restrict__ packed) {
  const int64_t gw = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gw >= total) return;
  const int64_t* moff = reinterpret_cast<const int64_t*>(plan + plan[3]);
  const int64_t* woff = reinterpret_cast<const int64_t*>(plan + plan[4]);
  int lo = 0, hi = B - 1;  // the request whose word range holds gw
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (woff[mid] <= gw) lo = mid; else hi = mid - 1;
  }
  const int b = lo;
  const int kv_len = kv_length(kv, b);
  const int64_t nw = (kv_len + 31) / 32;
  const int64_t local = gw - woff[b];
  const int64_t i = local / nw, w = local - i * nw;
  const uint8_t* src = mask + moff[b] + i * kv_len + 32 * w;
  const int n = (int)min((int64_t)32, (int64_t)kv_len - 32 * w);
  uint32_t bits = 0;
  for (int j = 0; j < n; ++j) bits |= (uint32_t)(src[j] != 0) << j;
  packed[gw] = bits;
}

extern "C" int pie_hip_attention_prefill(
    const pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride, const pie_bf16* k_cache,
    const pie_bf16* v_cache, int64_t page_stride, int64_t slot_stride, int64_t head_stride,
    int64_t num_pages, const int32_t* qo_indptr, const int32_t* kv_indptr, const int32_t* kv_indices,
    const int32_t* kv_last_page_len, int64_t num_qo_heads, int64_t num_kv_heads, int64_t head_dim,
    int64_t page_size, float sm_scale, int32_t mode, int64_t window_left, const float* sinks,
    const uint32_t* packed_mask, const int32_t* mask_extent, const int32_t* plan, int64_t num_items,
    int64_t mask_offsets_word, pie_bf16* out,
    int64_t o_tok_stride, int64_t o_head_stride, void* stream) {
  PagedKV kv;
  int rc = paged_kv_desc(&kv, k_cache, v_cache, page_stride, slot_stride, head_stride, num_pages,
                         kv_indptr, kv_indices, kv_last_page_len, page_size, head_dim,
                         "attention_prefill");
  if (rc) return rc;
  PIE_REQUIRE(q && out && plan && qo_indptr, "attention_prefill: null q, out, plan or qo_indptr");
  PIE_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256,
              "attention_prefill: head_dim %lld not in {64, 128, 256}", (long long)head_dim);
  PIE_REQUIRE(num_kv_heads > 0 && num_kv_heads <= 65535 && num_qo_heads % num_kv_heads == 0,
              "attention_prefill: num_qo_heads %lld not a multiple of num_kv_heads %lld",
              (long long)num_qo_heads, (long long)num_kv_heads);
  PIE_REQUIRE(mode >= 0 && mode <= 2 && (mode != 2 || (packed_mask && mask_extent && mask_offsets_word > 0 &&
                                                       mask_offsets_word % 2 == 0)),
              "attention_prefill: mode %d needs the packed mask and its plan offsets", mode);
  PIE_REQUIRE(num_items >= 0 && num_items * num_kv_heads < (1ll << 31), "attention_prefill: bad item count");
  PIE_REQUIRE(aligned16(q) && aligned16(out) && q_tok_stride % 8 == 0 && q_head_stride % 8 == 0 &&
                  o_tok_stride % 8 == 0 && o_head_stride % 8 == 0,
              "attention_prefill: q/out pointers and strides must be 16-byte aligned");
  if (num_items == 0) return PIE_HIP_OK;
  const int G = (int)(num_qo_heads / num_kv_heads);
  const float sl2 = sm_scale * 1.4426950408889634f;
  const int64_t* woff = mode == 2 ? reinterpret_cast<const int64_t*>(plan + mask_offsets_word) : nullptr;
  const int Wl = window_left < 0 ? -1 : (int)std::min<int64_t>(window_left, 1 << 30);
  const dim3 grid((unsigned)num_items, (unsigned)num_kv_heads);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // the head-dim-128 kernel counts its work in the plan's header words
  const bool counters = head_dim == 128;
  if (counters && (rc = inflight_check(plan, stream, "attention_prefill")) != PIE_HIP_OK) return rc;
  switch (head_dim) {
    case 64: launch_prefill<64>(st, grid, q, q_tok_stride, q_head_stride, kv, qo_indptr, G, sl2, plan,
                                mode, Wl, packed_mask, woff, mask_extent, out, o_tok_stride, o_head_stride, sinks); break;
    case 128: launch_prefill<128>(st, grid, q, q_tok_stride, q_head_stride, kv, qo_indptr, G, sl2, plan,
                                  mode, Wl, packed_mask, woff, mask_extent, out, o_tok_stride, o_head_stride, sinks); break;
    default: launch_prefill<256>(st, grid, q, q_tok_stride, q_head_stride, kv, qo_indptr, G, sl2, plan,
                                 mode, Wl, packed_mask, woff, mask_extent, out, o_tok_stride, o_head_stride, sinks); break;
  }
  rc = check_launch("attention_prefill");
  if (rc == PIE_HIP_OK && counters) inflight_mark(plan, stream);
  return rc;
}

extern "C" int pie_hip_attention_pack_mask(const uint8_t* custom_mask, const int32_t* plan,
                                           const int32_t* qo_indptr, const int32_t* kv_indptr,
                                           const int32_t* kv_last_page_len, int64_t batch,
                                           int64_t page_size, int64_t mask_words, int64_t num_tokens,
                                           uint32_t* packed_mask, int32_t* mask_extent, void* stream) {
  PIE_REQUIRE(custom_mask && plan && qo_indptr && kv_indptr && kv_last_page_len && packed_mask && mask_extent,
              "attention_pack_mask: null argument");
  PIE_REQUIRE(num_tokens >= 0 && num_tokens < (1ll << 31), "attention_pack_mask: bad token count");
  PIE_REQUIRE(batch > 0 && batch < (1 << 24) && page_size > 0 && mask_words >= 0,
              "attention_pack_mask: bad batch %lld / page_size %lld / words %lld", (long long)batch,
              (long long)page_size, (long long)mask_words);
  PagedKV kv{};
  kv.indptr = kv_indptr;
  kv.last_len = kv_last_page_len;
  kv.page_size = (int32_t)page_size;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (mask_words > 0)
    hipLaunchKernelGGL(attn_pack_mask_kernel, dim3((unsigned)((mask_words + 255) / 256)), dim3(256), 0, st,
                       custom_mask, plan, qo_indptr, kv, (int)batch, mask_words, packed_mask);
  if (num_tokens > 0)
    hipLaunchKernelGGL(attn_mask_extent_kernel, dim3((unsigned)((num_tokens + 255) / 256)), dim3(256), 0, st,
                       packed_mask, plan, qo_indptr, kv, (int)batch, (int)num_tokens, mask_extent);
  return check_launch("attention_pack_mask");
}
