// Device-side pieces of RoPE, the paged append and Qwen3's fused q/k prologue, shared by the
// standalone kernels (rope.hip) and the grouped decode launch (group.hip).
#pragma once

#include "common.h"

namespace pie {
namespace {

constexpr int kMaxPairs = 256;

struct HeadsDesc {
  uint16_t* q;
  uint16_t* k;
  const uint16_t* v;
  int64_t q_ts, q_hs, k_ts, k_hs, v_ts, v_hs;
  int32_t Hq, Hkv, D, rd;
};

struct CacheDesc {
  const int32_t* batch_indices;
  const int32_t* positions;
  const int32_t* kv_indices;
  const int32_t* kv_indptr;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t batch_size, num_pages, page_stride, slot_stride, head_stride;
  int32_t page_size;
};

struct RopeAppendArgs {
  HeadsDesc h;
  CacheDesc c;
  const int32_t* pos;
  int64_t T;
  int32_t wpt;         // waves per token (vector kernel)
  int32_t interleave;  // pair layout (scalar kernel)
  // Precomputed table instead of inv_freq (flashinfer's apply_rope_with_cos_sin_cache_inplace):
  // row p holds cos(angle_i) at [i] and sin(angle_i) at [rd/2 + i]; positions outside
  // [0, cs_rows) rotate by the identity.
  const float* cs;
  int64_t cs_rows, cs_ld;
  // last: read by vector loads, so the scalar fields above fit in the first few cache lines
  float inv_freq[kMaxPairs];
};

// (cos, sin) of the angle p * f for position p and frequency f, by the hardware sine / cosine,
// which take revolutions: the revolutions p * (f / 2pi) are formed exactly from the fp32 product
// and its fma-recovered low part (the error-free TwoProduct of Ogita, Rump and Oishi, "Accurate
// sum and dot product", SIAM J. Sci. Comput. 2005), so only the fractional part matters and no
// precision is lost to the angle's magnitude (positions up to 2^24); the result carries the
// rounding of f / 2pi (~p * f * 6e-8 rad, the order of the reference's own fp32 angle p * f).
// p = 0 gives (1, 0).
__device__ __forceinline__ float2 rope_pos_cs(int p, float f) {
  const float fr = f * 0.15915494309189535f;  // f / 2pi
  const float pf = (float)p;
  const float hi = pf * fr;
  const float lo = fmaf(pf, fr, -hi);
  const float rev = __builtin_amdgcn_fractf(__builtin_amdgcn_fractf(hi) + lo);
  return make_float2(__builtin_amdgcn_cosf(rev), __builtin_amdgcn_sinf(rev));
}

// cos/sin of pair i at position p: from the table when one is given, else from inv_freq.
__device__ __forceinline__ float2 rope_cs(const RopeAppendArgs& a, int p, int i, int half) {
  if (a.cs) {
    if (p < 0 || (int64_t)p >= a.cs_rows) return make_float2(1.f, 0.f);
    const float* row = a.cs + (int64_t)p * a.cs_ld;
    return make_float2(row[i], row[half + i]);
  }
  return rope_pos_cs(p, a.inv_freq[i]);
}


// The rotation with its fused multiply-adds spelled out, so every kernel variant (rope only,
// fused with the append, scalar fallback) rounds identically: x' = x c - y s, y' = x s + y c.
__device__ __forceinline__ float rot_x(float x, float y, float2 cs) { return fmaf(x, cs.x, -(y * cs.y)); }
__device__ __forceinline__ float rot_y(float x, float y, float2 cs) { return fmaf(x, cs.y, y * cs.x); }

// Cache element offset of (token's page, slot), or -1 when the token is skipped.
__device__ __forceinline__ int64_t slot_offset(const CacheDesc& c, int64_t t) {
  const int b = c.batch_indices[t];
  const int p = c.positions[t];
  if (b < 0 || (int64_t)b >= c.batch_size || p < 0) return -1;
  const int lo = c.kv_indptr[b], hi = c.kv_indptr[b + 1];
  const int64_t logical = (int64_t)lo + p / c.page_size;
  if (logical >= hi) return -1;
  const int page = c.kv_indices[logical];
  if (page < 0 || (int64_t)page >= c.num_pages) return -1;
  return (int64_t)page * c.page_stride + (int64_t)(p % c.page_size) * c.slot_stride;
}

// ---------------------------------------------------------------- q/k RMSNorm + RoPE + append
// Qwen3's attention prologue (qwen3.py:651-684: per-head q/k RMSNorm, RoPE, paged append) in
// one pass for D = 128, full rotary dim, half-split pairs. A 16-lane group owns one head row
// (8 elements per lane): it normalises the row exactly as rmsnorm_heads16 does (same sum
// order), rounds to bf16, fetches the rotation partner's 8 values from lane l^8 with DPP
// row_ror:8, rotates exactly as rope_append_vec does, and stores q_out/k_out (and k, v to the
// cache page). Results are bit-identical to the three separate kernels. Every lane runs the
// same instruction sequence (stores are predicated), so the DPP exchanges never sit in
// divergent code.
struct QkNormArgs {
  uint16_t* q_out;
  uint16_t* k_out;
  int64_t qo_ts, qo_hs, ko_ts, ko_hs;
  const uint16_t* qw;
  const uint16_t* kw;
  float eps;
  RopeAppendArgs r;  // q/k/v inputs, cache, pos, T, wpt, inv_freq (last, see RopeAppendArgs)
};
// Bytes of a QkNormArgs before its inverse-frequency array (the scalar part).
constexpr int kQkScalarBytes = (int)(offsetof(QkNormArgs, r) + offsetof(RopeAppendArgs, inv_freq));

__device__ __forceinline__ uint32_t dpp_ror8(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);
}

// The page lookup of slot_offset in two steps, so the loads that do not depend on each other are
// all in flight before anything waits: issue() requests the token's batch index and position
// together with the page range of request t, on the guess b == t (a decode batch: token t is
// request t's one new token); resolve() checks the guess (loading the range again when it was
// wrong) and requests the page id. Same result as slot_offset.
struct SlotLookup {
  int b, p, lo, hi;
};
__device__ __forceinline__ SlotLookup slot_issue(const CacheDesc& c, int64_t t) {
  SlotLookup s{-1, -1, 0, 0};
  if (c.batch_size <= 0) return s;
  const int64_t ts = t < c.batch_size ? t : c.batch_size - 1;
  s.b = c.batch_indices[t];
  s.p = c.positions[t];
  s.lo = c.kv_indptr[ts];
  s.hi = c.kv_indptr[ts + 1];
  return s;
}
// Returns the element offset of the slot (or -1 when the token is skipped); *page receives the
// page id load, still in flight, for slot_finish.
__device__ __forceinline__ int64_t slot_resolve(const CacheDesc& c, int64_t t, SlotLookup s, int* page) {
  *page = -1;
  if (s.b < 0 || (int64_t)s.b >= c.batch_size || s.p < 0) return -1;
  const int64_t ts = t < c.batch_size ? t : c.batch_size - 1;
  if (s.b != ts) {
    s.lo = c.kv_indptr[s.b];
    s.hi = c.kv_indptr[s.b + 1];
  }
  const int64_t logical = (int64_t)s.lo + s.p / c.page_size;
  if (logical >= s.hi) return -1;
  *page = c.kv_indices[logical];
  return (int64_t)(s.p % c.page_size) * c.slot_stride;
}
// The cache offset once the page id has landed: -1 for a page outside the pool.
__device__ __forceinline__ int64_t slot_finish(const CacheDesc& c, int64_t slot_off, int page) {
  if (slot_off < 0 || page < 0 || (int64_t)page >= c.num_pages) return -1;
  return (int64_t)page * c.page_stride + slot_off;
}

// Work of block `bid` (threadIdx.x as in a launch of blockDim.x = max(64 wpt, 256) threads).
// Every wave works alone (no LDS, no barrier): each lane evaluates the cos/sin of its own 8
// pairs, so nothing waits for the page lookup except the cache stores, and the q/k outputs are
// stored as soon as the rows have landed.
__device__ __forceinline__ void qk_norm_rope_append_block(const QkNormArgs& qa, int bid) {
  const RopeAppendArgs& a = qa.r;
  const int wpt = a.wpt;                 // 1, 2, 4 (256-thread blocks) or up to 16 (one token)
  const int tpb = wpt >= 4 ? 1 : 4 / wpt;
  const int slot = (threadIdx.x >> 6) / wpt;
  const int gt = threadIdx.x - slot * wpt * 64;
  const int gsize = wpt * 64;
  const int64_t t = (int64_t)bid * tpb + slot;
  if (t >= a.T) return;  // whole token groups (waves) leave together
  const HeadsDesc& h = a.h;

  const int sub = gt & 15;            // lane within the head row
  const int lo = sub & 7;             // pair block: pairs lo*8 .. lo*8+7
  const bool is_x = sub < 8;          // holds the x half (dims < 64) of its pairs
  const int sg = gt >> 4, nsg = gsize >> 4;
  const int nrows = h.Hq + 2 * h.Hkv;  // q heads, k heads, v heads
  // Wave-uniform token index: the per-token position and page lookup run on scalar loads,
  // which complete on their own counter instead of behind the vector data loads.
  const int64_t tq = uniform((int)t);

  // head rows per 16-lane group per batch: 3 holds the 48 rows of a Qwen3-8B token (32 q, 8 k, 8 v
  // heads over 16 groups) in one batch, and keeps the grouped decode kernel at 73 VGPRs (7 work
  // groups per CU instead of 6 at 4 rows: 8.24-8.27 against 8.32-8.33 us per chain)
  constexpr int UB = 3;
  struct Batch {
    uint4 X[UB], Wt[UB];
    int kind[UB], hd[UB];  // kind: 0 q, 1 k, 2 v, 3 none
  };
  // Branch-free loads (pointer chosen by selects, every load issued unconditionally): loads in
  // divergent branches would each be followed by a wait, serialising the batch. Rows past the
  // end re-read the token's first q row and are discarded.
  const uint16_t* qrow = h.q + tq * h.q_ts;
  const uint16_t* krow = h.k + tq * h.k_ts;
  const uint16_t* vrow = h.v + tq * h.v_ts;
  auto load_batch = [=](int r0) {
    Batch b;
#pragma unroll
    for (int i = 0; i < UB; ++i) {
      const int r = r0 + i * nsg;
      const int kd = r >= nrows ? 3 : (r < h.Hq ? 0 : (r < h.Hq + h.Hkv ? 1 : 2));
      const int hh = kd == 0 ? r : (kd == 1 ? r - h.Hq : (kd == 2 ? r - h.Hq - h.Hkv : 0));
      const uint16_t* src = kd == 1 ? krow + (int64_t)hh * h.k_hs
                          : kd == 2 ? vrow + (int64_t)hh * h.v_hs
                          : kd == 0 ? qrow + (int64_t)hh * h.q_hs
                                    : (h.Hq > 0 ? qrow : krow);
      b.kind[i] = kd;
      b.hd[i] = hh;
      b.X[i] = ld_nt(src + sub * 8);
      b.Wt[i] = ld16((kd == 1 || h.Hq == 0 ? qa.kw : qa.qw) + sub * 8);
    }
    return b;
  };
  // Latency order: every load that does not wait for another goes out first: the position and
  // the first step of the page lookup (scalar loads), this lane's 8 frequencies and the first
  // batch of rows (vector loads). Then the page id is requested; only the cache stores wait for
  // it (the q/k outputs are stored as soon as the rows have landed).
  const int p = a.pos[tq];
  const SlotLookup sl = slot_issue(a.c, tq);
  float fq[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) fq[e] = a.inv_freq[lo * 8 + e];
  Batch b = load_batch(sg);
  int page;
  const int64_t soff = slot_resolve(a.c, tq, sl, &page);
  float2 tb[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) tb[e] = rope_pos_cs(p, fq[e]);

  // uniform trip count over the wave: all 64 lanes execute every DPP exchange
  const int nbatch = (nrows + nsg * UB - 1) / (nsg * UB);
  for (int bi = 0; bi < nbatch; ++bi) {
    if (bi > 0) b = load_batch(sg + bi * nsg * UB);
    const uint4* X = b.X;
    const uint4* Wt = b.Wt;
    const int* kind = b.kind;
    const int* hd = b.hd;
#pragma unroll
    for (int i = 0; i < UB; ++i) {
      // rows of v heads and slots past the last row need no norm or rotation: a wave whose 16-lane
      // groups hold only such rows skips them (the test is wave-uniform, so the DPP exchanges
      // below still run on all 64 lanes when they run)
      uint4 o = X[i];
      if (__builtin_amdgcn_ballot_w64(kind[i] <= 1) != 0) {
        float f[8], wf[8];
        unpack8(X[i], f);
        unpack8(Wt[i], wf);
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
        const float rstd = rsqrtf(row16_sum(ss) / 128.0f + qa.eps);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = (f[e] * rstd) * wf[e];
        const uint4 g = pack8(f);  // normalised row, rounded to bf16 as the separate norm stores it
        const uint4 pg = make_uint4(dpp_ror8(g.x), dpp_ror8(g.y), dpp_ror8(g.z), dpp_ror8(g.w));
        float own[8], oth[8];
        unpack8(g, own);
        unpack8(pg, oth);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          own[e] = is_x ? rot_x(own[e], oth[e], tb[e]) : rot_y(oth[e], own[e], tb[e]);
        o = pack8(own);
      }
      if (kind[i] == 0) {
        st16(qa.q_out + tq * qa.qo_ts + (int64_t)hd[i] * qa.qo_hs + sub * 8, o);
      } else {
        if (kind[i] == 1) st16(qa.k_out + tq * qa.ko_ts + (int64_t)hd[i] * qa.ko_hs + sub * 8, o);
        // the page id is first needed here; opaque_v keeps its wait (and the offset) from being
        // hoisted ahead of the q stores
        const int64_t kc = slot_finish(a.c, soff, opaque_v(page));
        if (kind[i] == 1 && kc >= 0) st_nt(a.c.k_cache + kc + (int64_t)hd[i] * a.c.head_stride + sub * 8, o);
        if (kind[i] == 2 && kc >= 0) st_nt(a.c.v_cache + kc + (int64_t)hd[i] * a.c.head_stride + sub * 8, X[i]);
      }
    }
  }
}


// ---------------------------------------------------------------- host side
bool heads_vec_ok(const uint16_t* p, int64_t ts, int64_t hs) {
  return aligned16(p) && ts % 8 == 0 && hs % 8 == 0;
}

// Waves per token, measured on configuration 3 (T = 68k, steady state): RoPE alone 6.18 TB/s
// with 4 (5.96 with 2, 5.46 with 1); append alone 5.33 with 2 (4.70 with 4, 5.15 with 1);
// fused 5.68 with 2 or 4 (5.46 with 1). Small batches (decode) use 4 to spread over the chip.
int pick_wpt(int64_t T, bool rope, bool append) {
  if (T < 2048 || (rope && !append)) return 4;
  return 2;
}

int fill_heads(RopeAppendArgs& a, pie_bf16* q, int64_t qts, int64_t qhs, pie_bf16* k, int64_t kts,
               int64_t khs, const pie_bf16* v, int64_t vts, int64_t vhs, int64_t T, int64_t Hq,
               int64_t Hkv, int64_t D, int64_t rd) {
  PIE_REQUIRE(T >= 0 && T < (1ll << 31), "rope/append: bad token count %lld", (long long)T);
  PIE_REQUIRE(Hq >= 0 && Hkv >= 0 && Hq + Hkv < (1 << 20) && D > 0 && D < (1 << 16),
              "rope/append: bad head shape Hq=%lld Hkv=%lld D=%lld", (long long)Hq, (long long)Hkv, (long long)D);
  PIE_REQUIRE(rd >= 0 && rd <= D && rd % 2 == 0 && rd / 2 <= kMaxPairs,
              "rope: rotary_dim=%lld must be even, <= head_dim=%lld and <= %d", (long long)rd,
              (long long)D, 2 * kMaxPairs);
  a.h = HeadsDesc{q, k, v, qts, qhs, kts, khs, vts, vhs, (int32_t)Hq, (int32_t)Hkv, (int32_t)D, (int32_t)rd};
  a.T = T;
  return PIE_HIP_OK;
}

int fill_cache(RopeAppendArgs& a, const int32_t* bidx, const int32_t* pos, const int32_t* kv_indices,
               const int32_t* kv_indptr, int64_t B, pie_bf16* kc, pie_bf16* vc, int64_t num_pages,
               int64_t ps, int64_t ss, int64_t hs, int64_t P) {
  PIE_REQUIRE(B >= 0 && num_pages >= 0 && P > 0 && P < (1 << 30), "append: bad batch/page shape");
  PIE_REQUIRE(a.T == 0 || (bidx && pos && kv_indptr && kc && vc && (kv_indices || num_pages == 0)),
              "append: null pointer");
  PIE_REQUIRE(ps >= 0 && ss >= 0 && hs >= 0, "append: negative cache stride");
  a.c = CacheDesc{bidx, pos, kv_indices, kv_indptr, kc, vc, B, num_pages, ps, ss, hs, (int32_t)P};
  return PIE_HIP_OK;
}

// Validates the arguments of pie_hip_qk_rmsnorm_rope_append and builds the kernel arguments;
// vec = the fused D = 128 kernel applies (16-byte aligned rows and cache), else the separate
// kernels give the same results. The inverse frequencies are copied into the arguments.
int qk_prepare(const QkRec& r, QkNormArgs& qa, bool& vec) {
  qa = QkNormArgs{};
  RopeAppendArgs& a = qa.r;
  int rc = fill_heads(a, const_cast<pie_bf16*>(r.q), r.q_ts, r.q_hs, const_cast<pie_bf16*>(r.k),
                      r.k_ts, r.k_hs, r.v, r.v_ts, r.v_hs, r.T, r.Hq, r.Hkv, r.D, r.D);
  if (rc) return rc;
  rc = fill_cache(a, r.batch_indices, r.positions, r.kv_indices, r.kv_indptr, r.batch_size,
                  r.k_cache, r.v_cache, r.num_pages, r.page_stride, r.slot_stride, r.head_stride,
                  r.page_size);
  if (rc) return rc;
  vec = false;
  if (r.T == 0 || r.Hq + r.Hkv == 0) return PIE_HIP_OK;
  PIE_REQUIRE(r.pos && r.inv_freq && (r.Hq == 0 || (r.q && r.q_out && r.qw)) &&
                  (r.Hkv == 0 || (r.k && r.v && r.k_out && r.kw)),
              "qk_rmsnorm_rope_append: null pointer");
  vec = r.D == 128 &&
        (r.Hq == 0 || (heads_vec_ok(r.q, r.q_ts, r.q_hs) && heads_vec_ok(r.q_out, r.qo_ts, r.qo_hs) &&
                       aligned16(r.qw))) &&
        (r.Hkv == 0 || (heads_vec_ok(r.k, r.k_ts, r.k_hs) && heads_vec_ok(r.v, r.v_ts, r.v_hs) &&
                        heads_vec_ok(r.k_out, r.ko_ts, r.ko_hs) && aligned16(r.kw) &&
                        aligned16(r.k_cache) && aligned16(r.v_cache) && r.page_stride % 8 == 0 &&
                        r.slot_stride % 8 == 0 && r.head_stride % 8 == 0));
  a.pos = r.pos;
  for (int64_t i = 0; i < r.D / 2; ++i) a.inv_freq[i] = r.inv_freq[i];
  qa.q_out = r.q_out;
  qa.k_out = r.k_out;
  qa.qo_ts = r.qo_ts;
  qa.qo_hs = r.qo_hs;
  qa.ko_ts = r.ko_ts;
  qa.ko_hs = r.ko_hs;
  qa.qw = r.qw;
  qa.kw = r.kw;
  qa.eps = r.eps;
  return PIE_HIP_OK;
}

}  // namespace
}  // namespace pie
