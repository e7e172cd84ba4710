// RoPE on ragged q/k (in place) and the paged KV append, separately and fused, for gfx950.
//
// RoPE semantics: pie/src/flashinfer_metal/kernels/metal_rope.metal:26-107 (the in-repo
// restatement of flashinfer.apply_rope_pos_ids_inplace / apply_llama31_rope_pos_ids_inplace,
// called at pie/src/pie_worker/model/llama3.py:660-669 and qwen3.py:665-670):
//   angle_i = float(pos[t]) * inv_freq[i];  x' = x cos - y sin;  y' = x sin + y cos
// with (x, y) = (v[i], v[i + rd/2]) (interleave = 0) or (v[2i], v[2i+1]) (interleave = 1),
// fp32 math, bf16 in/out. inv_freq is computed on the host in float64 (capi.hip).
//
// Append semantics: pie/src/flashinfer_metal/kernels/metal_append_paged_kv_cache.metal:23-107
// (flashinfer.append_paged_kv_cache at llama3.py:675-685): token t goes to slot p % P of page
// kv_indices[kv_indptr[b] + p / P]; tokens with an out-of-range batch index, logical page or
// physical page are skipped.
//
// Mapping. A group of W wavefronts owns one token (W = 1, 2 or 4; a 256-thread block holds
// 4/W tokens). The group first stages the token's cos/sin table (rd/2 angles) in LDS, one
// sincos per pair, shared by all Hq+Hkv heads. Then every lane walks 16-byte units:
//   q/k rope units: 8 pairs of one head (x chunk + y chunk, interleave = 0) or 4 pairs
//                   (one chunk, interleave = 1), rotated in registers and stored back;
//   k rope units in the fused kernel are also stored to the cache page (k is already in
//   registers, so the append costs no extra read of k);
//   k tail units (dims >= rd) and v units: 16-byte copies into the cache page.
// A token's Hkv*D row in a page is contiguous for NHD, so the 64 lanes of a wave write whole
// 1 KiB runs of a page: the scatter is coalesced per (page, slot).
#include <stdlib.h>

#include "rope_dev.h"

namespace pie {
namespace {

// Per-token unit layout of rope_append_vec: [q rope | k rope | k tail copy | v copy].
struct UnitGeom {
  int gsize, total, nq, nrope, nkt, uph, tail, dv, half, rd_off;
  int64_t q_hs, k_hs, v_hs;
  const uint16_t *qrow, *krow, *vrow, *safe;
};
template <int UB>
struct UnitBatch {
  uint4 X[UB], Y[UB];
  const uint16_t* P[UB];  // rope: x chunk (updated in place); copy: source
  int head[UB], e0[UB], kind[UB];  // kind: 0 q rope, 1 k rope, 2 k tail copy, 3 v copy, -1 none
};

// Loads the UB units u0, u0+gsize, ... of one token. All loads are issued unconditionally,
// with pointers chosen by selects (units past the end re-read `safe` and are discarded):
// loads inside divergent branches would each be followed by a wait, serialising the batch.
template <bool ROPE, bool APPEND, bool INTERLEAVE, int UB>
__device__ __forceinline__ void load_units(UnitBatch<UB>& b, const UnitGeom g, int u0) {
#pragma unroll
  for (int i = 0; i < UB; ++i) {
    const int u = u0 + i * g.gsize;
    const bool valid = u < g.total;
    const bool isq = ROPE && u < g.nq;
    const bool isrope = ROPE && u < g.nrope;
    const bool istail = APPEND && !isrope && u - g.nrope < g.nkt;
    const int base = isq ? 0 : (isrope ? g.nq : (istail ? g.nrope : g.nrope + g.nkt));
    const int div = isrope ? g.uph : (istail ? g.tail : g.dv);
    const int uu = valid ? u - base : 0;
    const int hd = uu / (div > 0 ? div : 1);
    const int e0 = (istail ? g.rd_off : 0) + (uu - hd * div) * 8;
    const uint16_t* src = isq ? g.qrow + (int64_t)hd * g.q_hs
                        : (isrope || istail) ? g.krow + (int64_t)hd * g.k_hs
                                             : g.vrow + (int64_t)hd * g.v_hs;
    src = valid ? src + e0 : g.safe;
    b.P[i] = src;
    b.head[i] = hd;
    b.e0[i] = e0;
    b.kind[i] = !valid ? -1 : (isq ? 0 : (isrope ? 1 : (istail ? 2 : 3)));
    b.X[i] = ld_nt(src);  // non-temporal: 5.33 vs 4.90 TB/s cached (steady state)
    if constexpr (ROPE && !INTERLEAVE) b.Y[i] = ld_nt(isrope ? src + g.half : src);
  }
}

template <bool ROPE, bool APPEND, bool INTERLEAVE, int UB>
__global__ __launch_bounds__(256) void rope_append_vec(RopeAppendArgs a) {
  __shared__ float2 tab[4][ROPE ? kMaxPairs : 1];
  const int wpt = a.wpt;
  const int tpb = 4 / wpt;
  const int slot = (threadIdx.x >> 6) / wpt;               // token slot in block
  const int gt = threadIdx.x - slot * wpt * 64;           // thread id inside the token group
  const int gsize = wpt * 64;
  const int64_t t = (int64_t)blockIdx.x * tpb + slot;
  const bool live = t < a.T;
  const HeadsDesc h = a.h;
  const CacheDesc cd = a.c;  // by value: no reference into the kernel-argument block
  const int half = h.rd >> 1;

  const int uph = ROPE ? (INTERLEAVE ? h.rd >> 3 : h.rd >> 4) : 0;  // rope units per head
  const int nq = ROPE ? h.Hq * uph : 0;
  const int nk = ROPE ? h.Hkv * uph : 0;
  const int tail = (h.D - (ROPE ? h.rd : 0)) >> 3;                 // k chunks past rd
  const int nkt = APPEND ? h.Hkv * tail : 0;
  const int dv = h.D >> 3;
  const int nv = APPEND ? h.Hkv * dv : 0;
  const int nrope = nq + nk;
  const int total = live ? nrope + nkt + nv : 0;

  // Wave-uniform token index (clamped for the padding slot of the last block): position and
  // page lookup become scalar loads that do not wait behind the vector data loads.
  const int64_t tq = uniform((int)(live ? t : 0));
  const uint16_t* qrow = h.q + tq * h.q_ts;
  const uint16_t* krow = h.k + tq * h.k_ts;
  const uint16_t* vrow = h.v + tq * h.v_ts;
  const uint16_t* safe = h.Hq > 0 ? qrow : krow;  // a valid 16-byte chunk of this token

  // Batches of UB units per lane, loaded by load_units (below).
  const UnitGeom g{gsize, total, nq, nrope, nkt, uph, tail, dv, half, ROPE ? h.rd : 0,
                   h.q_hs, h.k_hs, h.v_hs, qrow, krow, vrow, safe};
  UnitBatch<UB> b;
  // Latency order: the position, the first batch of data and the page lookup chain are all
  // requested before the cos/sin table is computed, so they overlap it.
  const int p = ROPE ? a.pos[tq] : 0;
  // This lane's cos/sin inputs (pair gt: a frequency, or a table row's two entries) are requested
  // before the data: vector loads complete in order, so inputs requested after the data would
  // hold the table (and the barrier behind it) until every data load had landed.
  const bool early = ROPE && live && half <= gsize && gt < half;
  const bool in_tab = a.cs && p >= 0 && (int64_t)p < a.cs_rows;
  float in0 = 0.f, in1 = 0.f;
  if (early) {
    if (a.cs) {
      const float* row = a.cs + (int64_t)(in_tab ? p : 0) * a.cs_ld;
      in0 = row[gt];
      in1 = row[half + gt];
    } else {
      in0 = a.inv_freq[gt];
    }
  }
  load_units<ROPE, APPEND, INTERLEAVE, UB>(b, g, gt);
  int64_t kc = -1;
  if constexpr (APPEND) {
    if (live) kc = slot_offset(cd, tq);
  }
  if constexpr (ROPE) {
    if (early) {
      tab[slot][gt] = a.cs ? (in_tab ? make_float2(in0, in1) : make_float2(1.f, 0.f)) : rope_pos_cs(p, in0);
    } else if (live && half > gsize) {
      for (int i = gt; i < half; i += gsize) tab[slot][i] = rope_cs(a, p, i, half);
    }
    __syncthreads();
  }
  if (!live) return;
  const float2* tb = tab[slot];

  for (int u0 = gt; u0 < total; u0 += gsize * UB) {
    if (u0 != gt) load_units<ROPE, APPEND, INTERLEAVE, UB>(b, g, u0);
#pragma unroll
    for (int i = 0; i < UB; ++i) {
      const int kind = b.kind[i];
      if (kind < 0) continue;
      uint16_t* P = const_cast<uint16_t*>(b.P[i]);
      const int64_t hoff = (int64_t)b.head[i] * cd.head_stride + b.e0[i];
      if (ROPE && kind <= 1) {
        if constexpr (!INTERLEAVE) {
          float x[8], y[8];
          unpack8(b.X[i], x);
          unpack8(b.Y[i], y);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float2 cs = tb[b.e0[i] + e];
            const float xr = rot_x(x[e], y[e], cs);
            const float yr = rot_y(x[e], y[e], cs);
            x[e] = xr;
            y[e] = yr;
          }
          const uint4 xo = pack8(x), yo = pack8(y);
          st_nt(P, xo);
          st_nt(P + half, yo);
          if (APPEND && kind == 1 && kc >= 0) {
            st_nt(cd.k_cache + kc + hoff, xo);
            st_nt(cd.k_cache + kc + hoff + half, yo);
          }
        } else {
          float f[8];
          unpack8(b.X[i], f);
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const float2 cs = tb[(b.e0[i] >> 1) + m];
            const float xr = rot_x(f[2 * m], f[2 * m + 1], cs);
            const float yr = rot_y(f[2 * m], f[2 * m + 1], cs);
            f[2 * m] = xr;
            f[2 * m + 1] = yr;
          }
          const uint4 o = pack8(f);
          st_nt(P, o);
          if (APPEND && kind == 1 && kc >= 0) st_nt(cd.k_cache + kc + hoff, o);
        }
      } else if (APPEND && kc >= 0) {
        st_nt((kind == 2 ? cd.k_cache : cd.v_cache) + kc + hoff, b.X[i]);
      }
    }
  }
}

__global__ __launch_bounds__(1024) void qk_norm_rope_append_d128(QkNormArgs qa) {
  prefetch_kernarg<kQkScalarBytes>(qa);
  qk_norm_rope_append_block(qa, blockIdx.x);
}

// ---------------------------------------------------------------- paged append, flattened
// One 16-byte chunk of k or v per thread over all T * 2 * Hkv * D/8 chunks (like the
// embedding gather): every thread loads its chunk, resolves its token's page (the three index
// loads are shared by the token's threads and hit in cache) and stores the chunk.
struct AppendFlatArgs {
  HeadsDesc h;
  CacheDesc c;
  uint32_t nunits;  // T * 2 * Hkv * (D/8)
  FastDiv upt;      // units per token: 2 * Hkv * (D/8)
  FastDiv cph;      // chunks per head: D/8
  uint32_t kunits;  // Hkv * (D/8): k chunks come first in a token
};

// U chunks per thread (units base + 256 i), every data load and page lookup issued before the
// first store. WU: a token's units fill whole waves (units per token a multiple of 64), so the
// token index is made wave-uniform and its three index loads become scalar loads.
template <int U, bool WU>
__global__ __launch_bounds__(256) void append_flat(AppendFlatArgs a) {
  const uint32_t base = blockIdx.x * (256u * U) + threadIdx.x;
  uint4 x[U];
  int64_t dst[U];
  const uint16_t* cache[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const uint32_t n = base + 256u * i;
    const bool valid = n < a.nunits;
    uint32_t t = a.upt.div(valid ? n : 0);
    if constexpr (WU) t = (uint32_t)uniform((int)t);
    uint32_t r = (valid ? n : 0) - t * a.upt.d;
    const bool isv = r >= a.kunits;
    if (isv) r -= a.kunits;
    const uint32_t head = a.cph.div(r), c = r - head * a.cph.d;
    const uint16_t* src = isv ? a.h.v + (int64_t)t * a.h.v_ts + (int64_t)head * a.h.v_hs
                              : a.h.k + (int64_t)t * a.h.k_ts + (int64_t)head * a.h.k_hs;
    x[i] = ld_nt(src + c * 8);
    const int64_t kc = valid ? slot_offset(a.c, t) : -1;
    dst[i] = kc < 0 ? -1 : kc + (int64_t)head * a.c.head_stride + c * 8;
    cache[i] = isv ? a.c.v_cache : a.c.k_cache;
  }
#pragma unroll
  for (int i = 0; i < U; ++i)
    if (dst[i] >= 0) st_nt(const_cast<uint16_t*>(cache[i]) + dst[i], x[i]);
}

// ---------------------------------------------------------------- scalar fallbacks
// Any alignment, any D / rd: one thread per (token, head, pair) or (token, head, element).
__global__ __launch_bounds__(256) void rope_scalar(RopeAppendArgs a) {
  const HeadsDesc& h = a.h;
  const int half = h.rd >> 1;
  const int64_t per_tok = (int64_t)(h.Hq + h.Hkv) * half;
  const int64_t n = a.T * per_tok;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / per_tok;
    const int rem = (int)(i - t * per_tok);
    const int head = rem / half, pr = rem - head * half;
    uint16_t* base = head < h.Hq ? h.q + t * h.q_ts + (int64_t)head * h.q_hs
                                 : h.k + t * h.k_ts + (int64_t)(head - h.Hq) * h.k_hs;
    uint16_t* px = base + (a.interleave ? 2 * pr : pr);
    uint16_t* py = base + (a.interleave ? 2 * pr + 1 : pr + half);
    const float2 csn = rope_cs(a, a.pos[t], pr, half);
    const float x = bf1(*px), y = bf1(*py);
    *px = to_bf1(rot_x(x, y, csn));
    *py = to_bf1(rot_y(x, y, csn));
  }
}

__global__ __launch_bounds__(256) void append_scalar(RopeAppendArgs a) {
  const HeadsDesc& h = a.h;
  const int64_t per_tok = (int64_t)h.Hkv * h.D;
  const int64_t n = a.T * per_tok;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / per_tok;
    const int rem = (int)(i - t * per_tok);
    const int head = rem / h.D, d = rem - head * h.D;
    const int64_t kc = slot_offset(a.c, t);
    if (kc < 0) continue;
    const int64_t o = kc + (int64_t)head * a.c.head_stride + d;
    a.c.k_cache[o] = h.k[t * h.k_ts + (int64_t)head * h.k_hs + d];
    a.c.v_cache[o] = h.v[t * h.v_ts + (int64_t)head * h.v_hs + d];
  }
}

// ---------------------------------------------------------------- host side
int launch(RopeAppendArgs& a, bool rope, bool append, int interleave, hipStream_t st,
           const char* name) {
  if (a.T == 0) return PIE_HIP_OK;
  const HeadsDesc& h = a.h;
  bool vec = h.D % 8 == 0 && (interleave ? h.rd % 8 == 0 : h.rd % 16 == 0);
  if (rope) vec = vec && (h.Hq == 0 || heads_vec_ok(h.q, h.q_ts, h.q_hs)) &&
                  (h.Hkv == 0 || heads_vec_ok(h.k, h.k_ts, h.k_hs));
  if (append)
    vec = vec && heads_vec_ok(h.k, h.k_ts, h.k_hs) && heads_vec_ok(h.v, h.v_ts, h.v_hs) &&
          aligned16(a.c.k_cache) && aligned16(a.c.v_cache) && a.c.page_stride % 8 == 0 &&
          a.c.slot_stride % 8 == 0 && a.c.head_stride % 8 == 0;
  if (vec && append && !rope) {  // flattened: 5.28 vs 5.11 TB/s per-token waves (cfg 3)
    const int64_t kunits = (int64_t)h.Hkv * (h.D / 8), nunits = a.T * 2 * kunits;
    if (nunits < (1ll << 31)) {
      AppendFlatArgs f{h, a.c, (uint32_t)nunits, FastDiv::make((uint32_t)(2 * kunits)),
                       FastDiv::make((uint32_t)(h.D / 8)), (uint32_t)kunits};
      // one 16-byte unit per thread (2 and 4 per thread measured slower)
      const bool wu = (2 * kunits) % 64 == 0;
      const dim3 grd((unsigned)((nunits + 255) / 256)), blk(256);
      if (wu) hipLaunchKernelGGL((append_flat<1, true>), grd, blk, 0, st, f);
      else hipLaunchKernelGGL((append_flat<1, false>), grd, blk, 0, st, f);
      return check_launch(name);
    }
  }
  if (vec) {
    a.wpt = pick_wpt(a.T, rope, append);
    const int tpb = 4 / a.wpt;
    const dim3 grd((unsigned)((a.T + tpb - 1) / tpb)), blk(256);
    // Units per lane for one token: one batch holds them all (capped at 8 per batch).
    const int uph = rope ? (interleave ? h.rd >> 3 : h.rd >> 4) : 0;
    const int64_t units = (int64_t)(h.Hq + h.Hkv) * uph +
                          (append ? (int64_t)h.Hkv * ((h.D - (rope ? h.rd : 0)) / 8 + h.D / 8) : 0);
    int64_t ub = (units + 64 * a.wpt - 1) / (64 * a.wpt);
    if (ub < 1) ub = 1;
    if (ub > 8) ub = 8;
#define PIE_RA_UB(R, A, I)                                                              \
  switch (ub) {                                                                           \
    case 1: hipLaunchKernelGGL((rope_append_vec<R, A, I, 1>), grd, blk, 0, st, a); break; \
    case 2: hipLaunchKernelGGL((rope_append_vec<R, A, I, 2>), grd, blk, 0, st, a); break; \
    case 3: hipLaunchKernelGGL((rope_append_vec<R, A, I, 3>), grd, blk, 0, st, a); break; \
    case 4: hipLaunchKernelGGL((rope_append_vec<R, A, I, 4>), grd, blk, 0, st, a); break; \
    case 5: hipLaunchKernelGGL((rope_append_vec<R, A, I, 5>), grd, blk, 0, st, a); break; \
    case 6: hipLaunchKernelGGL((rope_append_vec<R, A, I, 6>), grd, blk, 0, st, a); break; \
    case 7: hipLaunchKernelGGL((rope_append_vec<R, A, I, 7>), grd, blk, 0, st, a); break; \
    default: hipLaunchKernelGGL((rope_append_vec<R, A, I, 8>), grd, blk, 0, st, a); break; \
  }
    if (rope && append) { if (interleave) PIE_RA_UB(true, true, true) else PIE_RA_UB(true, true, false) }
    else if (rope) { if (interleave) PIE_RA_UB(true, false, true) else PIE_RA_UB(true, false, false) }
    else PIE_RA_UB(false, true, false)
#undef PIE_RA_UB
    return check_launch(name);
  }
  const dim3 blk(256);
  const int64_t cap = (int64_t)num_cus() * 64;
  if (rope && (h.Hq + h.Hkv) > 0 && h.rd > 0) {
    a.interleave = interleave;
    const int64_t n = a.T * (h.Hq + h.Hkv) * (h.rd / 2);
    const int64_t b = (n + 255) / 256;
    hipLaunchKernelGGL(rope_scalar, dim3((unsigned)(b < cap ? b : cap)), blk, 0, st, a);
    int rc = check_launch(name);
    if (rc) return rc;
  }
  if (append && h.Hkv > 0) {
    const int64_t n = a.T * h.Hkv * h.D;
    const int64_t b = (n + 255) / 256;
    hipLaunchKernelGGL(append_scalar, dim3((unsigned)(b < cap ? b : cap)), blk, 0, st, a);
    return check_launch(name);
  }
  return PIE_HIP_OK;
}

}  // namespace
}  // namespace pie

using namespace pie;

extern "C" int pie_hip_rope_inplace(pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride,
                                    pie_bf16* k, int64_t k_tok_stride, int64_t k_head_stride,
                                    const int32_t* pos, int64_t T, int64_t Hq, int64_t Hkv,
                                    int64_t D, int64_t rotary_dim, int interleave,
                                    const float* inv_freq, void* stream) {
  RopeAppendArgs a{};
  int rc = fill_heads(a, q, q_tok_stride, q_head_stride, k, k_tok_stride, k_head_stride, nullptr,
                      0, 0, T, Hq, Hkv, D, rotary_dim);
  if (rc) return rc;
  if (T == 0 || Hq + Hkv == 0 || rotary_dim == 0) return PIE_HIP_OK;
  PIE_REQUIRE(pos && inv_freq && (Hq == 0 || q) && (Hkv == 0 || k), "rope: null pointer");
  a.pos = pos;
  for (int64_t i = 0; i < rotary_dim / 2; ++i) a.inv_freq[i] = inv_freq[i];
  return launch(a, true, false, interleave ? 1 : 0, (hipStream_t)stream, "rope_inplace");
}

extern "C" int pie_hip_paged_kv_append(const pie_bf16* k, int64_t k_tok_stride, int64_t k_head_stride,
                                       const pie_bf16* v, int64_t v_tok_stride, int64_t v_head_stride,
                                       const int32_t* batch_indices, const int32_t* positions,
                                       const int32_t* kv_indices, const int32_t* kv_indptr,
                                       int64_t batch_size, pie_bf16* k_cache, pie_bf16* v_cache,
                                       int64_t num_pages, int64_t page_stride, int64_t slot_stride,
                                       int64_t head_stride, int64_t page_size, int64_t T,
                                       int64_t Hkv, int64_t D, void* stream) {
  RopeAppendArgs a{};
  int rc = fill_heads(a, nullptr, 0, 0, const_cast<pie_bf16*>(k), k_tok_stride, k_head_stride, v,
                      v_tok_stride, v_head_stride, T, 0, Hkv, D, 0);
  if (rc) return rc;
  rc = fill_cache(a, batch_indices, positions, kv_indices, kv_indptr, batch_size, k_cache, v_cache,
                  num_pages, page_stride, slot_stride, head_stride, page_size);
  if (rc) return rc;
  if (T == 0 || Hkv == 0) return PIE_HIP_OK;
  PIE_REQUIRE(k && v, "append: null k/v");
  return launch(a, false, true, 0, (hipStream_t)stream, "paged_kv_append");
}

extern "C" int pie_hip_rope_append(pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride,
                                   pie_bf16* k, int64_t k_tok_stride, int64_t k_head_stride,
                                   const pie_bf16* v, int64_t v_tok_stride, int64_t v_head_stride,
                                   const int32_t* pos, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                                   int64_t rotary_dim, int interleave, const float* inv_freq,
                                   const int32_t* batch_indices, const int32_t* positions,
                                   const int32_t* kv_indices, const int32_t* kv_indptr,
                                   int64_t batch_size, pie_bf16* k_cache, pie_bf16* v_cache,
                                   int64_t num_pages, int64_t page_stride, int64_t slot_stride,
                                   int64_t head_stride, int64_t page_size, void* stream) {
  RopeAppendArgs a{};
  int rc = fill_heads(a, q, q_tok_stride, q_head_stride, k, k_tok_stride, k_head_stride, v,
                      v_tok_stride, v_head_stride, T, Hq, Hkv, D, rotary_dim);
  if (rc) return rc;
  rc = fill_cache(a, batch_indices, positions, kv_indices, kv_indptr, batch_size, k_cache, v_cache,
                  num_pages, page_stride, slot_stride, head_stride, page_size);
  if (rc) return rc;
  if (T == 0 || Hq + Hkv == 0) return PIE_HIP_OK;
  PIE_REQUIRE(pos && inv_freq && (Hq == 0 || q) && (Hkv == 0 || (k && v)), "rope_append: null pointer");
  a.pos = pos;
  for (int64_t i = 0; i < rotary_dim / 2; ++i) a.inv_freq[i] = inv_freq[i];
  if (rotary_dim == 0) return launch(a, false, true, 0, (hipStream_t)stream, "rope_append");
  return launch(a, true, Hkv > 0, interleave ? 1 : 0, (hipStream_t)stream, "rope_append");
}

extern "C" int pie_hip_qk_rmsnorm_rope_append(
    const pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride, const pie_bf16* k,
    int64_t k_tok_stride, int64_t k_head_stride, const pie_bf16* v, int64_t v_tok_stride,
    int64_t v_head_stride, pie_bf16* q_out, int64_t qo_tok_stride, int64_t qo_head_stride,
    pie_bf16* k_out, int64_t ko_tok_stride, int64_t ko_head_stride, const pie_bf16* qw,
    const pie_bf16* kw, float eps, const int32_t* pos, int64_t T, int64_t Hq, int64_t Hkv,
    int64_t D, const float* inv_freq, const int32_t* batch_indices, const int32_t* positions,
    const int32_t* kv_indices, const int32_t* kv_indptr, int64_t batch_size, pie_bf16* k_cache,
    pie_bf16* v_cache, int64_t num_pages, int64_t page_stride, int64_t slot_stride,
    int64_t head_stride, int64_t page_size, void* stream) {
  const QkRec r{q, q_tok_stride, q_head_stride, k, k_tok_stride, k_head_stride, v, v_tok_stride,
                v_head_stride, q_out, qo_tok_stride, qo_head_stride, k_out, ko_tok_stride,
                ko_head_stride, qw, kw, eps, pos, T, Hq, Hkv, D, inv_freq, batch_indices, positions,
                kv_indices, kv_indptr, batch_size, k_cache, v_cache, num_pages, page_stride,
                slot_stride, head_stride, page_size};
  QkNormArgs qa{};
  bool vec = false;
  int rc = qk_prepare(r, qa, vec);
  if (rc) return rc;
  if (T == 0 || Hq + Hkv == 0) return PIE_HIP_OK;
  if (group_is_open()) return group_add_qk(r, stream);
  if (!vec) {  // same results through the separate kernels
    rc = pie_hip_qk_rmsnorm(q, q_tok_stride, q_head_stride, q_out, qo_tok_stride, qo_head_stride, k,
                            k_tok_stride, k_head_stride, k_out, ko_tok_stride, ko_head_stride, qw, kw,
                            T, Hq, Hkv, D, eps, stream);
    if (rc) return rc;
    return pie_hip_rope_append(q_out, qo_tok_stride, qo_head_stride, k_out, ko_tok_stride,
                               ko_head_stride, v, v_tok_stride, v_head_stride, pos, T, Hq, Hkv, D, D,
                               0, inv_freq, batch_indices, positions, kv_indices, kv_indptr,
                               batch_size, k_cache, v_cache, num_pages, page_stride, slot_stride,
                               head_stride, page_size, stream);
  }
  qa.r.wpt = pick_wpt(T, true, true);
  const int tpb = qa.r.wpt >= 4 ? 1 : 4 / qa.r.wpt;
  const int threads = qa.r.wpt >= 4 ? 64 * qa.r.wpt : 256;
  hipLaunchKernelGGL(qk_norm_rope_append_d128, dim3((unsigned)((T + tpb - 1) / tpb)), dim3(threads), 0,
                     (hipStream_t)stream, qa);
  return check_launch("qk_rmsnorm_rope_append");
}

extern "C" int pie_hip_rope_cos_sin_cache_inplace(pie_bf16* q, int64_t q_tok_stride,
                                                  int64_t q_head_stride, pie_bf16* k,
                                                  int64_t k_tok_stride, int64_t k_head_stride,
                                                  const int32_t* pos, int64_t T, int64_t Hq,
                                                  int64_t Hkv, int64_t D, int interleave,
                                                  const float* cos_sin_cache, int64_t cache_rows,
                                                  int64_t rotary_dim, int64_t cache_ld,
                                                  void* stream) {
  RopeAppendArgs a{};
  int rc = fill_heads(a, q, q_tok_stride, q_head_stride, k, k_tok_stride, k_head_stride, nullptr,
                      0, 0, T, Hq, Hkv, D, rotary_dim);
  if (rc) return rc;
  if (T == 0 || Hq + Hkv == 0 || rotary_dim == 0) return PIE_HIP_OK;
  PIE_REQUIRE(pos && cos_sin_cache && (Hq == 0 || q) && (Hkv == 0 || k), "rope_cos_sin_cache: null pointer");
  PIE_REQUIRE(cache_rows >= 0 && cache_ld >= rotary_dim, "rope_cos_sin_cache: bad cache shape");
  a.pos = pos;
  a.cs = cos_sin_cache;
  a.cs_rows = cache_rows;
  a.cs_ld = cache_ld;
  return launch(a, true, false, interleave ? 1 : 0, (hipStream_t)stream, "rope_cos_sin_cache");
}
