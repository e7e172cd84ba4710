// Runs every C-ABI entry point of the kernel library, built for the host by the emulator in
// include/hip/hip_runtime.h, on exact-size heap buffers under AddressSanitizer, and compares
// the results with the CPU oracle (oracle/oracle.c). TEST INFRASTRUCTURE.
//
//   emu_main <case>    case = norm | qk | silu | embed | rope | fused | decode | index | qkfused |
//                      variants | fastdiv | attn | prefill | sample | group | all | big
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <random>
#include <string>
#include <vector>

#include "../../include/pie_hip.h"
#include "../../pie_amd/csrc/common.h"

extern "C" {
void oracle_rmsnorm(const uint16_t*, int64_t, int64_t, const uint16_t*, uint16_t*, int64_t, int64_t,
                    int64_t, int64_t, int64_t, double);
void oracle_add_rmsnorm(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, uint16_t*,
                        int64_t, int64_t, double);
void oracle_silu_and_mul(const uint16_t*, int64_t, uint16_t*, int64_t, int64_t, int);
int64_t oracle_embedding(const int32_t*, int64_t, const uint16_t*, int64_t, int64_t, uint16_t*);
void oracle_inv_freq_std(double*, int64_t, double, double);
void oracle_rope(uint16_t*, int64_t, int64_t, uint16_t*, int64_t, int64_t, const int32_t*, int64_t,
                 int64_t, int64_t, int64_t, int, const double*);
int64_t oracle_append(const uint16_t*, int64_t, int64_t, const uint16_t*, int64_t, int64_t,
                      const int32_t*, const int32_t*, const int32_t*, const int32_t*, int64_t,
                      uint16_t*, uint16_t*, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                      int64_t, int64_t);
void oracle_gemma_rmsnorm(const uint16_t*, int64_t, int64_t, const uint16_t*, uint16_t*, int64_t,
                          int64_t, int64_t, int64_t, int64_t, double);
void oracle_gemma_add_rmsnorm(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, uint16_t*,
                              int64_t, int64_t, double);
void oracle_gelu_tanh_and_mul(const uint16_t*, int64_t, uint16_t*, int64_t, int64_t);
int64_t oracle_embedding_scaled(const int32_t*, int64_t, const uint16_t*, int64_t, int64_t, float,
                                uint16_t*);
void oracle_rope_cs(uint16_t*, int64_t, int64_t, uint16_t*, int64_t, int64_t, const int32_t*, int64_t,
                    int64_t, int64_t, int64_t, int, const float*, int64_t, int64_t);
void oracle_attention(const uint16_t*, int64_t, int64_t, const uint16_t*, const uint16_t*, int64_t,
                      int64_t, int64_t, const int32_t*, const int32_t*, const int32_t*, const int32_t*,
                      const uint8_t*, const int64_t*, int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                      double,
                      uint16_t*, int64_t, int64_t, double*, const float*);
void oracle_sample(const float*, int64_t, int64_t, int64_t, int, const int32_t*, const float*, const float*,
                   const double*, int32_t*, unsigned char*);
void oracle_scaled_softmax(const float*, int64_t, int64_t, const float*, double, double*);
void oracle_seq_lens(const int32_t*, const int32_t*, int64_t, int64_t, int32_t*);
void oracle_batch_indices_positions(const int32_t*, const int32_t*, int64_t, int64_t, int32_t*, int32_t*);
}

static std::mt19937 rng(1234);
static int failures = 0;

template <typename T>
struct Buf {  // exact-size heap allocation: any access past the end trips ASan
  T* p;
  size_t n;
  explicit Buf(size_t n_) : p((T*)malloc(n_ ? n_ * sizeof(T) : 1)), n(n_) {}
  ~Buf() { free(p); }
  Buf(const Buf&) = delete;
  T& operator[](size_t i) { return p[i]; }
};

static uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
static float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static void fill_normal(Buf<uint16_t>& b, float mean = 0.f, float std = 1.f) {
  std::normal_distribution<float> d(mean, std);
  for (size_t i = 0; i < b.n; ++i) b[i] = f2bf(d(rng));
}

static void check_close(const char* what, const uint16_t* got, const uint16_t* want, size_t n) {
  size_t bad = 0;
  for (size_t i = 0; i < n; ++i) {
    float g = bf2f(got[i]), w = bf2f(want[i]);
    if (!(fabsf(g - w) <= 2e-2f + 1e-2f * fabsf(w))) ++bad;
  }
  printf("  %-40s %s (%zu / %zu outside tolerance)\n", what, bad ? "FAIL" : "ok", bad, n);
  failures += bad != 0;
}
template <typename T>
static void check_equal(const char* what, const T* got, const T* want, size_t n) {
  size_t bad = 0;
  for (size_t i = 0; i < n; ++i) bad += got[i] != want[i];
  printf("  %-40s %s (%zu / %zu differ)\n", what, bad ? "FAIL" : "ok", bad, n);
  for (size_t i = 0, shown = 0; i < n && shown < 3; ++i)
    if (got[i] != want[i]) { printf("    [%zu] got %lld want %lld\n", i, (long long)got[i], (long long)want[i]); ++shown; }
  failures += bad != 0;
}
static void rc_ok(int rc, const char* what) {
  if (rc != 0) {
    printf("  %s returned %d: %s\n", what, rc, pie_hip_last_error());
    ++failures;
  }
}

// ---------------------------------------------------------------------------- norms
static void case_norm(int64_t T, int64_t H) {
  printf("norm T=%lld H=%lld\n", (long long)T, (long long)H);
  Buf<uint16_t> x(T * H), r(T * H), w(H), y(T * H), s(T * H), wy(T * H), ws(T * H);
  fill_normal(x);
  fill_normal(r);
  fill_normal(w, 1.f, 0.1f);
  rc_ok(pie_hip_rmsnorm(x.p, H, w.p, y.p, H, T, H, 1e-5f, nullptr), "rmsnorm");
  oracle_rmsnorm(x.p, H, 0, w.p, wy.p, H, 0, T, 1, H, 1e-5);
  check_close("rmsnorm", y.p, wy.p, T * H);
  rc_ok(pie_hip_fused_add_rmsnorm(x.p, H, r.p, H, s.p, H, y.p, H, w.p, T, H, 1e-5f, nullptr), "add");
  oracle_add_rmsnorm(x.p, r.p, w.p, ws.p, wy.p, T, H, 1e-5);
  check_equal("add_rmsnorm s", s.p, ws.p, T * H);
  check_close("add_rmsnorm y", y.p, wy.p, T * H);
}

static void case_qk(int64_t T, int64_t Hq, int64_t Hkv, int64_t D) {
  printf("qk_rmsnorm T=%lld Hq=%lld Hkv=%lld D=%lld\n", (long long)T, (long long)Hq, (long long)Hkv, (long long)D);
  const int64_t row = (Hq + 2 * Hkv) * D;
  Buf<uint16_t> qkv(T * row), qw(D), kw(D), qo(T * Hq * D), ko(T * Hkv * D), wq(T * Hq * D), wk(T * Hkv * D);
  fill_normal(qkv);
  fill_normal(qw, 1.f, .1f);
  fill_normal(kw, 1.f, .1f);
  rc_ok(pie_hip_qk_rmsnorm(qkv.p, row, D, qo.p, Hq * D, D, qkv.p + Hq * D, row, D, ko.p, Hkv * D, D,
                           qw.p, kw.p, T, Hq, Hkv, D, 1e-6f, nullptr), "qk_rmsnorm");
  oracle_rmsnorm(qkv.p, row, D, qw.p, wq.p, Hq * D, D, T, Hq, D, 1e-6);
  oracle_rmsnorm(qkv.p + Hq * D, row, D, kw.p, wk.p, Hkv * D, D, T, Hkv, D, 1e-6);
  check_close("q", qo.p, wq.p, T * Hq * D);
  check_close("k", ko.p, wk.p, T * Hkv * D);
}

// ---------------------------------------------------------------------------- silu, embed
static void case_silu(int64_t T, int64_t I) {
  printf("silu T=%lld I=%lld\n", (long long)T, (long long)I);
  Buf<uint16_t> gu(T * 2 * I), o(T * I), wo(T * I);
  fill_normal(gu, 0.f, 1.414f);
  rc_ok(pie_hip_silu_and_mul(gu.p, 2 * I, o.p, I, T, I, nullptr), "silu");
  oracle_silu_and_mul(gu.p, 2 * I, wo.p, T, I, 0);
  check_close("silu_and_mul", o.p, wo.p, T * I);
}

static void case_embed(int64_t V, int64_t H, int64_t T) {
  printf("embedding V=%lld H=%lld T=%lld\n", (long long)V, (long long)H, (long long)T);
  Buf<uint16_t> W(V * H), o(T * H), wo(T * H);
  Buf<int32_t> ids(T);
  fill_normal(W);
  std::uniform_int_distribution<int> d(0, (int)V - 1);
  for (int64_t t = 0; t < T; ++t) ids[t] = d(rng);
  if (T > 2) ids[1] = (int32_t)V, ids[2] = -5;
  rc_ok(pie_hip_embedding(ids.p, T, W.p, V, H, H, o.p, H, nullptr), "embedding");
  oracle_embedding(ids.p, T, W.p, V, H, wo.p);
  check_equal("embedding", o.p, wo.p, T * H);
}

// ---------------------------------------------------------------------------- paged batch
struct Paged {
  int64_t B, T, pool, P;
  std::vector<int32_t> kv_indptr, kv_indices, last, qo, bidx, pos, seq;
};
static Paged make_paged(int64_t B, int64_t P, int lo_ctx, int hi_ctx, int lo_new, int hi_new) {
  Paged p;
  p.B = B;
  p.P = P;
  std::uniform_int_distribution<int> dc(lo_ctx, hi_ctx), dn(lo_new, hi_new);
  std::vector<int> ctx(B), nw(B);
  int64_t pages = 0;
  p.kv_indptr.push_back(0);
  p.qo.push_back(0);
  for (int64_t b = 0; b < B; ++b) {
    ctx[b] = dc(rng);
    nw[b] = dn(rng);
    int64_t tot = ctx[b] + nw[b], np = (tot + P - 1) / P;
    pages += np;
    p.kv_indptr.push_back((int32_t)pages);
    p.last.push_back(np ? (int32_t)(tot - P * (np - 1)) : 0);
    p.qo.push_back(p.qo.back() + nw[b]);
    p.seq.push_back((int32_t)tot);
    for (int i = 0; i < nw[b]; ++i) {
      p.bidx.push_back((int32_t)b);
      p.pos.push_back(ctx[b] + i);
    }
  }
  p.pool = pages + 3;
  std::vector<int32_t> perm(p.pool);
  for (int64_t i = 0; i < p.pool; ++i) perm[i] = (int32_t)i;
  std::shuffle(perm.begin(), perm.end(), rng);
  p.kv_indices.assign(perm.begin(), perm.begin() + pages);
  p.T = p.qo.back();
  return p;
}

template <typename T>
static void copy_in(Buf<T>& b, const std::vector<T>& v) { memcpy(b.p, v.data(), v.size() * sizeof(T)); }

static void case_rope_append(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int lo_ctx, int hi_ctx,
                             int lo_new, int hi_new, bool fused, int64_t rd = 0, int interleave = 0) {
  if (rd == 0) rd = D;
  Paged pg = make_paged(B, 16, lo_ctx, hi_ctx, lo_new, hi_new);
  const int64_t T = pg.T, row = (Hq + 2 * Hkv) * D, P = pg.P;
  printf("%s B=%lld T=%lld Hq=%lld Hkv=%lld D=%lld rd=%lld il=%d pool=%lld\n",
         fused ? "rope+append fused" : "rope, append", (long long)B, (long long)T, (long long)Hq,
         (long long)Hkv, (long long)D, (long long)rd, interleave, (long long)pg.pool);
  Buf<uint16_t> qkv(T * row), ref(T * row);
  fill_normal(qkv);
  memcpy(ref.p, qkv.p, T * row * 2);
  const int64_t page_elems = 2 * P * Hkv * D;
  Buf<uint16_t> cache(pg.pool * page_elems), wcache(pg.pool * page_elems);
  for (size_t i = 0; i < cache.n; ++i) cache[i] = wcache[i] = 0x7fa5;
  Buf<int32_t> bidx(T), pos(T), kvi(pg.kv_indices.size()), kvp(B + 1);
  copy_in(bidx, pg.bidx);
  copy_in(pos, pg.pos);
  copy_in(kvi, pg.kv_indices);
  copy_in(kvp, pg.kv_indptr);
  float inv[256];
  double invd[256];
  rc_ok(pie_hip_rope_inv_freq(inv, rd, 1.f, 1e6f), "inv_freq");
  oracle_inv_freq_std(invd, rd, 1.0, 1e6);
  uint16_t* q = qkv.p;
  uint16_t* k = qkv.p + Hq * D;
  uint16_t* v = qkv.p + (Hq + Hkv) * D;
  if (fused) {
    rc_ok(pie_hip_rope_append(q, row, D, k, row, D, v, row, D, pos.p, T, Hq, Hkv, D, rd, interleave, inv, bidx.p,
                              pos.p, kvi.p, kvp.p, B, cache.p, cache.p + P * Hkv * D, pg.pool,
                              page_elems, Hkv * D, D, P, nullptr), "rope_append");
  } else {
    rc_ok(pie_hip_rope_inplace(q, row, D, k, row, D, pos.p, T, Hq, Hkv, D, rd, interleave, inv, nullptr), "rope");
    rc_ok(pie_hip_paged_kv_append(k, row, D, v, row, D, bidx.p, pos.p, kvi.p, kvp.p, B, cache.p,
                                  cache.p + P * Hkv * D, pg.pool, page_elems, Hkv * D, D, P, T, Hkv, D,
                                  nullptr), "append");
  }
  oracle_rope(ref.p, row, D, ref.p + Hq * D, row, D, pos.p, T, Hq, Hkv, rd, interleave, invd);
  check_close("q/k rotated (v untouched)", qkv.p, ref.p, T * row);
  oracle_append(qkv.p + Hq * D, row, D, qkv.p + (Hq + Hkv) * D, row, D, bidx.p, pos.p, kvi.p, kvp.p, B,
                wcache.p, wcache.p + P * Hkv * D, pg.pool, page_elems, Hkv * D, D, P, T, Hkv, D);
  check_equal("cache", cache.p, wcache.p, cache.n);
}

// q/k RMSNorm + RoPE + append in one kernel vs the three separate entry points (bit-exact).
static void case_qk_fused(int64_t B, int64_t Hq, int64_t Hkv, int64_t D) {
  Paged pg = make_paged(B, 16, 100, 3000, 1, 1);
  const int64_t T = pg.T, row = (Hq + 2 * Hkv) * D, P = pg.P, page_elems = 2 * P * Hkv * D;
  printf("qk_rmsnorm_rope_append B=%lld Hq=%lld Hkv=%lld D=%lld\n", (long long)B, (long long)Hq,
         (long long)Hkv, (long long)D);
  Buf<uint16_t> qkv(T * row), qw(D), kw(D), qa(T * Hq * D), ka(T * Hkv * D), qb(T * Hq * D), kb(T * Hkv * D);
  Buf<uint16_t> ca(pg.pool * page_elems), cb(pg.pool * page_elems);
  fill_normal(qkv);
  fill_normal(qw, 1.f, .1f);
  fill_normal(kw, 1.f, .1f);
  for (size_t i = 0; i < ca.n; ++i) ca[i] = cb[i] = 0x7fa5;
  Buf<int32_t> bidx(T), pos(T), kvi(pg.kv_indices.size()), kvp(B + 1);
  copy_in(bidx, pg.bidx);
  copy_in(pos, pg.pos);
  copy_in(kvi, pg.kv_indices);
  copy_in(kvp, pg.kv_indptr);
  float inv[256];
  rc_ok(pie_hip_rope_inv_freq(inv, D, 1.f, 1e6f), "inv_freq");
  const uint16_t *q = qkv.p, *k = qkv.p + Hq * D, *v = qkv.p + (Hq + Hkv) * D;
  rc_ok(pie_hip_qk_rmsnorm_rope_append(q, row, D, k, row, D, v, row, D, qa.p, Hq * D, D, ka.p, Hkv * D, D,
                                       qw.p, kw.p, 1e-6f, pos.p, T, Hq, Hkv, D, inv, bidx.p, pos.p, kvi.p,
                                       kvp.p, B, ca.p, ca.p + P * Hkv * D, pg.pool, page_elems, Hkv * D,
                                       D, P, nullptr), "fused");
  rc_ok(pie_hip_qk_rmsnorm(q, row, D, qb.p, Hq * D, D, k, row, D, kb.p, Hkv * D, D, qw.p, kw.p, T, Hq,
                           Hkv, D, 1e-6f, nullptr), "qk_rmsnorm");
  rc_ok(pie_hip_rope_append(qb.p, Hq * D, D, kb.p, Hkv * D, D, v, row, D, pos.p, T, Hq, Hkv, D, D, 0,
                            inv, bidx.p, pos.p, kvi.p, kvp.p, B, cb.p, cb.p + P * Hkv * D, pg.pool,
                            page_elems, Hkv * D, D, P, nullptr), "rope_append");
  check_equal("q fused == separate", qa.p, qb.p, qa.n);
  check_equal("k fused == separate", ka.p, kb.p, ka.n);
  check_equal("cache fused == separate", ca.p, cb.p, ca.n);
}

// Gemma norms, GELU-tanh-and-mul, scaled embedding, RoPE from a cos/sin table.
static void case_variants(int64_t T, int64_t H, int64_t Hq, int64_t Hkv, int64_t D, int64_t I) {
  printf("variants T=%lld H=%lld Hq=%lld Hkv=%lld D=%lld I=%lld\n", (long long)T, (long long)H,
         (long long)Hq, (long long)Hkv, (long long)D, (long long)I);
  {
    Buf<uint16_t> x(T * H), r(T * H), w(H), y(T * H), s(T * H), wy(T * H), ws(T * H);
    fill_normal(x);
    fill_normal(r);
    fill_normal(w, 0.f, .5f);
    rc_ok(pie_hip_gemma_rmsnorm(x.p, H, w.p, y.p, H, T, H, 1e-6f, nullptr), "gemma_rmsnorm");
    oracle_gemma_rmsnorm(x.p, H, 0, w.p, wy.p, H, 0, T, 1, H, 1e-6);
    check_equal("gemma rmsnorm", y.p, wy.p, T * H);
    rc_ok(pie_hip_gemma_fused_add_rmsnorm(x.p, H, r.p, H, s.p, H, y.p, H, w.p, T, H, 1e-6f, nullptr),
          "gemma_add");
    oracle_gemma_add_rmsnorm(x.p, r.p, w.p, ws.p, wy.p, T, H, 1e-6);
    check_equal("gemma add s", s.p, ws.p, T * H);
    check_equal("gemma add y", y.p, wy.p, T * H);
  }
  const int64_t row = (Hq + 2 * Hkv) * D;
  {
    Buf<uint16_t> qkv(T * row), qw(D), kw(D), qo(T * Hq * D), ko(T * Hkv * D), wq(T * Hq * D),
        wk(T * Hkv * D);
    fill_normal(qkv);
    fill_normal(qw, 0.f, .5f);
    fill_normal(kw, 0.f, .5f);
    rc_ok(pie_hip_gemma_qk_rmsnorm(qkv.p, row, D, qo.p, Hq * D, D, qkv.p + Hq * D, row, D, ko.p,
                                   Hkv * D, D, qw.p, kw.p, T, Hq, Hkv, D, 1e-6f, nullptr), "gemma_qk");
    oracle_gemma_rmsnorm(qkv.p, row, D, qw.p, wq.p, Hq * D, D, T, Hq, D, 1e-6);
    oracle_gemma_rmsnorm(qkv.p + Hq * D, row, D, kw.p, wk.p, Hkv * D, D, T, Hkv, D, 1e-6);
    check_equal("gemma q", qo.p, wq.p, T * Hq * D);
    check_equal("gemma k", ko.p, wk.p, T * Hkv * D);
  }
  {
    Buf<uint16_t> gu(T * 2 * I), o(T * I), wo(T * I);
    fill_normal(gu, 0.f, 1.414f);
    rc_ok(pie_hip_gelu_tanh_and_mul(gu.p, 2 * I, o.p, I, T, I, nullptr), "gelu");
    oracle_gelu_tanh_and_mul(gu.p, 2 * I, wo.p, T, I);
    check_close("gelu_tanh_and_mul", o.p, wo.p, T * I);
  }
  {
    const int64_t V = 37;
    Buf<uint16_t> W(V * H), o(T * H), wo(T * H);
    Buf<int32_t> ids(T);
    fill_normal(W);
    std::uniform_int_distribution<int> d(0, (int)V - 1);
    for (int64_t t = 0; t < T; ++t) ids[t] = d(rng);
    if (T > 2) ids[1] = (int32_t)V, ids[2] = -1;
    const float scale = sqrtf((float)H);
    rc_ok(pie_hip_embedding_scaled(ids.p, T, W.p, V, H, H, o.p, H, scale, nullptr), "embed_scaled");
    oracle_embedding_scaled(ids.p, T, W.p, V, H, scale, wo.p);
    check_equal("embedding scaled", o.p, wo.p, T * H);
  }
  for (int il = 0; il < 4; ++il) {
    const int64_t rd = il < 2 ? D : D / 2, rows = 64, ld = rd + 8;  // padded table rows: ld > rotary_dim
    Buf<uint16_t> qkv(T * row), ref(T * row);
    Buf<float> cs(rows * ld);
    Buf<int32_t> pos(T);
    fill_normal(qkv);
    memcpy(ref.p, qkv.p, T * row * 2);
    for (int64_t p = 0; p < rows; ++p)
      for (int64_t i = 0; i < ld; ++i) {
        const double f = pow(10000.0, -2.0 * (double)(i % (rd / 2)) / (double)rd);
        cs[p * ld + i] = i >= rd ? NAN : i < rd / 2 ? (float)cos(p * f) : (float)sin(p * f);
      }
    std::uniform_int_distribution<int> dp(0, (int)rows - 1);
    for (int64_t t = 0; t < T; ++t) pos[t] = dp(rng);
    if (T > 2) pos[0] = (int32_t)rows, pos[2] = -3;  // out of the table: left unrotated
    rc_ok(pie_hip_rope_cos_sin_cache_inplace(qkv.p, row, D, qkv.p + Hq * D, row, D, pos.p, T, Hq, Hkv,
                                             D, il & 1, cs.p, rows, rd, ld, nullptr), "rope_cs");
    oracle_rope_cs(ref.p, row, D, ref.p + Hq * D, row, D, pos.p, T, Hq, Hkv, rd, il & 1, cs.p, rows, ld);
    const char* names[] = {"rope cos/sin table", "rope cos/sin table (interleaved)",
                           "rope cos/sin table, rd = D/2", "rope cos/sin table, rd = D/2, interleaved"};
    check_close(names[il], qkv.p, ref.p, T * row);
  }
}

// ---------------------------------------------------------------------------- attention
// Paged decode attention: contexts in [lo, hi], random page permutation of an exact-size pool,
// NHD cache; `chunk` = splits per request (0 = the library's choice).
static void fill_sinks(Buf<float>& sk) {
  std::uniform_real_distribution<float> du(-3.f, 8.f);  // from negligible to dominant
  for (size_t i = 0; i < sk.n; ++i) sk[i] = du(rng);
}

static void case_attn_decode(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t P, int lo, int hi,
                             int64_t chunk, int64_t window = -1, bool with_sinks = false) {
  printf("attn_decode B=%lld Hq=%lld Hkv=%lld D=%lld P=%lld ctx=[%d,%d] chunk=%lld window=%lld\n", (long long)B,
         (long long)Hq, (long long)Hkv, (long long)D, (long long)P, lo, hi, (long long)chunk, (long long)window);
  std::vector<int32_t> len(B), indptr(B + 1, 0), last(B);
  std::uniform_int_distribution<int> dl(lo, hi);
  for (int64_t b = 0; b < B; ++b) {
    len[b] = dl(rng);
    const int np = (len[b] + P - 1) / P;
    indptr[b + 1] = indptr[b] + np;
    last[b] = np ? len[b] - (np - 1) * (int)P : 0;
  }
  const int64_t pages = std::max<int64_t>(indptr[B], 1);
  Buf<int32_t> ip(B + 1), idx(pages), ll(B);
  std::vector<int32_t> perm(pages);
  for (int64_t i = 0; i < pages; ++i) perm[i] = (int32_t)i;
  std::shuffle(perm.begin(), perm.end(), rng);
  for (int64_t i = 0; i < pages; ++i) idx[i] = perm[i];
  for (int64_t b = 0; b <= B; ++b) ip[b] = indptr[b];
  for (int64_t b = 0; b < B; ++b) ll[b] = last[b];
  const int64_t page_elems = 2 * P * Hkv * D;
  Buf<uint16_t> cache(pages * page_elems), q(B * Hq * D), out(B * Hq * D), want(B * Hq * D);
  fill_normal(cache);
  fill_normal(q);
  Buf<float> sk(Hq);
  fill_sinks(sk);
  const float* sinks_ptr = with_sinks ? sk.p : nullptr;
  if (with_sinks) printf("  with attention sinks\n");
  int64_t splits = chunk;
  if (splits <= 0) rc_ok(pie_hip_attention_decode_plan(B, Hkv, hi, 4, &splits), "decode_plan");
  Buf<float> ws(std::max<int64_t>(B * splits * Hq * (D + 1), 1));
  rc_ok(pie_hip_attention_decode(q.p, Hq * D, D, cache.p, cache.p + P * Hkv * D, page_elems, Hkv * D, D,
                                 pages, ip.p, idx.p, ll.p, B, Hq, Hkv, D, P, 1.f / sqrtf((float)D),
                                 window, sinks_ptr, splits, ws.p, (int64_t)(ws.n * 4), out.p, Hq * D, D,
                                 nullptr),
        "attention_decode");
  std::vector<int32_t> qo(B + 1);
  for (int64_t b = 0; b <= B; ++b) qo[b] = (int32_t)b;
  oracle_attention(q.p, Hq * D, D, cache.p, cache.p + P * Hkv * D, page_elems, Hkv * D, D, qo.data(), ip.p,
                   idx.p, ll.p, nullptr, nullptr, 1, window, B, Hq, Hkv, D, P, 1.0 / sqrt((double)D), want.p, Hq * D,
                   D, nullptr, sinks_ptr);
  printf("  splits %lld\n", (long long)splits);
  check_close("decode attention", out.p, want.p, B * Hq * D);
  // tighter: attention outputs are averages (|o| < 1 here), so a dropped or doubled token
  // shows as an error of ~1/kv_len; rounding P to bf16 stays well below 1/256
  float worst = 0.f;
  for (int64_t i = 0; i < B * Hq * D; ++i) {
    const float w = bf2f(want[i]);
    worst = fmaxf(worst, fabsf(bf2f(out[i]) - w) / (1.f / 256 + fabsf(w) / 128));
  }
  printf("  max |err| / (1/256 + |want|/128) = %.3f\n", worst);
  failures += !(worst <= 1.f);
}

// The allocation-free decode entry point against the workspace one, bit for bit: two calls in
// a row, the second smaller, so partials left in the shared static array must not leak.
static void case_attn_decode_noalloc() {
  printf("attn_decode_noalloc\n");
  for (int pass = 0; pass < 2; ++pass) {
    const int64_t B = pass ? 2 : 5, Hq = 8, Hkv = 2, D = 128, P = 16, S = 3;
    std::vector<int32_t> len(B), indptr(B + 1, 0), last(B);
    std::uniform_int_distribution<int> dl(pass ? 1 : 300, pass ? 200 : 700);
    for (int64_t b = 0; b < B; ++b) {
      len[b] = dl(rng);
      const int np = (len[b] + P - 1) / P;
      indptr[b + 1] = indptr[b] + np;
      last[b] = len[b] - (np - 1) * (int)P;
    }
    const int64_t pages = indptr[B], page_elems = 2 * P * Hkv * D;
    Buf<int32_t> ip(B + 1), idx(pages), ll(B);
    for (int64_t i = 0; i < pages; ++i) idx[i] = (int32_t)(pages - 1 - i);
    for (int64_t b = 0; b <= B; ++b) ip[b] = indptr[b];
    for (int64_t b = 0; b < B; ++b) ll[b] = last[b];
    Buf<uint16_t> cache(pages * page_elems), q(B * Hq * D), a(B * Hq * D), b2(B * Hq * D);
    fill_normal(cache);
    fill_normal(q);
    Buf<float> ws(B * S * Hq * (D + 1));
    rc_ok(pie_hip_attention_decode(q.p, Hq * D, D, cache.p, cache.p + P * Hkv * D, page_elems, Hkv * D, D,
                                   pages, ip.p, idx.p, ll.p, B, Hq, Hkv, D, P, 0.09f, -1, nullptr, S, ws.p,
                                   (int64_t)(ws.n * 4), a.p, Hq * D, D, nullptr), "decode");
    rc_ok(pie_hip_attention_decode_noalloc(q.p, Hq * D, D, cache.p, cache.p + P * Hkv * D, page_elems,
                                           Hkv * D, D, pages, ip.p, idx.p, ll.p, B, Hq, Hkv, D, P, 0.09f,
                                           -1, nullptr, S, b2.p, Hq * D, D, nullptr), "decode_noalloc");
    check_equal("noalloc decode == workspace decode", b2.p, a.p, a.n);
  }
  const int rc = pie_hip_attention_decode_noalloc(nullptr, 0, 0, nullptr, nullptr, 0, 0, 0, 1, nullptr,
                                                  nullptr, nullptr, 256, 32, 8, 128, 16, 1.f, -1, nullptr, 64,
                                                  nullptr, 0, 0, nullptr);
  if (rc != PIE_HIP_EINVAL) { printf("  FAIL: oversize noalloc decode accepted\n"); ++failures; }
}

// The grouped launch (embedding -> add + RMSNorm, q/k prologue, SiLU-and-mul in one kernel)
// against the separate entry points, bit for bit.
static void case_group(int64_t B, int64_t H, int64_t I, int64_t V, bool gelu) {
  const int64_t Hq = 8, Hkv = 2, D = 128;
  Paged pg = make_paged(B, 16, 10, 300, 1, 1);
  const int64_t T = pg.T, row = (Hq + 2 * Hkv) * D, P = pg.P, page_elems = 2 * P * Hkv * D;
  printf("group T=%lld H=%lld I=%lld V=%lld gelu=%d\n", (long long)T, (long long)H, (long long)I,
         (long long)V, (int)gelu);
  Buf<uint16_t> W(V * H), res(T * H), wn(H), qkv(T * row), qw(D), kw(D), gu(T * 2 * I);
  fill_normal(W);
  fill_normal(res);
  fill_normal(wn, 1.f, .1f);
  fill_normal(qkv);
  fill_normal(qw, 1.f, .1f);
  fill_normal(kw, 1.f, .1f);
  fill_normal(gu);
  Buf<int32_t> ids(T), bidx(T), pos(T), kvi(pg.kv_indices.size()), kvp(B + 1);
  std::uniform_int_distribution<int> di(-2, (int)V + 1);  // a few out-of-range ids: zero rows
  for (int64_t t = 0; t < T; ++t) ids[t] = di(rng);
  copy_in(bidx, pg.bidx);
  copy_in(pos, pg.pos);
  copy_in(kvi, pg.kv_indices);
  copy_in(kvp, pg.kv_indptr);
  float inv[256];
  rc_ok(pie_hip_rope_inv_freq(inv, D, 1.f, 1e6f), "inv_freq");
  const uint16_t *q = qkv.p, *k = qkv.p + Hq * D, *v = qkv.p + (Hq + Hkv) * D;
  struct Out {
    Buf<uint16_t> hid, s, y, qo, ko, cache, act;
    Out(int64_t T, int64_t H, int64_t Hq, int64_t Hkv, int64_t D, int64_t pool, int64_t pe, int64_t I)
        : hid(T * H), s(T * H), y(T * H), qo(T * Hq * D), ko(T * Hkv * D), cache(pool * pe), act(T * I) {
      for (size_t i = 0; i < cache.n; ++i) cache[i] = 0x7fa5;
    }
  };
  Out a(T, H, Hq, Hkv, D, pg.pool, page_elems, I), b(T, H, Hq, Hkv, D, pg.pool, page_elems, I);
  auto run = [&](Out& o) {
    rc_ok(pie_hip_embedding(ids.p, T, W.p, V, H, H, o.hid.p, H, nullptr), "embedding");
    rc_ok(pie_hip_fused_add_rmsnorm(o.hid.p, H, res.p, H, o.s.p, H, o.y.p, H, wn.p, T, H, 1e-6f, nullptr),
          "add_rmsnorm");
    rc_ok(pie_hip_qk_rmsnorm_rope_append(q, row, D, k, row, D, v, row, D, o.qo.p, Hq * D, D, o.ko.p,
                                         Hkv * D, D, qw.p, kw.p, 1e-6f, pos.p, T, Hq, Hkv, D, inv, bidx.p,
                                         pos.p, kvi.p, kvp.p, B, o.cache.p, o.cache.p + P * Hkv * D,
                                         pg.pool, page_elems, Hkv * D, D, P, nullptr), "qk");
    rc_ok((gelu ? pie_hip_gelu_tanh_and_mul : pie_hip_silu_and_mul)(gu.p, 2 * I, o.act.p, I, T, I, nullptr),
          "act");
  };
  run(a);
  rc_ok(pie_hip_group_begin(), "group_begin");
  run(b);
  rc_ok(pie_hip_group_end(nullptr), "group_end");
  check_equal("group hidden", b.hid.p, a.hid.p, a.hid.n);
  check_equal("group residual", b.s.p, a.s.p, a.s.n);
  check_equal("group normed", b.y.p, a.y.p, a.y.n);
  check_equal("group q", b.qo.p, a.qo.p, a.qo.n);
  check_equal("group k", b.ko.p, a.ko.p, a.ko.n);
  check_equal("group cache", b.cache.p, a.cache.p, a.cache.n);
  check_equal("group act", b.act.p, a.act.p, a.act.n);
  // the same group saved and launched twice (the second over cleared outputs)
  Out c(T, H, Hq, Hkv, D, pg.pool, page_elems, I);
  void* saved = nullptr;
  rc_ok(pie_hip_group_begin(), "group_begin");
  run(c);
  rc_ok(pie_hip_group_save(nullptr, &saved), "group_save");
  for (int rep = 0; rep < 2; ++rep) {
    for (size_t i = 0; i < c.act.n; ++i) c.act[i] = 0;
    for (size_t i = 0; i < c.y.n; ++i) c.y[i] = 0;
    for (size_t i = 0; i < c.cache.n; ++i) c.cache[i] = 0x7fa5;
    rc_ok(pie_hip_group_launch(saved, nullptr), "group_launch");
    check_equal("saved group normed", c.y.p, a.y.p, a.y.n);
    check_equal("saved group cache", c.cache.p, a.cache.p, a.cache.n);
    check_equal("saved group act", c.act.p, a.act.p, a.act.n);
  }
  pie_hip_group_free(saved);
  // a hazard (the activation writes the norm's residual input) is rejected without launching
  rc_ok(pie_hip_group_begin(), "group_begin");
  rc_ok(pie_hip_fused_add_rmsnorm(b.hid.p, H, res.p, H, b.s.p, H, b.y.p, H, wn.p, T, H, 1e-6f, nullptr), "n");
  rc_ok(pie_hip_silu_and_mul(gu.p, 2 * I, res.p, I, T, std::min<int64_t>(I, H), nullptr), "a");
  if (pie_hip_group_end(nullptr) != PIE_HIP_EINVAL) { printf("  FAIL: hazard accepted\n"); ++failures; }
  check_equal("rejected group launched nothing", b.s.p, a.s.p, a.s.n);
  if (pie_hip_group_end(nullptr) != PIE_HIP_EINVAL) { printf("  FAIL: end without begin\n"); ++failures; }
}

// Paged prefill attention: requests with ctx in [0, cmax] cached tokens and qo in [0, qmax] new
// query tokens; mode 0 full, 1 causal, 2 a random custom mask.
static void case_attn_prefill(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t P, int cmax, int qmax,
                              int mode, bool causal_mask = false, int64_t window = -1,
                              bool with_sinks = false) {
  Buf<float> sk(Hq);
  fill_sinks(sk);
  const float* sinks_ptr = with_sinks ? sk.p : nullptr;
  if (with_sinks) printf("with attention sinks: ");
  printf("attn_prefill B=%lld Hq=%lld Hkv=%lld D=%lld P=%lld ctx<=%d qo<=%d mode=%d window=%lld\n", (long long)B,
         (long long)Hq, (long long)Hkv, (long long)D, (long long)P, cmax, qmax, mode, (long long)window);
  std::vector<int32_t> qo(B + 1, 0), indptr(B + 1, 0), last(B), kvl(B);
  std::uniform_int_distribution<int> dc(0, cmax), dq(0, qmax);
  for (int64_t b = 0; b < B; ++b) {
    const int n = dq(rng);
    kvl[b] = dc(rng) + n;
    qo[b + 1] = qo[b] + n;
    const int np = (kvl[b] + P - 1) / P;
    indptr[b + 1] = indptr[b] + np;
    last[b] = np ? kvl[b] - (np - 1) * (int)P : 0;
  }
  const int64_t T = qo[B], pages = std::max<int64_t>(indptr[B], 1);
  Buf<int32_t> qi(B + 1), ip(B + 1), idx(pages), ll(B);
  std::vector<int32_t> perm(pages);
  for (int64_t i = 0; i < pages; ++i) perm[i] = (int32_t)i;
  std::shuffle(perm.begin(), perm.end(), rng);
  for (int64_t i = 0; i < pages; ++i) idx[i] = perm[i];
  for (int64_t b = 0; b <= B; ++b) { ip[b] = indptr[b]; qi[b] = qo[b]; }
  for (int64_t b = 0; b < B; ++b) ll[b] = last[b];
  const int64_t page_elems = 2 * P * Hkv * D;
  Buf<uint16_t> cache(pages * page_elems), q(std::max<int64_t>(T, 1) * Hq * D), out(std::max<int64_t>(T, 1) * Hq * D),
      want(std::max<int64_t>(T, 1) * Hq * D);
  fill_normal(cache);
  fill_normal(q);
  int64_t mbytes = 0;
  for (int64_t b = 0; b < B; ++b) mbytes += (int64_t)(qo[b + 1] - qo[b]) * kvl[b];
  Buf<uint8_t> mask(std::max<int64_t>(mbytes, 1));
  std::vector<int64_t> moff(B, 0);
  for (int64_t b = 1; b < B; ++b) moff[b] = moff[b - 1] + (int64_t)(qo[b] - qo[b - 1]) * kvl[b - 1];
  std::bernoulli_distribution bit(0.7);
  for (int64_t i = 0; i < mbytes; ++i) mask[i] = bit(rng) ? 1 : 0;
  if (causal_mask)  // random bits inside the causal window only: extents shorter than kv_len
    for (int64_t b = 0; b < B; ++b) {
      const int64_t qn = qo[b + 1] - qo[b];
      for (int64_t i = 0; i < qn; ++i)
        for (int64_t t = 0; t < kvl[b]; ++t)
          if (t > kvl[b] - qn + i) mask[moff[b] + i * kvl[b] + t] = 0;
    }
  const int64_t cap = 16 + 8 * (T * Hq / 32 + 2 * B + 2) + 4 * B + 8 + (T * Hq / 32 + 2 * B + 2) * Hkv + 4096;
  Buf<int32_t> plan(cap);
  int64_t words = 0, items = 0, mb = 0, mw = 0;
  rc_ok(pie_hip_attention_prefill_plan(qi.p, ip.p, ll.p, B, P, Hq, Hkv, D, mode, plan.p, cap, &words, &items, &mb,
                                       &mw),
        "prefill_plan");
  if (mode == 2 && mb != mbytes) { printf("  mask bytes %lld != %lld\n", (long long)mb, (long long)mbytes); ++failures; }
  Buf<uint32_t> packed(std::max<int64_t>(mw, 1));
  Buf<int32_t> extent(std::max<int64_t>(T, 1));
  if (mode == 2)
    rc_ok(pie_hip_attention_pack_mask(mask.p, plan.p, qi.p, ip.p, ll.p, B, P, mw, T, packed.p, extent.p, nullptr),
          "pack_mask");
  rc_ok(pie_hip_attention_prefill(q.p, Hq * D, D, cache.p, cache.p + P * Hkv * D, page_elems, Hkv * D, D, pages,
                                  qi.p, ip.p, idx.p, ll.p, Hq, Hkv, D, P, 1.f / sqrtf((float)D), mode, window,
                                  sinks_ptr,
                                  mode == 2 ? packed.p : nullptr, mode == 2 ? extent.p : nullptr, plan.p, items,
                                  plan[4], out.p, Hq * D, D,
                                  nullptr),
        "attention_prefill");
  oracle_attention(q.p, Hq * D, D, cache.p, cache.p + P * Hkv * D, page_elems, Hkv * D, D, qi.p, ip.p, idx.p,
                   ll.p, mode == 2 ? mask.p : nullptr, mode == 2 ? moff.data() : nullptr, mode == 1, window, B, Hq,
                   Hkv, D, P, 1.0 / sqrt((double)D), want.p, Hq * D,
                   D, nullptr, sinks_ptr);
  printf("  T=%lld items=%lld\n", (long long)T, (long long)items);
  check_close("prefill attention", out.p, want.p, T * Hq * D);
  float worst = 0.f;
  for (int64_t i = 0; i < T * Hq * D; ++i) {
    const float w = bf2f(want[i]);
    worst = fmaxf(worst, fabsf(bf2f(out[i]) - w) / (1.f / 256 + fabsf(w) / 128));
  }
  printf("  max |err| / (1/256 + |want|/128) = %.3f\n", worst);
  failures += !(worst <= 1.f);
}

// ---------------------------------------------------------------------------- sampling
// Probabilities are multiples of 2^-30 (exact in the kernel's 2^-40 fixed point and in float64),
// so kept sets and draws must match the oracle exactly; ties are forced in some rows.
// peaked: p = softmax of N(0, 3) logits (a few dominant tokens, as after an LM head) with k up to
// 64, so the candidate lists are short; otherwise near-uniform rows whose lists can overflow.
static void case_sample(int64_t B, int64_t V, int mode, bool row_map, bool peaked = false, int64_t pad = 0,
                        int64_t zero_head = 0) {
  printf("sample B=%lld V=%lld mode=%d rows=%d peaked=%d pad=%lld zero_head=%lld\n", (long long)B, (long long)V,
         mode, (int)row_map, (int)peaked, (long long)pad, (long long)zero_head);
  Buf<float> probs(B * V);
  std::uniform_int_distribution<int> dq(0, 1 << 12);
  std::normal_distribution<double> dn(0.0, 3.0);
  for (int64_t r = 0; r < B; ++r) {
    double tot = 0;
    for (int64_t i = 0; i < V; ++i) {
      // zero_head > 0: the first zero_head entries are 0; < 0: the first -zero_head are tiny
      probs[r * V + i] = i < zero_head ? 0.f : i < -zero_head ? 50.f
                         : peaked ? (float)(exp(dn(rng)) * 1024.0) : (float)dq(rng);
      tot += probs[r * V + i];
    }
    if (r % 3 == 1) for (int64_t i = 0; i < V; i += 7) probs[r * V + i] = probs[r * V];  // ties
    if (r % 4 == 2) probs[r * V + 3] = 0.f;
    for (int64_t i = 0; i < V; ++i) probs[r * V + i] = (float)(ldexp(floor(probs[r * V + i] / tot * 1073741824.0), -30));
  }
  Buf<int32_t> rows(B), topk(B), out(B), want(B);
  Buf<float> topp(B), minp(B);
  Buf<double> u(B);
  std::uniform_real_distribution<double> du(0.0, 1.0);
  std::uniform_int_distribution<int> dk(1, peaked ? 64 : (int)V + 2);
  for (int64_t r = 0; r < B; ++r) {
    rows[r] = row_map ? (int32_t)((r * 5 + 1) % B) : (int32_t)r;
    topk[r] = r == 0 ? 0 : dk(rng);
    topp[r] = (float)du(rng);
    minp[r] = (float)du(rng) * 0.5f;
    u[r] = du(rng);
  }
  const int64_t S = V + pad;  // row stride of the copy the kernel reads (exact-size buffer)
  Buf<float> padded(B * S - pad);
  for (int64_t r = 0; r < B; ++r) memcpy(padded.p + r * S, probs.p + r * V, V * 4);
  rc_ok(pie_hip_sample(padded.p, S, B, V, B, row_map ? rows.p : nullptr, mode, topk.p, 0, topp.p, 0.f, minp.p, 0.f,
                       u.p, 0, 0, out.p, nullptr), "sample");
  Buf<float> mapped(B * V);
  for (int64_t r = 0; r < B; ++r) memcpy(mapped.p + r * V, probs.p + (int64_t)rows[r] * V, V * 4);
  oracle_sample(mapped.p, B, V, V, mode, topk.p, topp.p, minp.p, u.p, want.p, nullptr);
  check_equal("sample", out.p, want.p, B);
}

// masked: rows carry -inf logits (padding / banned tokens): row 1 its first 3/4, row 2 every
// other 16-byte vector, row 3 everything but one token (B >= 4); the rest random.
static void case_softmax(int64_t B, int64_t V, bool bf16, bool masked = false) {
  printf("scaled_softmax B=%lld V=%lld bf16=%d masked=%d\n", (long long)B, (long long)V, (int)bf16, (int)masked);
  Buf<float> x(B * V), temps(B), out(B * V);
  Buf<uint16_t> xb(B * V), ob(B * V);
  std::normal_distribution<float> d(0.f, 3.f);
  for (int64_t i = 0; i < B * V; ++i) {
    const int64_t r = i / V, c = i % V;
    const bool m = masked && ((r == 1 && c < 3 * V / 4) || (r == 2 && (c / (bf16 ? 8 : 4)) % 2 == 0) ||
                              (r == 3 && c != V / 3));
    xb[i] = m ? (uint16_t)0xff80 : f2bf(d(rng));
    x[i] = bf2f(xb[i]);
  }
  for (int64_t r = 0; r < B; ++r) temps[r] = r == 0 ? 0.f : 0.3f + 0.4f * (float)r;
  if (bf16) rc_ok(pie_hip_scaled_softmax(xb.p, 1, V, B, V, temps.p, 1e-5f, ob.p, V, nullptr), "softmax");
  else rc_ok(pie_hip_scaled_softmax(x.p, 0, V, B, V, temps.p, 1e-5f, out.p, V, nullptr), "softmax");
  std::vector<double> want(B * V);
  oracle_scaled_softmax(x.p, B, V, temps.p, 1e-5, want.data());
  size_t bad = 0;
  for (int64_t i = 0; i < B * V; ++i) {
    const double g = bf16 ? bf2f(ob[i]) : out[i];
    if (!(fabs(g - want[i]) <= 1e-2 * fabs(want[i]) + 1e-7)) ++bad;
  }
  printf("  %-40s %s (%zu / %lld outside 1e-2 rel + 1e-7 abs)\n", "scaled_softmax", bad ? "FAIL" : "ok", bad,
         (long long)(B * V));
  failures += bad != 0;
}

static void case_index(int64_t B) {
  printf("index helpers B=%lld\n", (long long)B);
  Paged pg = make_paged(B, 16, 0, 100, 0, 9);
  Buf<int32_t> kvp(B + 1), last(B), qo(B + 1), sl(B), wsl(B), bi(pg.T), po(pg.T), wbi(pg.T), wpo(pg.T);
  copy_in(kvp, pg.kv_indptr);
  copy_in(last, pg.last);
  copy_in(qo, pg.qo);
  rc_ok(pie_hip_get_seq_lens(kvp.p, last.p, B, 16, sl.p, nullptr), "seq_lens");
  oracle_seq_lens(kvp.p, last.p, B, 16, wsl.p);
  check_equal("seq_lens", sl.p, wsl.p, B);
  rc_ok(pie_hip_get_batch_indices_positions(qo.p, sl.p, B, pg.T, bi.p, po.p, nullptr), "bip");
  oracle_batch_indices_positions(qo.p, wsl.p, B, pg.T, wbi.p, wpo.p);
  check_equal("batch_indices", bi.p, wbi.p, pg.T);
  check_equal("positions", po.p, wpo.p, pg.T);
}

static void case_fastdiv() {
  printf("fastdiv\n");
  size_t bad = 0, n = 0;
  std::uniform_int_distribution<uint32_t> du(0, 0xffffffffu);
  const uint32_t ds[] = {1, 2, 3, 5, 7, 64, 96, 100, 512, 1536, 1792, 3000, 65535, 65536, 1000003,
                         0x7fffffffu, 0x80000000u, 0xfffffffbu};
  for (uint32_t d : ds) {
    const pie::FastDiv f = pie::FastDiv::make(d);
    for (int i = 0; i < 20000; ++i, ++n) {
      const uint32_t x = i < 4 ? (uint32_t[]){0u, d - 1, d, 0xffffffffu}[i] : du(rng);
      bad += f.div(x) != x / d;
    }
  }
  printf("  %-40s %s (%zu / %zu wrong)\n", "FastDiv vs /", bad ? "FAIL" : "ok", bad, n);
  failures += bad != 0;
}

int main(int argc, char** argv) {
  std::string c = argc > 1 ? argv[1] : "all";
  const bool all = c == "all";
  if (all || c == "fastdiv") case_fastdiv();
  if (all || c == "norm") {
    case_norm(3, 512);
    case_norm(5, 4096);
    case_norm(2, 896);
    case_norm(3, 100);
    case_norm(4, 128);
    case_norm(3, 5120);   // W = 2 waves per row
    case_norm(2, 2048);   // W = 4
    case_norm(40, 1024);  // W = 2, several row groups per block
  }
  if (all || c == "qk") {
    case_qk(5, 4, 2, 128);
    case_qk(3, 2, 1, 64);
    case_qk(2, 2, 1, 96);
  }
  if (all || c == "silu") {
    case_silu(3, 1536);
    case_silu(2, 13);
    case_silu(8, 2048);   // 2 vectors per thread
    case_silu(9, 4096);   // 4 vectors per thread
  }
  if (all || c == "embed") {
    case_embed(50, 4096, 9);
    case_embed(20, 100, 5);
    case_embed(64, 4096, 40);  // 4 vectors per thread
  }
  if (all || c == "rope") case_rope_append(3, 4, 2, 128, 0, 40, 1, 20, false);
  if (all || c == "fused") {
    case_rope_append(3, 4, 2, 128, 0, 40, 1, 20, true);
    case_rope_append(3, 4, 2, 128, 0, 40, 1, 20, true, 64, 0);   // partial rotary: k tail copied
    case_rope_append(3, 4, 2, 128, 0, 40, 1, 20, true, 128, 1);  // interleaved pairs
    case_rope_append(3, 3, 1, 32, 0, 40, 1, 20, true, 24, 0);    // scalar fallback kernels
    case_rope_append(2, 3, 1, 32, 0, 40, 1, 20, false, 24, 1);
  }
  if (c == "big") case_rope_append(4, 2, 1, 64, 0, 100, 600, 700, true);  // T >= 2048: 2 tokens/block
  if (all || c == "decode") {
    // Qwen3-8B decode shape (the faulting chain's rope/append and norms), fewer sequences
    case_rope_append(6, 32, 8, 128, 128, 4096, 1, 1, true);
    case_rope_append(6, 32, 8, 128, 128, 4096, 1, 1, false);
    case_qk(6, 32, 8, 128);
    case_norm(6, 4096);
  }
  if (all || c == "index") case_index(40);
  if (all || c == "attn") {
    case_attn_decode(3, 8, 2, 128, 16, 1, 90, 1);     // one work group per request
    case_attn_decode(3, 8, 2, 128, 16, 100, 400, 3);  // 3 splits + merge (some empty)
    case_attn_decode(2, 4, 4, 64, 4, 0, 50, 2);       // G = 1, page 4, an empty request possible
    case_attn_decode(2, 6, 1, 256, 8, 30, 300, 0);    // G = 6, D = 256, library's split count
    case_attn_decode(2, 16, 1, 128, 5, 20, 700, 5);   // G = 16, page size 5
    case_attn_decode(2, 4, 2, 64, 1, 600, 1500, 1);   // page size 1: several page-table windows
    case_attn_decode(3, 8, 2, 128, 16, 1, 700, 3, 100);  // sliding window of 100 (+ the query)
    case_attn_decode(3, 8, 2, 128, 16, 1, 300, 1, -1, true);   // attention sinks, one split
    case_attn_decode(3, 8, 2, 64, 16, 0, 500, 3, 60, true);    // sinks + merge + window
  }
  if (all || c == "sample") {
    for (int mode = 0; mode <= 4; ++mode) case_sample(mode == 4 ? 5 : 3, 301, mode, mode == 4);
    case_sample(2, 4099, 4, false);  // several 4096-element scan tiles
    for (int mode = 1; mode <= 4; ++mode) case_sample(1, 10000, mode, false, true);  // candidate lists
    case_sample(1, 10003, 4, false, true);  // candidate lists, scalar loads
    case_sample(2, 10003, 4, false, true, 1);  // 16-byte rows whose length is not a multiple of 4
    case_sample(2, 10001, 3, false, true, 3);
    case_sample(1, 40000, 1, false);        // top_p over a flat row: the threshold's histogram bin
    case_sample(3, 70000, 1, false);        // top_p, flat rows: the bin's keys (and the ties of row 1)
    case_sample(2, 70000, 1, false, true);  // top_p, peaked rows: every key from the bin up
    case_sample(2, 70000, 1, false, false, 0, -69990);  // a bin of 69990 equal keys: search over the row
    // top_k and min_p over long rows: one read with a floor from a sample of the row (the start
    // of every wave segment; a row of ties overflows the list and falls back, zeros at the row's
    // start leave wave 0 without sampled positives, tiny entries there lower the floor)
    case_sample(4, 70000, 2, false, true);
    case_sample(4, 70000, 4, false, true);
    case_sample(3, 70000, 4, false, true, 0, 8192);
    case_sample(3, 70000, 2, false, true, 0, 8190);
    case_sample(3, 70000, 4, false, true, 0, -8192);
    case_sample(4, 70000, 3, false, true);
    case_sample(3, 70000, 3, false);                  // flat rows: most entries kept, the lists overflow
    case_sample(3, 70000, 3, false, true, 0, -8192);
    // (rows of more than 256 tiles, whose draw chunks span several tiles, run in the GPU tests)
    case_softmax(3, 1000, false);
    case_softmax(3, 777, true);
    case_softmax(2, 70003, false);   // rows not 16-byte aligned: the streaming kernel
    case_softmax(4, 1000, false, true);   // -inf logits, register-resident kernel
    case_softmax(4, 4096, true, true);
    case_softmax(4, 70003, false, true);  // -inf logits, streaming kernel
  }
  if (all || c == "prefill") {
    case_attn_prefill(3, 8, 2, 128, 16, 40, 45, 1);   // causal, chunked prefill over cached context
    case_attn_prefill(2, 4, 4, 64, 4, 20, 40, 0);     // full (non-causal), G = 1
    case_attn_prefill(3, 6, 2, 128, 8, 30, 30, 2);    // custom mask, G = 3
    case_attn_prefill(2, 2, 1, 256, 16, 10, 20, 1);   // D = 256
    case_attn_prefill(2, 4, 1, 64, 1, 600, 10, 1);    // page size 1: several page-table windows
    case_attn_prefill(2, 8, 2, 128, 5, 60, 50, 1);    // D = 128, page size 5: a tile's rows on several pages
    case_attn_prefill(2, 4, 2, 128, 1, 600, 30, 2);   // D = 128, page size 1, custom mask, windows
    case_attn_prefill(2, 8, 2, 128, 4, 70, 40, 0);    // D = 128, page size 4, full (non-causal)
    case_attn_prefill(2, 8, 2, 128, 16, 50, 100, 1);  // up to 400 rows: several items per request
    case_attn_prefill(2, 8, 2, 128, 16, 50, 100, 2);
    case_attn_prefill(3, 8, 2, 128, 16, 20, 120, 2, true);  // masks within the causal window
    case_attn_prefill(3, 8, 2, 128, 16, 200, 120, 1, false, 70);  // causal + sliding window
    case_attn_prefill(2, 8, 2, 128, 8, 100, 90, 2, false, 40);    // custom mask + sliding window
    case_attn_prefill(3, 8, 2, 128, 16, 60, 70, 1, false, -1, true);  // causal + sinks (32-row kernel)
    case_attn_prefill(2, 4, 2, 64, 16, 30, 40, 1, false, 20, true);   // D = 64 + window + sinks
  }
  if (all || c == "group") {
    case_group(5, 4096, 1536, 40, false);  // 8 norm vectors per lane pair (NJ = 2)
    case_group(3, 1024, 256, 9, true);      // GELU, 2 waves per row
    case_group(2, 896, 512, 7, false);      // norm width outside the group kernel: separate launches
    case_attn_decode_noalloc();
  }
  if (all || c == "qkfused") {
    case_qk_fused(5, 4, 2, 128);  // fused kernel
    case_qk_fused(3, 4, 2, 64);   // D != 128: separate-kernel path
    case_qk_fused(3, 32, 8, 128);
  }
  if (all || c == "variants") {
    case_variants(5, 2304, 4, 2, 128, 1536);   // vector paths
    case_variants(3, 100, 2, 1, 64, 13);       // scalar / generic fallbacks
    case_variants(4, 3584, 8, 4, 256, 2048);   // Gemma-2 9B widths, D = 256
  }
  printf("%s\n", failures ? "FAILURES" : "all ok");
  return failures ? 1 : 0;
}
