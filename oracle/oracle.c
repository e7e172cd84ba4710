/*
 * CPU oracle for the per-layer hot path of Pie's Python backend. TEST INFRASTRUCTURE ONLY:
 * it is the checker that the GPU kernels are compared with, never a compute path of the
 * product. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Arithmetic is float64 (the "exact" value) with bf16 round-to-nearest-even on output, except
 * where the reference itself rounds an intermediate to bf16 (the residual sum, silu before
 * the multiply), which is reproduced bit for bit. bf16 values are passed as uint16_t bits.
 *
 * Reference behaviour restated (paths relative to the zyma98/pie repository root):
 *   rmsnorm            torch rms_norm decomposition, torch/_decomp/decompositions.py:1760-1810,
 *                      called at pie/src/pie_worker/model/llama3.py:555-560, qwen3.py:651-662
 *   add_rmsnorm        `residual + down` (llama3.py:586) then the next rms_norm (llama3.py:555)
 *   silu_and_mul       `fun.silu(gate) * up` after torch.split (llama3.py:569-572)
 *   embedding          fun.embedding(ids, W) (llama3.py:471)
 *   gemma_rmsnorm      pie/src/pie_worker/model/gemma2.py:514-526, gemma3.py:491-510
 *   gelu_tanh_and_mul  gemma2.py:224-226, :608
 *   embedding_scaled   gemma3.py:476-489
 *   rope_cs            flashinfer.apply_rope_with_cos_sin_cache_inplace (gpt_oss.py:671-678)
 *   rope               pie/src/flashinfer_metal/kernels/metal_rope.metal:26-107
 *   inv_freq_llama31   metal_rope.metal:63-89
 *   append             pie/src/flashinfer_metal/kernels/metal_append_paged_kv_cache.metal:23-107
 *   seq_lens           pie/src/flashinfer_metal/ops.py:392-407
 *   batch_indices_positions  pie/src/flashinfer_metal/ops.py:410-436
 *   attention          flashinfer Batch{Prefill,Decode}WithPagedKVCacheWrapper.run as restated
 *                      in pie/src/flashinfer_metal/ops.py:163-282 and
 *                      kernels/metal_attention_simdgroup_opt.metal:120-470 (causal window),
 *                      custom masks as built at pie/src/pie_worker/batching.py:335-386
 *   scaled_softmax     safe_scaled_softmax, pie/src/pie_worker/model/common.py:38-59 (torch
 *                      form) and :68-188 (the Triton kernel Pie runs on GPUs)
 *   sample             flashinfer.sampling.{sampling,top_p,top_k,min_p,top_k_top_p}_sampling_from_probs
 *                      as called at common.py:316-344; restated (with a simplified top-k and a
 *                      boundary-excluding top-p) in pie/src/flashinfer_metal/sampling.py:19-79
 */
#include <math.h>
#include <stdlib.h>
#include <stdint.h>
#include <string.h>

/* ------------------------------------------------------------------ bf16 */
static float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* fp32 -> bf16, round to nearest even; NaN stays NaN (quiet). */
static uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* float64 -> bf16 in one rounding (no intermediate fp32 rounding). */
static uint16_t d2bf(double d) {
  if (isnan(d)) return 0x7fc0;
  float f = (float)d; /* RNE to 24 bits; fix the rare double-rounding tie below */
  uint16_t h = f2bf(f);
  /* If f landed exactly on a bf16 halfway point, decide the tie from the exact value. */
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0xffffu) == 0x8000u && isfinite(f)) {
    double lo = bf2f((uint16_t)(u >> 16));
    double hi = bf2f((uint16_t)((u >> 16) + 1));
    if (fabs(d - lo) < fabs(hi - d)) h = (uint16_t)(u >> 16);
    else if (fabs(d - lo) > fabs(hi - d)) h = (uint16_t)((u >> 16) + 1);
  }
  return h;
}

uint16_t oracle_f32_to_bf16(float f) { return f2bf(f); }
float oracle_bf16_to_f32(uint16_t h) { return bf2f(h); }
uint16_t oracle_f64_to_bf16(double d) { return d2bf(d); }

/* ------------------------------------------------------------------ RMSNorm */
static void norm_row(const uint16_t* x, const uint16_t* w, uint16_t* y, int64_t cols, double eps) {
  double ss = 0.0;
  for (int64_t j = 0; j < cols; ++j) {
    double v = bf2f(x[j]);
    ss += v * v;
  }
  double rstd = 1.0 / sqrt(ss / (double)cols + eps);
  for (int64_t j = 0; j < cols; ++j) y[j] = d2bf((double)bf2f(x[j]) * rstd * (double)bf2f(w[j]));
}

/* Rows addressed as (token, head): row r = t*heads + h at offset t*ts + h*hs. */
void oracle_rmsnorm(const uint16_t* x, int64_t x_ts, int64_t x_hs, const uint16_t* w, uint16_t* y,
                    int64_t y_ts, int64_t y_hs, int64_t T, int64_t heads, int64_t cols, double eps) {
  for (int64_t t = 0; t < T; ++t)
    for (int64_t h = 0; h < heads; ++h)
      norm_row(x + t * x_ts + h * x_hs, w, y + t * y_ts + h * y_hs, cols, eps);
}

void oracle_add_rmsnorm(const uint16_t* x, const uint16_t* r, const uint16_t* w, uint16_t* s,
                        uint16_t* y, int64_t rows, int64_t cols, double eps) {
  for (int64_t i = 0; i < rows; ++i) {
    for (int64_t j = 0; j < cols; ++j) {
      /* torch bf16 add: fp32 sum of the two widened values, one RNE rounding */
      float sum = bf2f(r[i * cols + j]) + bf2f(x[i * cols + j]);
      s[i * cols + j] = f2bf(sum);
    }
    norm_row(s + i * cols, w, y + i * cols, cols, eps);
  }
}

/* Gemma RMSNorm, pie/src/pie_worker/model/gemma2.py:514-526 / gemma3.py:491-510:
 *   variance = x.pow(2).mean(-1); x * rsqrt(variance + eps) * (1.0 + weight)
 * as separate bf16 torch ops: each step's result is rounded to bf16 (the mean's sum itself is
 * exact here, torch accumulates it in fp32). */
static void gemma_row(const uint16_t* x, const uint16_t* w, uint16_t* y, int64_t cols, double eps) {
  double ss = 0.0;
  for (int64_t j = 0; j < cols; ++j) {
    float v = bf2f(x[j]);
    ss += bf2f(f2bf(v * v));
  }
  float var = bf2f(d2bf(ss / (double)cols));
  float t = bf2f(f2bf(var + (float)eps));
  float r = bf2f(d2bf(1.0 / sqrt((double)t)));
  for (int64_t j = 0; j < cols; ++j) {
    float xn = bf2f(d2bf((double)bf2f(x[j]) * r));
    float w1 = bf2f(f2bf(1.0f + bf2f(w[j])));
    y[j] = d2bf((double)xn * w1);
  }
}

void oracle_gemma_rmsnorm(const uint16_t* x, int64_t x_ts, int64_t x_hs, const uint16_t* w,
                          uint16_t* y, int64_t y_ts, int64_t y_hs, int64_t T, int64_t heads,
                          int64_t cols, double eps) {
  for (int64_t t = 0; t < T; ++t)
    for (int64_t h = 0; h < heads; ++h)
      gemma_row(x + t * x_ts + h * x_hs, w, y + t * y_ts + h * y_hs, cols, eps);
}

void oracle_gemma_add_rmsnorm(const uint16_t* x, const uint16_t* r, const uint16_t* w, uint16_t* s,
                              uint16_t* y, int64_t rows, int64_t cols, double eps) {
  for (int64_t i = 0; i < rows; ++i) {
    for (int64_t j = 0; j < cols; ++j) s[i * cols + j] = f2bf(bf2f(r[i * cols + j]) + bf2f(x[i * cols + j]));
    gemma_row(s + i * cols, w, y + i * cols, cols, eps);
  }
}

/* ------------------------------------------------------------------ SiLU-and-mul */
/* mode 0: torch's rounding, bf16(bf16(silu(g)) * up); mode 1: single rounding of silu(g)*up. */
void oracle_silu_and_mul(const uint16_t* gu, int64_t in_rs, uint16_t* out, int64_t rows,
                         int64_t I, int mode) {
  for (int64_t i = 0; i < rows; ++i)
    for (int64_t j = 0; j < I; ++j) {
      double g = bf2f(gu[i * in_rs + j]);
      double u = bf2f(gu[i * in_rs + I + j]);
      double s = g / (1.0 + exp(-g));
      if (mode == 0) out[i * I + j] = d2bf((double)bf2f(d2bf(s)) * u);
      else out[i * I + j] = d2bf(s * u);
    }
}

/* GELU(tanh)-and-mul, `_gelu_pytorch_tanh(gate) * up` (gemma2.py:224-226, :608):
 * torch gelu(approximate="tanh") rounded to bf16, times up, rounded again. */
void oracle_gelu_tanh_and_mul(const uint16_t* gu, int64_t in_rs, uint16_t* out, int64_t rows,
                              int64_t I) {
  const double k0 = sqrt(2.0 / M_PI);
  for (int64_t i = 0; i < rows; ++i)
    for (int64_t j = 0; j < I; ++j) {
      double g = bf2f(gu[i * in_rs + j]);
      double u = bf2f(gu[i * in_rs + I + j]);
      double gl = 0.5 * g * (1.0 + tanh(k0 * (g + 0.044715 * g * g * g)));
      out[i * I + j] = d2bf((double)bf2f(d2bf(gl)) * u);
    }
}

/* ------------------------------------------------------------------ embedding */
/* Returns the number of ids outside [0, V); their rows are zero-filled. */
int64_t oracle_embedding(const int32_t* ids, int64_t T, const uint16_t* W, int64_t V, int64_t H,
                         uint16_t* out) {
  int64_t bad = 0;
  for (int64_t t = 0; t < T; ++t) {
    if (ids[t] < 0 || ids[t] >= V) {
      memset(out + t * H, 0, (size_t)H * 2);
      ++bad;
    } else {
      memcpy(out + t * H, W + (int64_t)ids[t] * H, (size_t)H * 2);
    }
  }
  return bad;
}

/* `fun.embedding(ids, W) * self.embed_normalizer` (gemma3.py:476-489): torch multiplies the bf16
 * rows by the scalar in fp32 and rounds once. Out-of-range ids give zero rows. */
int64_t oracle_embedding_scaled(const int32_t* ids, int64_t T, const uint16_t* W, int64_t V,
                                int64_t H, float scale, uint16_t* out) {
  int64_t bad = 0;
  for (int64_t t = 0; t < T; ++t) {
    if (ids[t] < 0 || ids[t] >= V) {
      memset(out + t * H, 0, (size_t)H * 2);
      ++bad;
      continue;
    }
    for (int64_t j = 0; j < H; ++j) out[t * H + j] = f2bf(bf2f(W[(int64_t)ids[t] * H + j]) * scale);
  }
  return bad;
}

/* ------------------------------------------------------------------ RoPE */
void oracle_inv_freq_std(double* f, int64_t rd, double scale, double theta) {
  for (int64_t i = 0; i < rd / 2; ++i) f[i] = 1.0 / (scale * pow(theta, (2.0 * i) / (double)rd));
}

void oracle_inv_freq_llama31(double* f, int64_t rd, double scale, double theta, double lo,
                             double hi, double L) {
  for (int64_t i = 0; i < rd / 2; ++i) {
    double base = 1.0 / pow(theta, (2.0 * i) / (double)rd);
    double wavelen = 2.0 * M_PI / base;
    if (wavelen > L / lo) f[i] = base / scale;
    else if (wavelen < L / hi) f[i] = base;
    else {
      double smooth = (L / wavelen - lo) / (hi - lo);
      f[i] = (1.0 - smooth) * base / scale + smooth * base;
    }
  }
}

static void rope_head(uint16_t* v, int64_t rd, int interleave, double p, const double* f) {
  for (int64_t i = 0; i < rd / 2; ++i) {
    int64_t ix = interleave ? 2 * i : i, iy = interleave ? 2 * i + 1 : i + rd / 2;
    double a = p * f[i], c = cos(a), s = sin(a);
    double x = bf2f(v[ix]), y = bf2f(v[iy]);
    v[ix] = d2bf(x * c - y * s);
    v[iy] = d2bf(x * s + y * c);
  }
}

/* In place on q [T,Hq,D] and k [T,Hkv,D] (strided: token stride, head stride; unit inner). */
void oracle_rope(uint16_t* q, int64_t q_ts, int64_t q_hs, uint16_t* k, int64_t k_ts, int64_t k_hs,
                 const int32_t* pos, int64_t T, int64_t Hq, int64_t Hkv, int64_t rd,
                 int interleave, const double* inv_freq) {
  for (int64_t t = 0; t < T; ++t) {
    double p = (double)pos[t];
    for (int64_t h = 0; h < Hq; ++h) rope_head(q + t * q_ts + h * q_hs, rd, interleave, p, inv_freq);
    for (int64_t h = 0; h < Hkv; ++h) rope_head(k + t * k_ts + h * k_hs, rd, interleave, p, inv_freq);
  }
}

/* RoPE from a cos/sin table (flashinfer.apply_rope_with_cos_sin_cache_inplace, gpt_oss.py:671):
 * row pos of `cs` (stride ld) holds cos at [0, rd/2) and sin at [rd/2, rd); positions outside
 * [0, rows) leave the token unchanged. */
static void rope_head_cs(uint16_t* v, int64_t rd, int interleave, const float* row) {
  for (int64_t i = 0; i < rd / 2; ++i) {
    int64_t ix = interleave ? 2 * i : i, iy = interleave ? 2 * i + 1 : i + rd / 2;
    double c = row[i], s = row[rd / 2 + i];
    double x = bf2f(v[ix]), y = bf2f(v[iy]);
    v[ix] = d2bf(x * c - y * s);
    v[iy] = d2bf(x * s + y * c);
  }
}

void oracle_rope_cs(uint16_t* q, int64_t q_ts, int64_t q_hs, uint16_t* k, int64_t k_ts, int64_t k_hs,
                    const int32_t* pos, int64_t T, int64_t Hq, int64_t Hkv, int64_t rd,
                    int interleave, const float* cs, int64_t rows, int64_t ld) {
  for (int64_t t = 0; t < T; ++t) {
    if (pos[t] < 0 || pos[t] >= rows) continue;
    const float* row = cs + (int64_t)pos[t] * ld;
    for (int64_t h = 0; h < Hq; ++h) rope_head_cs(q + t * q_ts + h * q_hs, rd, interleave, row);
    for (int64_t h = 0; h < Hkv; ++h) rope_head_cs(k + t * k_ts + h * k_hs, rd, interleave, row);
  }
}

/* ------------------------------------------------------------------ paged append */
/* Returns the number of tokens written (skipped tokens follow the Metal kernel's checks). */
int64_t oracle_append(const uint16_t* k, int64_t k_ts, int64_t k_hs, const uint16_t* v, int64_t v_ts,
                      int64_t v_hs, const int32_t* bidx, const int32_t* pos,
                      const int32_t* kv_indices, const int32_t* kv_indptr, int64_t B,
                      uint16_t* kc, uint16_t* vc, int64_t num_pages, int64_t page_stride,
                      int64_t slot_stride, int64_t head_stride, int64_t P, int64_t T, int64_t Hkv,
                      int64_t D) {
  int64_t written = 0;
  for (int64_t t = 0; t < T; ++t) {
    int64_t b = bidx[t], p = pos[t];
    if (b < 0 || b >= B || p < 0) continue;
    int64_t logical = (int64_t)kv_indptr[b] + p / P;
    if (logical >= kv_indptr[b + 1]) continue;
    int64_t page = kv_indices[logical];
    if (page < 0 || page >= num_pages) continue;
    int64_t base = page * page_stride + (p % P) * slot_stride;
    for (int64_t h = 0; h < Hkv; ++h) {
      memcpy(kc + base + h * head_stride, k + t * k_ts + h * k_hs, (size_t)D * 2);
      memcpy(vc + base + h * head_stride, v + t * v_ts + h * v_hs, (size_t)D * 2);
    }
    ++written;
  }
  return written;
}

/* ------------------------------------------------------------------ index helpers */
void oracle_seq_lens(const int32_t* indptr, const int32_t* last, int64_t B, int64_t P, int32_t* out) {
  for (int64_t b = 0; b < B; ++b) {
    int32_t np = indptr[b + 1] - indptr[b];
    out[b] = np > 0 ? (int32_t)((np - 1) * P + last[b]) : 0;
  }
}

void oracle_batch_indices_positions(const int32_t* indptr, const int32_t* seq_lens, int64_t B,
                                    int64_t nnz, int32_t* bidx, int32_t* pos) {
  for (int64_t b = 0; b < B; ++b) {
    int32_t start = indptr[b], end = indptr[b + 1], n = end - start;
    for (int32_t t = start; t < end && t < nnz; ++t) {
      if (t < 0) continue;
      bidx[t] = (int32_t)b;
      pos[t] = seq_lens[b] - n + (t - start);
    }
  }
}

/* ------------------------------------------------------------------ paged attention
 * For request b: kv_len = (npages-1)*P + last_len[b] (0 with no pages), qo_len =
 * qo_indptr[b+1]-qo_indptr[b]. Query token i of the request attends kv position t iff
 *   custom mask:  mask[mask_off[b] + i*kv_len + t] != 0   (row-major [qo_len, kv_len] per request,
 *                 the layout decode_brle_batch writes, batching.py:335-386)
 *   causal:       t <= kv_len - qo_len + i                  (metal_attention...:176, 243)
 *   neither:      every t < kv_len (flashinfer's prefill default, causal=False)
 * and, with window_left >= 0 (flashinfer's sliding window), also t >= kv_len - qo_len + i - window_left.
 * Head h reads kv head h / (Hq/Hkv). Scores are q.k * sm_scale in float64, softmax in float64,
 * output rounded once to bf16. A row with no allowed position gives 0 and lse = -inf.
 * Token t of request b lives in page kv_indices[kv_indptr[b] + t/P], slot t%P; k and v are
 * addressed as k_cache/v_cache + page*page_stride + slot*slot_stride + head*head_stride.
 * lse (optional, [T, Hq]) is the natural-log sum of exp(scaled scores).
 * sinks (optional, fp32 [Hq]): gpt-oss attention sinks (pie/src/pie_worker/model/gpt_oss.py:693-697,
 * flashinfer's BatchAttentionWithAttentionSinkWrapper; the published gpt-oss attention appends
 * the head's sink logit as one more score column, takes the softmax and drops that column):
 * the denominator gains exp(sinks[h]), the numerator nothing; lse includes it.            */
void oracle_attention(const uint16_t* q, int64_t q_ts, int64_t q_hs, const uint16_t* kc,
                      const uint16_t* vc, int64_t page_stride, int64_t slot_stride,
                      int64_t head_stride, const int32_t* qo_indptr, const int32_t* kv_indptr,
                      const int32_t* kv_indices, const int32_t* last_len, const uint8_t* mask,
                      const int64_t* mask_off, int causal, int64_t window_left, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                      int64_t P, double sm_scale, uint16_t* out, int64_t o_ts, int64_t o_hs,
                      double* lse, const float* sinks) {
  const int64_t G = Hq / Hkv;
  for (int64_t b = 0; b < B; ++b) {
    const int64_t np = kv_indptr[b + 1] - kv_indptr[b];
    const int64_t kv_len = np > 0 ? (np - 1) * P + last_len[b] : 0;
    const int64_t q0 = qo_indptr[b], qo_len = qo_indptr[b + 1] - q0;
    double* s = (double*)malloc(sizeof(double) * (size_t)(kv_len > 0 ? kv_len : 1));
    double* acc = (double*)malloc(sizeof(double) * (size_t)D);
    for (int64_t i = 0; i < qo_len; ++i) {
      for (int64_t h = 0; h < Hq; ++h) {
        const uint16_t* qv = q + (q0 + i) * q_ts + h * q_hs;
        const int64_t kh = h / G;
        double mx = -INFINITY;
        for (int64_t t = 0; t < kv_len; ++t) {
          int ok = mask ? mask[mask_off[b] + i * kv_len + t] != 0 : (!causal || t <= kv_len - qo_len + i);
          if (window_left >= 0 && t < kv_len - qo_len + i - window_left) ok = 0;
          if (!ok) { s[t] = -INFINITY; continue; }
          const int64_t page = kv_indices[kv_indptr[b] + t / P];
          const uint16_t* kv = kc + page * page_stride + (t % P) * slot_stride + kh * head_stride;
          double d = 0;
          for (int64_t e = 0; e < D; ++e) d += (double)bf2f(qv[e]) * (double)bf2f(kv[e]);
          s[t] = d * sm_scale;
          if (s[t] > mx) mx = s[t];
        }
        for (int64_t e = 0; e < D; ++e) acc[e] = 0;
        double den = 0;
        const double sk = sinks ? (double)sinks[h] : -INFINITY;
        if (sk > mx) mx = sk;
        if (mx > -INFINITY) {
          if (sinks) den = exp(sk - mx);
          for (int64_t t = 0; t < kv_len; ++t) {
            if (s[t] == -INFINITY) continue;
            const double p = exp(s[t] - mx);
            den += p;
            const int64_t page = kv_indices[kv_indptr[b] + t / P];
            const uint16_t* vv = vc + page * page_stride + (t % P) * slot_stride + kh * head_stride;
            for (int64_t e = 0; e < D; ++e) acc[e] += p * (double)bf2f(vv[e]);
          }
        }
        uint16_t* o = out + (q0 + i) * o_ts + h * o_hs;
        for (int64_t e = 0; e < D; ++e) o[e] = den > 0 ? d2bf(acc[e] / den) : 0;
        if (lse) lse[(q0 + i) * Hq + h] = den > 0 ? mx + log(den) : -INFINITY;
      }
    }
    free(s);
    free(acc);
  }
}

/* ------------------------------------------------------------------ sampling path
 * scaled_softmax: row r of logits (fp32 values given as float) -> probs, float64 math.
 * temperature < greedy_threshold: one-hot at the first maximum; otherwise softmax(x / T).     */
void oracle_scaled_softmax(const float* x, int64_t B, int64_t V, const float* temps, double greedy,
                           double* out) {
  for (int64_t r = 0; r < B; ++r) {
    const float* xr = x + r * V;
    double* o = out + r * V;
    int64_t am = 0;
    for (int64_t i = 1; i < V; ++i)
      if (xr[i] > xr[am]) am = i;
    if ((double)temps[r] < greedy) {
      for (int64_t i = 0; i < V; ++i) o[i] = i == am ? 1.0 : 0.0;
      continue;
    }
    const double T = temps[r];
    const double m = (double)xr[am] / T;
    double s = 0;
    for (int64_t i = 0; i < V; ++i) s += exp((double)xr[i] / T - m);
    for (int64_t i = 0; i < V; ++i) o[i] = exp((double)xr[i] / T - m) / s;
  }
}

/* Kept set of one row (flashinfer's filter semantics), kept[i] = 1/0:
 *   mode 0 every p > 0; 1 top_p: keep i iff sum_{p_j > p_i} p_j < top_p * sum_j p_j (the most
 *   probable tokens always stay, which matters only for top_p <= 0);
 *   2 top_k: keep i iff #{j : p_j > p_i} < k (all tokens tied with the k-th largest stay;
 *   k <= 0 or k >= V keeps all); 3 min_p: keep i iff p_i >= min_p * max_j p_j;
 *   4 top_k then top_p inside the top-k set (the top-p mass rule over that set).
 * Only p > 0 is ever kept; negative or NaN probabilities count as 0.                           */
static double pval(float p) { return p > 0.f ? (double)p : 0.0; }

typedef struct { double p; int64_t i; } PI;
static int cmp_desc(const void* x, const void* y) {
  const double a = ((const PI*)x)->p, b = ((const PI*)y)->p;
  return a < b ? 1 : a > b ? -1 : 0;
}

/* Sorts the positive probabilities once (descending) and applies the rules group by group of
 * equal values, so ties share one decision; O(V log V).                                     */
static void kept_set(const float* p, int64_t V, int mode, int32_t k, double top_p, double min_p,
                     unsigned char* kept) {
  PI* s = (PI*)malloc(sizeof(PI) * (size_t)(V > 0 ? V : 1));
  int64_t n = 0;
  for (int64_t i = 0; i < V; ++i) {
    kept[i] = 0;
    if (pval(p[i]) > 0) { s[n].p = pval(p[i]); s[n].i = i; ++n; }
  }
  qsort(s, (size_t)n, sizeof(PI), cmp_desc);
  int64_t m = n;  /* s[0..m) is the current kept set, most probable first */
  if ((mode == 2 || mode == 4) && k > 0 && k < n) {
    const double tau = s[k - 1].p;
    m = k;
    while (m < n && s[m].p == tau) ++m;
  }
  if (mode == 1 || mode == 4) {
    double tot = 0;
    for (int64_t j = 0; j < m; ++j) tot += s[j].p;
    double above = 0;
    int64_t j = 0, keep = 0;
    while (j < m) {
      int64_t e = j;
      double g = 0;
      while (e < m && s[e].p == s[j].p) { g += s[e].p; ++e; }
      if (above < top_p * tot || j == 0) keep = e; /* the most probable tokens always stay */
      else break;
      above += g;
      j = e;
    }
    m = keep;
  }
  if (mode == 3) {
    const double thr = n > 0 ? min_p * s[0].p : 0;
    int64_t e = 0;
    while (e < m && s[e].p >= thr) ++e;
    m = e;
  }
  for (int64_t j = 0; j < m; ++j) kept[s[j].i] = 1;
  free(s);
}

/* Inverse-CDF draw in index order over the kept set: the first kept index whose running kept
 * mass exceeds u * (total kept mass); -1 if nothing is kept. kept_out (optional) receives the
 * kept set, row-major [B, V].                                                                   */
void oracle_sample(const float* probs, int64_t B, int64_t V, int64_t stride, int mode,
                   const int32_t* top_k, const float* top_p, const float* min_p, const double* u,
                   int32_t* out, unsigned char* kept_out) {
  unsigned char* kept = (unsigned char*)malloc((size_t)(V > 0 ? V : 1));
  for (int64_t r = 0; r < B; ++r) {
    const float* p = probs + r * stride;
    kept_set(p, V, mode, top_k ? top_k[r] : 0, top_p ? top_p[r] : 1.0, min_p ? min_p[r] : 0.0, kept);
    if (kept_out) memcpy(kept_out + r * V, kept, (size_t)V);
    double tot = 0;
    for (int64_t i = 0; i < V; ++i) if (kept[i]) tot += pval(p[i]);
    const double target = u[r] * tot;
    int32_t pick = -1, last = -1;
    double run = 0;
    for (int64_t i = 0; i < V; ++i) {
      if (!kept[i]) continue;
      last = (int32_t)i;
      run += pval(p[i]);
      if (run > target) { pick = (int32_t)i; break; }
    }
    out[r] = pick >= 0 ? pick : last;
  }
  free(kept);
}
