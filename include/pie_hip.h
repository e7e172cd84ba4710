/*
 * pie_hip.h — C ABI of the MI355X (gfx950) per-layer kernels of Pie's Python backend.
 *
 * Every entry point:
 *   - takes plain device pointers, element strides (in elements, not bytes) and sizes;
 *   - enqueues its kernels asynchronously on `stream` (a hipStream_t; NULL = the null stream);
 *   - never allocates, frees or synchronises, so it may be recorded into a HIP graph;
 *   - returns PIE_HIP_OK (0) or a nonzero PIE_HIP_E* code; pie_hip_last_error() then holds a
 *     message for the calling thread.
 *
 * bf16 buffers are passed as uint16_t (raw bfloat16 bits). int32 index buffers are int32_t.
 *
 * Reference interfaces each function replaces are cited as file:line of zyma98/pie
 * (paths relative to the repository root) or of the torch / flashinfer API those files call.
 */
#ifndef PIE_HIP_H
#define PIE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t pie_bf16;

enum {
  PIE_HIP_OK = 0,
  PIE_HIP_EINVAL = 1,  /* bad size, stride, null pointer or unsupported parameter */
  PIE_HIP_ELAUNCH = 2, /* the HIP runtime rejected the launch */
  PIE_HIP_EBUSY = 3,   /* shared device state (static scratch, a prefill plan) still in use by
                          a launch on another stream */
};

/* Message describing the last nonzero return on this thread ("" if none). */
const char* pie_hip_last_error(void);

/* ABI version; bumped whenever a signature below changes (2: paged attention and sampling;
 * 3: attention sinks). */
int pie_hip_abi_version(void);

/*
 * RMSNorm over the last dimension:
 *   y[r,:] = bf16( f32(x[r,:]) * rsqrt(mean_j f32(x[r,j])^2 + eps) * f32(w) )
 * Replaces torch.nn.functional.rms_norm(x, [cols], w, eps) at
 *   pie/src/pie_worker/model/llama3.py:555-560, :618-623, :504-509 and qwen3.py:538-543, :605-610.
 * y may alias x (same strides).
 */
int pie_hip_rmsnorm(const pie_bf16* x, int64_t x_row_stride,
                    const pie_bf16* w,
                    pie_bf16* y, int64_t y_row_stride,
                    int64_t rows, int64_t cols, float eps, void* stream);

/*
 * Gemma RMSNorm: the expression of pie/src/pie_worker/model/gemma2.py:514-526 and
 * gemma3.py:491-510 (and their q/k norm, gemma3.py:499-510),
 *   variance = x.pow(2).mean(-1); x * rsqrt(variance + eps) * (1.0 + weight)
 * evaluated as separate bf16 torch ops: every intermediate is rounded to bf16. Same arguments
 * as pie_hip_rmsnorm / pie_hip_fused_add_rmsnorm / pie_hip_qk_rmsnorm (the add variant sums
 * first, as `residual + down` (gemma3.py:585) feeding the next layer's norm).
 */
int pie_hip_gemma_rmsnorm(const pie_bf16* x, int64_t x_row_stride, const pie_bf16* w,
                          pie_bf16* y, int64_t y_row_stride, int64_t rows, int64_t cols, float eps,
                          void* stream);
int pie_hip_gemma_fused_add_rmsnorm(const pie_bf16* x, int64_t x_row_stride, const pie_bf16* r,
                                    int64_t r_row_stride, pie_bf16* s, int64_t s_row_stride,
                                    pie_bf16* y, int64_t y_row_stride, const pie_bf16* w,
                                    int64_t rows, int64_t cols, float eps, void* stream);
int pie_hip_gemma_qk_rmsnorm(const pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride,
                             pie_bf16* q_out, int64_t qo_tok_stride, int64_t qo_head_stride,
                             const pie_bf16* k, int64_t k_tok_stride, int64_t k_head_stride,
                             pie_bf16* k_out, int64_t ko_tok_stride, int64_t ko_head_stride,
                             const pie_bf16* qw, const pie_bf16* kw, int64_t T, int64_t Hq,
                             int64_t Hkv, int64_t D, float eps, void* stream);

/*
 * Residual add followed by RMSNorm of the sum:
 *   s = bf16(f32(r) + f32(x));  y = rmsnorm(s)
 * Replaces `residual + down` / `residual + attn_proj` (llama3.py:586, :710; qwen3.py:571, :710)
 * together with the next layer's fun.rms_norm (llama3.py:555/:618). Both the new residual
 * stream s and the normalised y are written. s may alias r or x.
 */
int pie_hip_fused_add_rmsnorm(const pie_bf16* x, int64_t x_row_stride,
                              const pie_bf16* r, int64_t r_row_stride,
                              pie_bf16* s, int64_t s_row_stride,
                              pie_bf16* y, int64_t y_row_stride,
                              const pie_bf16* w,
                              int64_t rows, int64_t cols, float eps, void* stream);

/*
 * Per-head RMSNorm of q [T,Hq,D] (weight qw[D]) and k [T,Hkv,D] (weight kw[D]) in one launch.
 * Replaces the two fun.rms_norm calls at qwen3.py:651-662 (normalized_shape=[D]).
 * Inputs may be strided views (token stride, head stride; innermost stride 1).
 * Outputs may alias inputs.
 */
int pie_hip_qk_rmsnorm(const pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride,
                       pie_bf16* q_out, int64_t qo_tok_stride, int64_t qo_head_stride,
                       const pie_bf16* k, int64_t k_tok_stride, int64_t k_head_stride,
                       pie_bf16* k_out, int64_t ko_tok_stride, int64_t ko_head_stride,
                       const pie_bf16* qw, const pie_bf16* kw,
                       int64_t T, int64_t Hq, int64_t Hkv, int64_t D, float eps, void* stream);

/*
 * SiLU-and-mul over gate_up [rows, 2I] (gate = cols [0,I), up = cols [I,2I)):
 *   out = bf16( f32(bf16(silu(f32(gate)))) * f32(up) )
 * Replaces `gate, up = torch.split(gate_up, [I, I], -1); fun.silu(gate) * up`
 * at llama3.py:569-572 and qwen3.py:553-556.
 */
int pie_hip_silu_and_mul(const pie_bf16* gate_up, int64_t in_row_stride,
                         pie_bf16* out, int64_t out_row_stride,
                         int64_t rows, int64_t I, void* stream);

/*
 * GELU(tanh)-and-mul: out = bf16( f32(bf16(gelu_tanh(f32(gate)))) * f32(up) ), the
 * `_gelu_pytorch_tanh(gate) * up` of pie/src/pie_worker/model/gemma2.py:224-226, :608 and
 * gemma3.py:246-248, :566 (torch gelu with approximate="tanh"). Same layout as
 * pie_hip_silu_and_mul.
 */
int pie_hip_gelu_tanh_and_mul(const pie_bf16* gate_up, int64_t in_row_stride,
                              pie_bf16* out, int64_t out_row_stride,
                              int64_t rows, int64_t I, void* stream);

/*
 * Token-embedding gather: out[t,:] = W[ids[t],:] (bit copy).
 * Replaces fun.embedding(token_ids, W) at llama3.py:471 and qwen3.py:468-472.
 * Ids outside [0, V) produce a zero row (torch raises instead; a graph-capturable kernel
 * cannot, so the Python wrapper offers an explicit host-side check).
 */
int pie_hip_embedding(const int32_t* ids, int64_t T,
                      const pie_bf16* W, int64_t V, int64_t H, int64_t w_row_stride,
                      pie_bf16* out, int64_t out_row_stride, void* stream);

/*
 * Scaled embedding: out[t,:] = bf16(f32(W[ids[t],:]) * scale), the
 * `fun.embedding(ids, W) * self.embed_normalizer` of pie/src/pie_worker/model/gemma3.py:476-489
 * and gemma2.py (scale = fp32(sqrt(hidden))). Out-of-range ids give zero rows.
 */
int pie_hip_embedding_scaled(const int32_t* ids, int64_t T,
                             const pie_bf16* W, int64_t V, int64_t H, int64_t w_row_stride,
                             pie_bf16* out, int64_t out_row_stride, float scale, void* stream);

/*
 * Rotary embedding applied in place to q [T,Hq,D] and k [T,Hkv,D] at positions pos[T].
 * inv_freq is a HOST array of rotary_dim/2 fp32 inverse frequencies (<= 256 entries); it is
 * copied into the kernel arguments, so no device table exists.
 * interleave=0 rotates (v[i], v[i+rotary_dim/2]) (NeoX half split); interleave=1 rotates
 * (v[2i], v[2i+1]). Dimensions >= rotary_dim are left untouched.
 * Replaces flashinfer.apply_rope_pos_ids_inplace (qwen3.py:665-670) and
 * flashinfer.apply_llama31_rope_pos_ids_inplace (llama3.py:660-669); the frequency rules
 * are computed on the host by pie_hip_rope_inv_freq / pie_hip_llama31_inv_freq.
 */
int pie_hip_rope_inplace(pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride,
                         pie_bf16* k, int64_t k_tok_stride, int64_t k_head_stride,
                         const int32_t* pos, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                         int64_t rotary_dim, int interleave, const float* inv_freq,
                         void* stream);

/*
 * RoPE in place from a precomputed fp32 table: row pos[t] of cos_sin_cache holds cos at
 * [0, rotary_dim/2) and sin at [rotary_dim/2, rotary_dim) (row stride cache_ld elements).
 * interleave=0 is is_neox=True. Positions outside [0, cache_rows) leave the token unchanged.
 * Replaces flashinfer.apply_rope_with_cos_sin_cache_inplace (gpt_oss.py:671-678,
 * olmo3.py:797-804; YaRN tables built at gpt_oss.py:520-547, olmo3.py:447-525).
 */
int pie_hip_rope_cos_sin_cache_inplace(pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride,
                                       pie_bf16* k, int64_t k_tok_stride, int64_t k_head_stride,
                                       const int32_t* pos, int64_t T, int64_t Hq, int64_t Hkv,
                                       int64_t D, int interleave, const float* cos_sin_cache,
                                       int64_t cache_rows, int64_t rotary_dim, int64_t cache_ld,
                                       void* stream);

/*
 * Host helpers: fill inv_freq[rotary_dim/2] (computed in float64, rounded to fp32).
 *   standard:  f_i = 1 / (rope_scale * theta^(2i/rotary_dim))
 *   llama31:   f_i = theta^(-2i/rotary_dim), then wavelength-based smoothing with
 *              (rope_scale, low_freq_factor, high_freq_factor, old_context_len)
 * Follow pie/src/flashinfer_metal/kernels/metal_rope.metal:63-89 and
 * flashinfer_metal/ops.py:285-346.
 */
int pie_hip_rope_inv_freq(float* inv_freq, int64_t rotary_dim, float rope_scale, float rope_theta);
int pie_hip_llama31_inv_freq(float* inv_freq, int64_t rotary_dim, float rope_scale,
                             float rope_theta, float low_freq_factor, float high_freq_factor,
                             float old_context_len);

/*
 * Paged KV append: for token t, b = batch_indices[t], p = positions[t],
 *   page = kv_indices[kv_indptr[b] + p / page_size], slot = p % page_size,
 *   k_cache[page*page_stride + slot*slot_stride + h*head_stride + d] = k[t,h,d]   (same for v).
 * Tokens whose batch index, logical page or physical page is out of range are skipped, as in
 * pie/src/flashinfer_metal/kernels/metal_append_paged_kv_cache.metal:51-70.
 * Cache strides cover the reference layouts: NHD [pages,2,P,Hkv,D] (llama3.py:966-979) gives
 * page_stride=2*P*Hkv*D, slot_stride=Hkv*D, head_stride=D, v_cache=k_cache+P*Hkv*D; HND and
 * split (k_cache, v_cache) tensors are other stride choices.
 * Replaces flashinfer.append_paged_kv_cache (llama3.py:675-685, qwen3.py:674-684).
 */
int pie_hip_paged_kv_append(const pie_bf16* k, int64_t k_tok_stride, int64_t k_head_stride,
                            const pie_bf16* v, int64_t v_tok_stride, int64_t v_head_stride,
                            const int32_t* batch_indices, const int32_t* positions,
                            const int32_t* kv_indices, const int32_t* kv_indptr,
                            int64_t batch_size,
                            pie_bf16* k_cache, pie_bf16* v_cache, int64_t num_pages,
                            int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                            int64_t page_size, int64_t T, int64_t Hkv, int64_t D, void* stream);

/*
 * Fused RoPE (in place on q and k, positions pos[T]) + paged append of the rotated k and raw
 * v: one HBM pass over q/k/v instead of two. Equivalent to pie_hip_rope_inplace followed by
 * pie_hip_paged_kv_append with the same arguments (llama3.py:660-685 call order).
 */
int pie_hip_rope_append(pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride,
                        pie_bf16* k, int64_t k_tok_stride, int64_t k_head_stride,
                        const pie_bf16* v, int64_t v_tok_stride, int64_t v_head_stride,
                        const int32_t* pos, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                        int64_t rotary_dim, int interleave, const float* inv_freq,
                        const int32_t* batch_indices, const int32_t* positions,
                        const int32_t* kv_indices, const int32_t* kv_indptr,
                        int64_t batch_size,
                        pie_bf16* k_cache, pie_bf16* v_cache, int64_t num_pages,
                        int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                        int64_t page_size, void* stream);

/*
 * Per-head q/k RMSNorm + standard/any-frequency RoPE + paged append in one pass: the
 * consecutive calls of pie/src/pie_worker/model/qwen3.py:651-684 (fun.rms_norm on q and k,
 * flashinfer.apply_rope_pos_ids_inplace, flashinfer.append_paged_kv_cache). Reads q/k/v (views
 * of the qkv projection), writes normalised+rotated q_out/k_out and the k/v cache rows. Full
 * rotary dim, half-split pairs. Results equal pie_hip_qk_rmsnorm followed by
 * pie_hip_rope_append on (q_out, k_out, v) bit for bit (that path is taken for D != 128 or
 * unaligned tensors).
 */
int pie_hip_qk_rmsnorm_rope_append(const pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride,
                                   const pie_bf16* k, int64_t k_tok_stride, int64_t k_head_stride,
                                   const pie_bf16* v, int64_t v_tok_stride, int64_t v_head_stride,
                                   pie_bf16* q_out, int64_t qo_tok_stride, int64_t qo_head_stride,
                                   pie_bf16* k_out, int64_t ko_tok_stride, int64_t ko_head_stride,
                                   const pie_bf16* qw, const pie_bf16* kw, float eps,
                                   const int32_t* pos, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                                   const float* inv_freq, const int32_t* batch_indices,
                                   const int32_t* positions, const int32_t* kv_indices,
                                   const int32_t* kv_indptr, int64_t batch_size,
                                   pie_bf16* k_cache, pie_bf16* v_cache, int64_t num_pages,
                                   int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                                   int64_t page_size, void* stream);

/*
 * Grouped launch of independent per-layer ops: after pie_hip_group_begin, calls on this thread
 * of pie_hip_embedding, pie_hip_fused_add_rmsnorm, pie_hip_silu_and_mul,
 * pie_hip_gelu_tanh_and_mul and pie_hip_qk_rmsnorm_rope_append validate their arguments and are
 * recorded (at most 8) instead of launched; pie_hip_group_end(stream) launches them, all on
 * `stream` (every recorded call must name that stream), as ONE kernel whose block ranges run
 * one q/k prologue, one add + RMSNorm (cols = 512, 1024, 2048 or 4096) and one gated activation
 * side by side; whatever does not fit is launched after it as its own kernel. Results equal the
 * separate calls' bit for bit. The recorded ops must be independent, with one exception: an
 * embedding whose output is the x of a recorded add + RMSNorm (same rows, cols and row stride)
 * runs fused into it, as the sequence embedding -> add -> norm. Any other overlap between one
 * op's outputs and another op's operands makes pie_hip_group_end fail without launching. Other
 * entry points called inside a group launch immediately. The group closes at
 * pie_hip_group_end even when it fails.
 * No single reference function: it replaces consecutive launches of the ops above in a decode
 * step (pie/src/pie_worker/model/qwen3.py:468-472, :571 -> :538, :651-684, :553-556), which the
 * reference issues one kernel each.
 */
int pie_hip_group_begin(void);
int pie_hip_group_end(void* stream);

/*
 * A recorded group kept for relaunching: pie_hip_group_save closes the open group like
 * pie_hip_group_end (same checks, same kernels) but launches nothing and returns a handle;
 * pie_hip_group_launch(group, stream) launches what pie_hip_group_end would have, on `stream`,
 * reading and writing the recorded buffers at launch time, as often as the caller likes (a decode
 * loop whose ops keep their buffers from step to step: one call per step, no per-op argument
 * validation). The caller keeps every recorded buffer alive and in place while the handle is
 * used; pie_hip_group_free releases the handle (host memory only).
 * No reference counterpart: it replaces the per-step re-issue of the grouped ops' launches.
 */
int pie_hip_group_save(void* stream, void** group);
int pie_hip_group_launch(const void* group, void* stream);
void pie_hip_group_free(void* group);

/*
 * seq_lens[b] = (kv_indptr[b+1]-kv_indptr[b]-1)*page_size + last_page_len[b], or 0 when the
 * request holds no page. Replaces flashinfer.get_seq_lens (llama3.py:745-749;
 * spec pie/src/flashinfer_metal/ops.py:392-407).
 */
int pie_hip_get_seq_lens(const int32_t* kv_indptr, const int32_t* last_page_len,
                         int64_t batch_size, int64_t page_size, int32_t* seq_lens, void* stream);

/*
 * For every token t in request b (append_indptr[b] <= t < append_indptr[b+1]):
 *   batch_indices[t] = b,  positions[t] = seq_lens[b] - (append_indptr[b+1]-append_indptr[b])
 *                                          + (t - append_indptr[b]).
 * Tokens t < nnz outside every request are left untouched.
 * Replaces flashinfer.get_batch_indices_positions (llama3.py:751-755;
 * spec pie/src/flashinfer_metal/ops.py:410-436).
 */
int pie_hip_get_batch_indices_positions(const int32_t* append_indptr, const int32_t* seq_lens,
                                        int64_t batch_size, int64_t nnz,
                                        int32_t* batch_indices, int32_t* positions,
                                        void* stream);


/*
 * Paged attention, decode form: one query token per request (query row b = request b),
 *   out[b, h, :] = softmax_t( q[b,h,:] . k_t * sm_scale ) @ v_t   over the request's kv_len tokens,
 * k_t / v_t of kv head h / (Hq/Hkv) read from the paged cache (token t in page
 * kv_indices[kv_indptr[b] + t/P], slot t%P; element (page, slot, head, d) at
 * page*page_stride + slot*slot_stride + head*head_stride + d from k_cache / v_cache).
 * Replaces flashinfer.BatchDecodeWithPagedKVCacheWrapper.plan/.run as Pie calls them:
 *   pie/src/pie_worker/model/llama3.py:293-301, :765-777 (plan), :689 (run); the API restated
 *   in pie/src/flashinfer_metal/ops.py:226-282.
 *
 * pie_hip_attention_decode_plan (host only) picks `splits`, the number of pieces each request's
 * kv range is cut into (max_kv_len < 0: unknown). pie_hip_attention_decode launches
 * batch * splits work groups per kv head; each piece's range is derived on the device from the
 * request's current length, so one launch configuration (and one captured graph) serves any
 * lengths, as Pie's graph replay requires (llama3.py:340-414, :905-950). Batches of at most 256
 * requests are worked on longest request first (the order is found on the device, per launch);
 * the results do not depend on the order. With splits > 1 the
 * run needs `workspace` (16-byte aligned) of batch * splits * num_qo_heads * (head_dim + 1) * 4
 * bytes. head_dim in {64, 128, 256}; num_qo_heads / num_kv_heads <= 16. Page ids outside
 * [0, num_pages) are treated as masked positions. window_left >= 0 is flashinfer's sliding
 * window (as olmo3.py:381-391, :973-1005 plans it): the query at position p = kv_len - 1 sees only
 * positions >= p - window_left; -1 = no window.
 * sinks: NULL, or fp32 [num_qo_heads] attention-sink logits in the units of the scaled scores
 * (gpt-oss, pie/src/pie_worker/model/gpt_oss.py:693-697, flashinfer's
 * BatchAttentionWithAttentionSinkWrapper): head h's softmax denominator gains exp(sinks[h] - max)
 * and no value, i.e. out = sum_t e^{s_t} v_t / (sum_t e^{s_t} + e^{sinks[h]}).
 */
int pie_hip_attention_decode_plan(int64_t batch, int64_t num_kv_heads, int64_t max_kv_len,
                                  int64_t num_cus, int64_t* splits);
int pie_hip_attention_decode(const pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride,
                             const pie_bf16* k_cache, const pie_bf16* v_cache, int64_t page_stride,
                             int64_t slot_stride, int64_t head_stride, int64_t num_pages,
                             const int32_t* kv_indptr, const int32_t* kv_indices,
                             const int32_t* kv_last_page_len, int64_t batch, int64_t num_qo_heads,
                             int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                             float sm_scale, int64_t window_left, const float* sinks,
                             int64_t splits, void* workspace,
                             int64_t workspace_bytes,
                             pie_bf16* out, int64_t o_tok_stride, int64_t o_head_stride,
                             void* stream);


/*
 * pie_hip_attention_decode without a workspace argument and without any allocation: the split
 * partials go to a static device array of 32 MiB held by each GPU the library runs on until the
 * process ends (need = batch * splits * num_qo_heads * (head_dim + 1) * 4 bytes when splits > 1;
 * larger requests return PIE_HIP_EINVAL). Results equal pie_hip_attention_decode's bit for bit.
 * No counterpart in the reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops). Calls that overlap on one GPU share the array and race, so
 * use it from one stream per GPU: an eager call (splits > 1) made while the previous one is
 * still running on a different stream returns PIE_HIP_EBUSY instead of racing. Calls recorded
 * under graph capture are not checked; replays of such graphs must not overlap other users.
 */
int pie_hip_attention_decode_noalloc(const pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride,
                                     const pie_bf16* k_cache, const pie_bf16* v_cache,
                                     int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                                     int64_t num_pages, const int32_t* kv_indptr,
                                     const int32_t* kv_indices, const int32_t* kv_last_page_len,
                                     int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads,
                                     int64_t head_dim, int64_t page_size, float sm_scale,
                                     int64_t window_left, const float* sinks, int64_t splits,
                                     pie_bf16* out,
                                     int64_t o_tok_stride, int64_t o_head_stride, void* stream);

/*
 * Paged attention, prefill form: ragged query tokens per request (qo_indptr [B+1]), each
 * request's query tokens being its last qo_len positions. Query token i of request b attends
 * kv position t < kv_len when: mode 0 always (flashinfer's default, causal=False), mode 1
 * t <= kv_len - qo_len + i (causal=True), mode 2 custom_mask[off_b + i*kv_len + t] != 0 (bytes;
 * per request a row-major [qo_len, kv_len] block, blocks concatenated in request order, as
 * pie/src/pie_worker/batching.py:335-386 builds it). Cache addressing, heads and scale as in
 * the decode form. window_left >= 0 additionally hides positions t < p - window_left, with
 * p = kv_len - qo_len + i the query's own position (flashinfer's sliding window; -1 = none).
 * Rows that see nothing are 0. sinks: as in the decode form (NULL = none).
 * Replaces flashinfer.BatchPrefillWithPagedKVCacheWrapper.plan/.run as Pie calls them:
 *   pie/src/pie_worker/model/llama3.py:307-309 (construction), :779-790 (plan with the custom
 *   mask), :689 (run); API restated in pie/src/flashinfer_metal/ops.py:163-223.
 *
 * pie_hip_attention_prefill_plan runs on the host over host copies of qo_indptr, kv_indptr and
 * kv_last_page_len and writes the work list (`plan`, int32 words: 16 header words, then 8 per
 * work item, so plan_capacity >= 16 + 8 * (num_tokens * num_qo_heads / num_kv_heads / 64 +
 * batch + 1) + 4 * (batch + 1) always suffices; *num_items work groups per kv
 * head; for mode 2 the int64 byte offsets of the mask blocks at word plan[3] and of their packed
 * words at plan[4], *mask_bytes = the mask's size, *mask_words = its packed size in uint32).
 * The caller copies the plan to device memory. For mode 2, pie_hip_attention_pack_mask (device,
 * on the stream) packs the byte mask into 32-position words (bit j of word w of query token i =
 * position 32w+j; 0 past kv_len) in a caller buffer of mask_words uint32, and writes every query
 * token's visible extent (1 + its last visible position; int32 [num_tokens]) so the run skips kv
 * tiles no row of a work group can see. The run reads both with the plan, num_items and plan[4]
 * (mask_offsets_word). For head_dim 128 the run also writes the device copy of the plan: header
 * words 7-15 count the work taken (one queue per XCD) and are back to zero when the run ends, so
 * the device plan is mutable state: two runs with one plan must not overlap in time (on one
 * stream they never do). An eager run whose plan is still in use by a run on another stream
 * returns PIE_HIP_EBUSY; runs recorded under graph capture are not checked. A plan made for
 * head_dim 256 run with head_dim 64/128 (or the reverse) fills the output with NaN.
 */
int pie_hip_attention_prefill_plan(const int32_t* qo_indptr, const int32_t* kv_indptr,
                                   const int32_t* kv_last_page_len, int64_t batch,
                                   int64_t page_size, int64_t num_qo_heads, int64_t num_kv_heads,
                                   int64_t head_dim, int32_t mode, int32_t* plan, int64_t plan_capacity,
                                   int64_t* plan_words, int64_t* num_items, int64_t* mask_bytes,
                                   int64_t* mask_words);
int pie_hip_attention_pack_mask(const uint8_t* custom_mask, const int32_t* plan,
                                const int32_t* qo_indptr, const int32_t* kv_indptr,
                                const int32_t* kv_last_page_len, int64_t batch, int64_t page_size,
                                int64_t mask_words, int64_t num_tokens, uint32_t* packed_mask,
                                int32_t* mask_extent, void* stream);
int pie_hip_attention_prefill(const pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride,
                              const pie_bf16* k_cache, const pie_bf16* v_cache,
                              int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                              int64_t num_pages, const int32_t* qo_indptr,
                              const int32_t* kv_indptr, const int32_t* kv_indices,
                              const int32_t* kv_last_page_len, int64_t num_qo_heads,
                              int64_t num_kv_heads, int64_t head_dim, int64_t page_size,
                              float sm_scale, int32_t mode, int64_t window_left,
                              const float* sinks,
                              const uint32_t* packed_mask, const int32_t* mask_extent,
                              const int32_t* plan, int64_t num_items,
                              int64_t mask_offsets_word,
                              pie_bf16* out, int64_t o_tok_stride, int64_t o_head_stride,
                              void* stream);


/*
 * Sampling from probabilities, one draw per row: flashinfer.sampling.sampling_from_probs (mode 0),
 * top_p_ (1), top_k_ (2), min_p_ (3) and top_k_top_p_sampling_from_probs (4) as Pie calls them
 * (pie/src/pie_worker/model/common.py:316-344; API restated in
 * pie/src/flashinfer_metal/sampling.py:19-79).
 * probs: fp32 [prob_rows, prob_stride], non-negative (NaN and p <= 0 are never drawn). Output
 * row r uses probs row row_indices[r] (NULL: row r; an index outside [0, prob_rows) gives -1). Kept set: top_p keeps token i iff the mass of
 * strictly more probable tokens is below top_p times the row's (top-k set's) mass; top_k keeps i
 * iff fewer than k tokens are strictly more probable (k <= 0 or k >= vocab keeps all); min_p keeps
 * p_i >= min_p * max p. Per-row parameters come from the arrays when non-NULL, else the scalars.
 * The draw is the first kept index (in index order) whose running kept mass exceeds u times the
 * kept mass, u = uniforms[r] when non-NULL, else Philox4x32-10 of (seed, offset, r). Masses are
 * summed in 64-bit fixed point (2^-40), so results do not depend on thread order.
 * out: int32 [batch]; a row with nothing kept gives -1.
 */
int pie_hip_sample(const float* probs, int64_t prob_stride, int64_t prob_rows, int64_t vocab,
                   int64_t batch, const int32_t* row_indices, int32_t mode, const int32_t* top_k,
                   int32_t top_k_scalar, const float* top_p, float top_p_scalar,
                   const float* min_p, float min_p_scalar, const double* uniforms, uint64_t seed,
                   uint64_t offset, int32_t* out, void* stream);

/*
 * safe_scaled_softmax of pie/src/pie_worker/model/common.py:38-59, :68-188 (the Triton kernel Pie
 * runs on GPUs): per row, softmax(logits / T) with fp32 math, or the one-hot of the first maximum
 * when T < greedy_threshold (greedy decoding). logits and out are fp32 (is_bf16 = 0) or bf16
 * (is_bf16 = 1), out in the logits' dtype; temperatures: fp32 [batch]. out may alias logits.
 */
int pie_hip_scaled_softmax(const void* logits, int32_t is_bf16, int64_t stride, int64_t batch,
                           int64_t vocab, const float* temperatures, float greedy_threshold,
                           void* out, int64_t out_stride, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PIE_HIP_H */
