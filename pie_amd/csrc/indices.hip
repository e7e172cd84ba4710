// Per-forward-pass index helpers that feed the paged append (run once per forward pass,
// not per layer): flashinfer.get_seq_lens and flashinfer.get_batch_indices_positions as
// called at pie/src/pie_worker/model/llama3.py:745-755, restated in
// pie/src/flashinfer_metal/ops.py:392-436 (and the host-side positions of
// pie/src/pie_worker/batching.py:104-122).
//
// Both are single small launches with no host synchronisation, so the whole forward pass
// stays graph-capturable (the reference's Metal restatement loops on the host with .item()).
#include "common.h"

namespace pie {
namespace {

__global__ __launch_bounds__(256) void seq_lens_kernel(const int32_t* indptr, const int32_t* last,
                                                       int64_t B, int32_t P, int32_t* out) {
  const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int32_t np = indptr[b + 1] - indptr[b];
  out[b] = np > 0 ? (np - 1) * P + last[b] : 0;
}

// One thread per token: binary search for the last request whose start is <= t.
__global__ __launch_bounds__(256) void batch_pos_kernel(const int32_t* indptr, const int32_t* seq_lens,
                                                        int64_t B, int64_t nnz, int32_t* bidx,
                                                        int32_t* pos) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= nnz) return;
  if (B == 0 || t < indptr[0] || t >= indptr[B]) return;
  int64_t lo = 0, hi = B - 1;  // invariant: indptr[lo] <= t
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (indptr[mid] <= t) lo = mid;
    else hi = mid - 1;
  }
  const int32_t start = indptr[lo], end = indptr[lo + 1];
  if (t >= end) return;  // non-monotone indptr: no request owns t
  bidx[t] = (int32_t)lo;
  pos[t] = seq_lens[lo] - (end - start) + (int32_t)(t - start);
}

}  // namespace
}  // namespace pie

using namespace pie;

extern "C" int pie_hip_get_seq_lens(const int32_t* kv_indptr, const int32_t* last_page_len,
                                    int64_t batch_size, int64_t page_size, int32_t* seq_lens,
                                    void* stream) {
  PIE_REQUIRE(batch_size >= 0 && page_size > 0 && page_size < (1 << 30), "get_seq_lens: bad shape");
  if (batch_size == 0) return PIE_HIP_OK;
  PIE_REQUIRE(kv_indptr && last_page_len && seq_lens, "get_seq_lens: null pointer");
  const dim3 grd((unsigned)((batch_size + 255) / 256)), blk(256);
  hipLaunchKernelGGL(seq_lens_kernel, grd, blk, 0, (hipStream_t)stream, kv_indptr, last_page_len,
                     batch_size, (int32_t)page_size, seq_lens);
  return check_launch("get_seq_lens");
}

extern "C" int pie_hip_get_batch_indices_positions(const int32_t* append_indptr,
                                                   const int32_t* seq_lens, int64_t batch_size,
                                                   int64_t nnz, int32_t* batch_indices,
                                                   int32_t* positions, void* stream) {
  PIE_REQUIRE(batch_size >= 0 && nnz >= 0 && nnz < (1ll << 31), "get_batch_indices_positions: bad shape");
  if (nnz == 0 || batch_size == 0) return PIE_HIP_OK;
  PIE_REQUIRE(append_indptr && seq_lens && batch_indices && positions,
              "get_batch_indices_positions: null pointer");
  const dim3 grd((unsigned)((nnz + 255) / 256)), blk(256);
  hipLaunchKernelGGL(batch_pos_kernel, grd, blk, 0, (hipStream_t)stream, append_indptr, seq_lens,
                     batch_size, nnz, batch_indices, positions);
  return check_launch("get_batch_indices_positions");
}
