// Token-embedding gather for gfx950: out[t,:] = W[ids[t],:], a bit copy.
// Replaces fun.embedding(token_ids, W) (pie/src/pie_worker/model/llama3.py:471,
// qwen3.py:468-472; ids are int32 per llama3.py:429-433).
//
// One wavefront per token row: the id is read once into a scalar register, then each lane
// issues U independent 16-byte loads of the table row (1 KiB per wave instruction, fully
// coalesced) before storing them. Table rows are loaded with the normal cached path so the
// repeated ids of a batch are served from L2/MALL; the output is written non-temporally.
#include "common.h"

namespace pie {
namespace {

struct EmbedArgs {
  const int32_t* ids;
  const uint16_t* W;
  uint16_t* out;
  int64_t T, V, H, w_rs, out_rs;
};

template <int U>
__global__ __launch_bounds__(256) void embed_vec(EmbedArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  const int64_t nvec = a.H >> 3;
  for (int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); t < a.T; t += nwaves) {
    const int id = uniform(a.ids[t]);
    uint16_t* o = a.out + t * a.out_rs;
    if (id < 0 || (int64_t)id >= a.V) {
      for (int64_t c = lane; c < nvec; c += 64) st_stream(o + c * 8, make_uint4(0, 0, 0, 0));
      continue;
    }
    const uint16_t* src = a.W + (int64_t)id * a.w_rs;
    for (int64_t base = lane; base < nvec; base += 64 * U) {
      uint4 v[U];
#pragma unroll
      for (int i = 0; i < U; ++i)
        if (base + 64 * i < nvec) v[i] = ld16(src + (base + 64 * i) * 8);
#pragma unroll
      for (int i = 0; i < U; ++i)
        if (base + 64 * i < nvec) st_stream(o + (base + 64 * i) * 8, v[i]);
    }
  }
}

__global__ __launch_bounds__(256) void embed_scalar(EmbedArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  for (int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); t < a.T; t += nwaves) {
    const int id = a.ids[t];
    uint16_t* o = a.out + t * a.out_rs;
    const bool ok = id >= 0 && (int64_t)id < a.V;
    for (int64_t c = lane; c < a.H; c += 64) o[c] = ok ? a.W[(int64_t)id * a.w_rs + c] : 0;
  }
}

}  // namespace
}  // namespace pie

using namespace pie;

extern "C" int pie_hip_embedding(const int32_t* ids, int64_t T, const pie_bf16* W, int64_t V,
                                 int64_t H, int64_t w_row_stride, pie_bf16* out,
                                 int64_t out_row_stride, void* stream) {
  PIE_REQUIRE(T >= 0 && V >= 0 && H >= 0, "embedding: bad shape");
  if (T == 0 || H == 0) return PIE_HIP_OK;
  PIE_REQUIRE(ids && out && (W || V == 0), "embedding: null pointer");
  PIE_REQUIRE(w_row_stride >= H && out_row_stride >= H, "embedding: row stride smaller than H");
  EmbedArgs a{ids, W, out, T, V, H, w_row_stride, out_row_stride};
  const int64_t blocks = (T + 3) / 4, cap = (int64_t)num_cus() * 64;
  const dim3 grd((unsigned)(blocks < cap ? blocks : cap)), blk(256);
  const bool vec = H % 8 == 0 && w_row_stride % 8 == 0 && out_row_stride % 8 == 0 &&
                   (V == 0 || aligned16(W)) && aligned16(out);
  if (vec) hipLaunchKernelGGL(embed_vec<8>, grd, blk, 0, (hipStream_t)stream, a);
  else hipLaunchKernelGGL(embed_scalar, grd, blk, 0, (hipStream_t)stream, a);
  return check_launch("embedding");
}
