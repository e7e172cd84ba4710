// Token-embedding gather for gfx950: out[t,:] = W[ids[t],:], a bit copy.
// Replaces fun.embedding(token_ids, W) (pie/src/pie_worker/model/llama3.py:471,
// qwen3.py:468-472; ids are int32 per llama3.py:429-433).
//
// The grid is flattened over 16-byte output vectors (1 KiB of one table row per wave
// instruction), so a decode batch of a few hundred tokens still spreads over every CU. Table
// rows are loaded with the normal cached path so the repeated ids of a batch are served from
// L2/MALL.
#include "common.h"




namespace pie {
namespace {

struct EmbedArgs {
  const int32_t* ids;
  const uint16_t* W;
  uint16_t* out;
  int64_t T, V, H, w_rs, out_rs;
  uint32_t nvec;  // T * H / 8 (vector path)
  FastDiv vpr;    // H / 8 vectors per row
  float scale;    // SCALE: out = bf16(f32(W[id]) * scale)
};

// Flattened over the 16-byte vectors of the output: thread t of block b copies vectors
// b*256*U + t + 256*i (i < U). All U table loads are issued before any store. The id of a
// vector's token is re-read per vector (an L1 hit); ids outside [0, V) give zero rows.
template <int U, bool SCALE>
__global__ __launch_bounds__(256) void embed_vec(EmbedArgs a) {
  prefetch_kernarg<(int)sizeof(EmbedArgs)>(a);
  const uint32_t base = blockIdx.x * (256u * U) + threadIdx.x;
  uint4 v[U];
  int64_t dst[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const uint32_t n = base + 256u * i;
    dst[i] = -1;
    if (n < a.nvec) {
      const uint32_t t = a.vpr.div(n), c = n - t * a.vpr.d;
      const int id = a.ids[t];
      dst[i] = (int64_t)t * a.out_rs + (int64_t)c * 8;
      v[i] = (id >= 0 && (int64_t)id < a.V) ? ld16(a.W + (int64_t)id * a.w_rs + (int64_t)c * 8)
                                            : make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < U; ++i) {
    if (dst[i] < 0) continue;
    if constexpr (SCALE) {
      float f[8];
      unpack8(v[i], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] *= a.scale;
      v[i] = pack8(f);
    }
    st_nt(a.out + dst[i], v[i]);
  }
}

template <bool SCALE>
__global__ __launch_bounds__(256) void embed_scalar(EmbedArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  for (int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); t < a.T; t += nwaves) {
    const int id = a.ids[t];
    uint16_t* o = a.out + t * a.out_rs;
    const bool ok = id >= 0 && (int64_t)id < a.V;
    for (int64_t c = lane; c < a.H; c += 64) {
      const uint16_t v = ok ? a.W[(int64_t)id * a.w_rs + c] : 0;
      o[c] = SCALE ? to_bf1(bf1(v) * a.scale) : v;
    }
  }
}

}  // namespace
}  // namespace pie

using namespace pie;

namespace {
template <bool SCALE>
int embedding_impl(const int32_t* ids, int64_t T, const pie_bf16* W, int64_t V, int64_t H,
                   int64_t w_row_stride, pie_bf16* out, int64_t out_row_stride, float scale,
                   void* stream) {
  PIE_REQUIRE(T >= 0 && V >= 0 && H >= 0, "embedding: bad shape");
  if (T == 0 || H == 0) return PIE_HIP_OK;
  PIE_REQUIRE(ids && out && (W || V == 0), "embedding: null pointer");
  PIE_REQUIRE(w_row_stride >= H && out_row_stride >= H, "embedding: row stride smaller than H");
  if (!SCALE && group_is_open())
    return group_add_embedding(EmbedRec{ids, T, W, V, H, w_row_stride, out, out_row_stride}, stream);
  EmbedArgs a{ids, W, out, T, V, H, w_row_stride, out_row_stride, 0, FastDiv{}, scale};
  const dim3 blk(256);
  const hipStream_t st = (hipStream_t)stream;
  const int64_t nvec = T * (H / 8);
  const bool vec = H % 8 == 0 && w_row_stride % 8 == 0 && out_row_stride % 8 == 0 &&
                   (V == 0 || aligned16(W)) && aligned16(out) && nvec < (1ll << 31);
  if (vec) {
    a.nvec = (uint32_t)nvec;
    a.vpr = FastDiv::make((uint32_t)(H / 8));
    // One 16-byte vector per thread (configuration 4 steady state: 6.29 TB/s, against 6.27
    // with 2 and 5.98 with 4 vectors per thread); the scaled form, whose arithmetic sits between
    // a vector's load and its store, two (44.2-44.7 us against 45.8-46.0 with one and 45.2-45.3
    // with four at configuration 4's shape).
    constexpr int U = SCALE ? 2 : 1;
    hipLaunchKernelGGL((embed_vec<U, SCALE>), dim3((unsigned)((nvec + 256 * U - 1) / (256 * U))), blk, 0, st, a);
  } else {
    const int64_t blocks = (T + 3) / 4, cap = (int64_t)num_cus() * 64;
    hipLaunchKernelGGL(embed_scalar<SCALE>, dim3((unsigned)(blocks < cap ? blocks : cap)), blk, 0, st, a);
  }
  return check_launch(SCALE ? "embedding_scaled" : "embedding");
}
}  // namespace

extern "C" int pie_hip_embedding(const int32_t* ids, int64_t T, const pie_bf16* W, int64_t V,
                                 int64_t H, int64_t w_row_stride, pie_bf16* out,
                                 int64_t out_row_stride, void* stream) {
  return embedding_impl<false>(ids, T, W, V, H, w_row_stride, out, out_row_stride, 1.0f, stream);
}

extern "C" int pie_hip_embedding_scaled(const int32_t* ids, int64_t T, const pie_bf16* W, int64_t V,
                                        int64_t H, int64_t w_row_stride, pie_bf16* out,
                                        int64_t out_row_stride, float scale, void* stream) {
  return embedding_impl<true>(ids, T, W, V, H, w_row_stride, out, out_row_stride, scale, stream);
}
