// SiLU-and-mul for gfx950.
//
// Reference expression (pie/src/pie_worker/model/llama3.py:569-572, qwen3.py:553-556):
//   gate, up = torch.split(gate_up, [I, I], dim=-1);  hidden = fun.silu(gate) * up
// torch evaluates silu in fp32 and rounds it to bf16, then multiplies in fp32 and rounds again:
//   out = bf16( f32(bf16(g / (1 + exp(-g)))) * f32(up) ).
// This kernel keeps both roundings, so it differs from torch only through exp().
//
// One pass over HBM: read gate_up [rows, 2I], write out [rows, I] (the reference makes three
// passes plus a [rows, I] temporary). One 256-thread block per row; each thread issues U
// independent 16-byte gate loads and U up loads before any math, so every CU keeps
// > 64 KiB of reads in flight.
#include "common.h"

namespace pie {
namespace {

__device__ __forceinline__ float silu_bf(float g) {
  // exp(-g) via the hardware base-2 exponential; 1/(1+e) via the hardware reciprocal.
  const float e = __builtin_amdgcn_exp2f(-g * 1.44269504088896341f);
  return round_bf(g * __builtin_amdgcn_rcpf(1.0f + e));
}

struct SiluArgs {
  const uint16_t* in;
  uint16_t* out;
  int64_t in_rs, out_rs, rows, I;
};

template <int U>
__global__ __launch_bounds__(256) void silu_and_mul_vec(SiluArgs a) {
  const int64_t nvec = a.I >> 3;
  for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
    const uint16_t* g = a.in + row * a.in_rs;
    const uint16_t* u = g + a.I;
    uint16_t* o = a.out + row * a.out_rs;
    for (int64_t base = threadIdx.x; base < nvec; base += 256 * U) {
      uint4 gv[U], uv[U];
#pragma unroll
      for (int i = 0; i < U; ++i) {
        const int64_t c = base + 256 * i;
        if (c < nvec) {
          gv[i] = ld_stream(g + c * 8);
          uv[i] = ld_stream(u + c * 8);
        }
      }
#pragma unroll
      for (int i = 0; i < U; ++i) {
        const int64_t c = base + 256 * i;
        if (c < nvec) {
          float gf[8], uf[8];
          unpack8(gv[i], gf);
          unpack8(uv[i], uf);
#pragma unroll
          for (int e = 0; e < 8; ++e) gf[e] = silu_bf(gf[e]) * uf[e];
          st_stream(o + c * 8, pack8(gf));
        }
      }
    }
  }
}

__global__ __launch_bounds__(256) void silu_and_mul_scalar(SiluArgs a) {
  for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
    const uint16_t* g = a.in + row * a.in_rs;
    uint16_t* o = a.out + row * a.out_rs;
    for (int64_t c = threadIdx.x; c < a.I; c += 256)
      o[c] = to_bf1(silu_bf(bf1(g[c])) * bf1(g[a.I + c]));
  }
}

}  // namespace
}  // namespace pie

using namespace pie;

extern "C" int pie_hip_silu_and_mul(const pie_bf16* gate_up, int64_t in_row_stride, pie_bf16* out,
                                    int64_t out_row_stride, int64_t rows, int64_t I, void* stream) {
  PIE_REQUIRE(rows >= 0 && I >= 0, "silu_and_mul: bad shape rows=%lld I=%lld", (long long)rows, (long long)I);
  if (rows == 0 || I == 0) return PIE_HIP_OK;
  PIE_REQUIRE(gate_up && out, "silu_and_mul: null pointer");
  PIE_REQUIRE(in_row_stride >= 2 * I && out_row_stride >= I, "silu_and_mul: row stride too small");
  SiluArgs a{gate_up, out, in_row_stride, out_row_stride, rows, I};
  const int64_t cap = (int64_t)num_cus() * 64;
  const dim3 grd((unsigned)(rows < cap ? rows : cap)), blk(256);
  const bool vec = I % 8 == 0 && in_row_stride % 8 == 0 && out_row_stride % 8 == 0 &&
                   aligned16(gate_up) && aligned16(out);
  if (vec) hipLaunchKernelGGL(silu_and_mul_vec<4>, grd, blk, 0, (hipStream_t)stream, a);
  else hipLaunchKernelGGL(silu_and_mul_scalar, grd, blk, 0, (hipStream_t)stream, a);
  return check_launch("silu_and_mul");
}
