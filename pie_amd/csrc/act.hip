// SiLU-and-mul for gfx950.
//
// Reference expression (pie/src/pie_worker/model/llama3.py:569-572, qwen3.py:553-556):
//   gate, up = torch.split(gate_up, [I, I], dim=-1);  hidden = fun.silu(gate) * up
// torch evaluates silu in fp32 and rounds it to bf16, then multiplies in fp32 and rounds again:
//   out = bf16( f32(bf16(g / (1 + exp(-g)))) * f32(up) ).
// This kernel keeps both roundings, so it differs from torch only through exp().
//
// One pass over HBM: read gate_up [rows, 2I], write out [rows, I] (the reference makes three
// passes plus a [rows, I] temporary). The grid is flattened over output vectors; each thread
// issues U independent 16-byte gate loads and U up loads before any math.
#include "act_dev.h"

namespace pie {
namespace {

template <int U, int ACT>
__global__ __launch_bounds__(256) void silu_and_mul_vec(SiluArgs a) {
  prefetch_kernarg<(int)sizeof(SiluArgs)>(a);
  act_and_mul_block<U, ACT>(a, blockIdx.x);
}

template <int ACT>
__global__ __launch_bounds__(256) void silu_and_mul_scalar(SiluArgs a) {
  for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
    const uint16_t* g = a.in + row * a.in_rs;
    uint16_t* o = a.out + row * a.out_rs;
    for (int64_t c = threadIdx.x; c < a.I; c += 256)
      o[c] = to_bf1((ACT == kSilu ? silu_bf(bf1(g[c])) : gelu_tanh_bf(bf1(g[c]))) * bf1(g[a.I + c]));
  }
}

}  // namespace
}  // namespace pie

using namespace pie;

namespace {
template <int ACT>
int act_and_mul(const pie_bf16* gate_up, int64_t in_row_stride, pie_bf16* out,
                int64_t out_row_stride, int64_t rows, int64_t I, void* stream) {
  PIE_REQUIRE(rows >= 0 && I >= 0, "act_and_mul: bad shape rows=%lld I=%lld", (long long)rows, (long long)I);
  if (rows == 0 || I == 0) return PIE_HIP_OK;
  PIE_REQUIRE(gate_up && out, "silu_and_mul: null pointer");
  PIE_REQUIRE(in_row_stride >= 2 * I && out_row_stride >= I, "silu_and_mul: row stride too small");
  if (group_is_open())
    return group_add_act(ActRec{gate_up, in_row_stride, out, out_row_stride, rows, I, ACT == kGeluTanh}, stream);
  SiluArgs a{gate_up, out, in_row_stride, out_row_stride, rows, I, 0, FastDiv{}};
  const dim3 blk(256);
  const int64_t nvec = rows * (I / 8);
  const bool vec = I % 8 == 0 && in_row_stride % 8 == 0 && out_row_stride % 8 == 0 &&
                   aligned16(gate_up) && aligned16(out) && nvec < (1ll << 31);
  if (vec) {
    a.nvec = (uint32_t)nvec;
    a.vpr = FastDiv::make((uint32_t)(I / 8));
    // One 16-byte vector per thread over a grid of nvec/256 blocks: measured fastest on MI355X
    // (configuration 2 steady state: 6.46 TB/s, against 6.25 with 2 and 5.99 with 4 vectors).
    hipLaunchKernelGGL((silu_and_mul_vec<1, ACT>), dim3((unsigned)((nvec + 255) / 256)), blk, 0,
                       (hipStream_t)stream, a);
  } else {
    const int64_t cap = (int64_t)num_cus() * 64;
    hipLaunchKernelGGL(silu_and_mul_scalar<ACT>, dim3((unsigned)(rows < cap ? rows : cap)), blk, 0,
                       (hipStream_t)stream, a);
  }
  return check_launch(ACT == kSilu ? "silu_and_mul" : "gelu_tanh_and_mul");
}
}  // namespace

extern "C" int pie_hip_silu_and_mul(const pie_bf16* gate_up, int64_t in_row_stride, pie_bf16* out,
                                    int64_t out_row_stride, int64_t rows, int64_t I, void* stream) {
  return act_and_mul<kSilu>(gate_up, in_row_stride, out, out_row_stride, rows, I, stream);
}

extern "C" int pie_hip_gelu_tanh_and_mul(const pie_bf16* gate_up, int64_t in_row_stride,
                                         pie_bf16* out, int64_t out_row_stride, int64_t rows,
                                         int64_t I, void* stream) {
  return act_and_mul<kGeluTanh>(gate_up, in_row_stride, out, out_row_stride, rows, I, stream);
}
