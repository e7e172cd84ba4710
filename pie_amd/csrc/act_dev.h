// Device-side gated activations (SiLU / GELU-tanh and mul), shared by the standalone kernels
// (act.hip) and the grouped decode launch (group.hip).
#pragma once

#include "common.h"

namespace pie {
namespace {

enum { kSilu = 0, kGeluTanh = 1 };

// GELU with the tanh approximation (torch.nn.functional.gelu(x, approximate="tanh"), used by
// gemma2.py:224-226 / gemma3.py:246-248): 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))),
// tanh(u) = 1 - 2 / (1 + e^{2u}) with the hardware exp2 and reciprocal; rounded to bf16 like
// torch's bf16 gelu output before the multiply.
__device__ __forceinline__ float gelu_tanh_bf(float x) {
  const float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
  const float e = __builtin_amdgcn_exp2f(2.0f * 1.44269504088896341f * u);
  const float th = 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + e);
  return round_bf(0.5f * x * (1.0f + th));
}

__device__ __forceinline__ float silu_bf(float g) {
  // exp(-g) via the hardware base-2 exponential; 1/(1+e) via the hardware reciprocal.
  const float e = __builtin_amdgcn_exp2f(-g * 1.44269504088896341f);
  return round_bf(g * __builtin_amdgcn_rcpf(1.0f + e));
}

struct SiluArgs {
  const uint16_t* in;
  uint16_t* out;
  int64_t in_rs, out_rs, rows, I;
  uint32_t nvec;   // rows * I / 8 (vector path)
  FastDiv vpr;     // I / 8 vectors per row
};

// Flattened over all 16-byte output vectors: block b owns vectors [b*256*U, (b+1)*256*U), thread
// t handles b*256*U + t + 256*i for i < U, so every wave instruction covers 1 KiB contiguous
// (rows split only at row ends) and small row counts still spread over the whole chip.
template <int U, int ACT>
__device__ __forceinline__ void act_and_mul_block(const SiluArgs& a, uint32_t bid) {
  const uint32_t base = bid * (256u * U) + threadIdx.x;
  uint4 gv[U], uv[U];
  int64_t orow[U];
#pragma unroll
  for (int i = 0; i < U; ++i) {
    const uint32_t v = base + 256u * i;
    if (v < a.nvec) {
      const uint32_t row = a.vpr.div(v), c = v - row * a.vpr.d;
      const uint16_t* g = a.in + (int64_t)row * a.in_rs + (int64_t)c * 8;
      gv[i] = ld_nt(g);
      uv[i] = ld_nt(g + a.I);
      orow[i] = (int64_t)row * a.out_rs + (int64_t)c * 8;
    }
  }
#pragma unroll
  for (int i = 0; i < U; ++i) {
    if (base + 256u * i < a.nvec) {
      float gf[8], uf[8];
      unpack8(gv[i], gf);
      unpack8(uv[i], uf);
#pragma unroll
      for (int e = 0; e < 8; ++e) gf[e] = (ACT == kSilu ? silu_bf(gf[e]) : gelu_tanh_bf(gf[e])) * uf[e];
      st_nt(a.out + orow[i], pack8(gf));
    }
  }
}

}  // namespace
}  // namespace pie
