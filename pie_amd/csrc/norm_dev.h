// Device-side RMSNorm arithmetic (standard and Gemma rules), shared by the standalone norm
// kernels (norm.hip) and the grouped decode launch (group.hip), so both round identically.
#pragma once

#include <type_traits>

#include "common.h"

namespace pie {
namespace {

// Normalisation rules. Standard: torch's rms_norm (one rounding at the end):
//   y = bf16((x * rsqrt(mean(x^2) + eps)) * w)
// Gemma (pie/src/pie_worker/model/gemma2.py:514-526, gemma3.py:491-510): the expression
//   variance = x.pow(2).mean(-1); x * rsqrt(variance + eps) * (1.0 + weight)
// evaluated as separate bf16 torch ops, i.e. rounded to bf16 after every step.
// Gemma sums its bf16-rounded squares in fp64: each term has an 8-bit significand, so the sum
// is exact in any order (unless the squares span more than ~2^44) and the bf16 variance is the
// correctly rounded mean, independent of the reduction tree. The mean and the rsqrt are formed
// in fp32 and rounded to bf16, then checked against the two neighbouring bf16 midpoints with fp64
// products that are exact (a 9-bit midpoint times a 17-bit column count, or a 9-bit midpoint
// squared times an 8-bit t), and moved one bf16 step when they fall on the wrong side: an fp32
// result a few ulp off can only misround by one bf16 step. Both are then correctly rounded.
template <bool GEMMA>
using acc_t = std::conditional_t<GEMMA, double, float>;
template <bool GEMMA>
__device__ __forceinline__ float nsq(float x) { return GEMMA ? round_bf(x * x) : x * x; }
// ss += sum of the 8 squares. Gemma: a pairwise tree (exact, so the order is free and the
// dependent chain is short); standard: sequential fp32 adds.
template <bool GEMMA>
__device__ __forceinline__ void accum8(acc_t<GEMMA>& ss, const float* f) {
  if constexpr (GEMMA) {
    double p[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) p[e] = (double)nsq<true>(f[2 * e]) + (double)nsq<true>(f[2 * e + 1]);
    ss += (p[0] + p[1]) + (p[2] + p[3]);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += nsq<false>(f[e]);
  }
}
// bf16 neighbours of a non-negative bf16 value held as fp32 (NaN below zero: compares false).
__device__ __forceinline__ float bf_step(float b, int d) {
  return __builtin_bit_cast(float, __builtin_bit_cast(unsigned, b) + (unsigned)(d * 0x10000));
}
__device__ __forceinline__ bool bf_odd(float b) { return (__builtin_bit_cast(unsigned, b) >> 16) & 1u; }
// Correctly rounded bf16(tot / cols) for tot >= 0 (exact fp64), ties to even.
__device__ __forceinline__ float gemma_mean(double tot, int cols) {
  float b = round_bf((float)tot / (float)cols);
  const float dn = bf_step(b, -1), up = bf_step(b, 1);
  const double lo = 0.5 * ((double)dn + (double)b) * cols, hi = 0.5 * ((double)b + (double)up) * cols;
  if (tot < lo || (tot == lo && bf_odd(b))) b = dn;
  else if (tot > hi || (tot == hi && bf_odd(b))) b = up;
  return b;
}
// Correctly rounded bf16(1 / sqrt(t)) for a bf16 value t >= 0 (never exactly on a midpoint).
__device__ __forceinline__ float gemma_rsqrt(float t) {
  float b = round_bf(rsqrtf(t));
  const double ml = 0.5 * ((double)bf_step(b, -1) + (double)b), mh = 0.5 * ((double)b + (double)bf_step(b, 1));
  if (ml * ml * (double)t > 1.0) b = bf_step(b, -1);
  else if (mh * mh * (double)t < 1.0) b = bf_step(b, 1);
  return b;
}
template <bool GEMMA>
__device__ __forceinline__ float nscale(acc_t<GEMMA> tot, float cols, float eps) {
  if constexpr (GEMMA) return gemma_rsqrt(round_bf(gemma_mean(tot, (int)cols) + eps));
  return rsqrtf(tot / cols + eps);
}
// Weights enter napply already passed through wprep: Gemma's bf16(1 + w) is formed once, where
// the weights are loaded, not per element.
template <bool GEMMA>
__device__ __forceinline__ float wprep(float w) { return GEMMA ? round_bf(1.0f + w) : w; }
template <bool GEMMA>
__device__ __forceinline__ uint4 wprep8(uint4 v) {
  if constexpr (!GEMMA) return v;
  float f[8];
  unpack8(v, f);
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = wprep<true>(f[e]);
  return pack8(f);  // exact: every value is already a bf16
}
template <bool GEMMA>
__device__ __forceinline__ float napply(float x, float r, float wp) {
  if constexpr (GEMMA) return round_bf(x * r) * wp;
  return (x * r) * wp;
}

}  // namespace
}  // namespace pie
