// RMSNorm family for gfx950: plain rows, residual-add + RMSNorm, per-head q/k RMSNorm.
//
// Semantics follow torch's rms_norm decomposition (torch/_decomp/decompositions.py:1760-1810),
// which is what fun.rms_norm computes at pie/src/pie_worker/model/llama3.py:555/:618 and
// qwen3.py:651-662:   y = bf16( (f32(x) * rsqrt(mean(f32(x)^2) + eps)) * f32(w) ).
// The residual add is torch's bf16 `residual + x`: s = bf16(f32(r) + f32(x)), and the norm is
// taken of the rounded s (llama3.py:586 feeding the next layer's :555).
//
// Mapping. Rows of cols = NV*512 elements are held entirely in registers by ONE wavefront:
// lane l owns the 16-byte vectors l, l+64, ..., so every load/store instruction of a wave
// covers 1 KiB of contiguous row. The sum of squares is reduced with DPP row rotations and
// four readlanes (no LDS, no barrier). The weight row is loaded once per wave and reused for
// every row the wave visits. Per-head rows (D = 64/128/256) use 16-lane groups instead, four
// rows per wave instruction. Any other shape takes a generic two-pass path (one wave per row).
#include <stdlib.h>

#include "norm_dev.h"

namespace pie {
namespace {

// A set of rows addressed as (token, head): offset = t*tok_stride + h*head_stride.
struct RowSet {
  const uint16_t* in;
  const uint16_t* res;  // residual input (fused add only)
  uint16_t* sum;        // residual output s (fused add only)
  uint16_t* out;
  const uint16_t* w;
  int64_t in_ts, in_hs, res_ts, res_hs, sum_ts, sum_hs, out_ts, out_hs;
  int64_t heads;  // rows = T * heads
  int64_t rows;
};

struct NormArgs {
  RowSet set[2];  // q and k for the per-head norm; set[1].rows == 0 otherwise
  int64_t cols;
  float eps;
};

__device__ __forceinline__ void row_offsets(const RowSet& s, int64_t r, int64_t& oi, int64_t& orr,
                                            int64_t& os, int64_t& oo) {
  int64_t t = r, h = 0;
  if (s.heads != 1) {
    if (r < 0x7fffffff && s.heads < 0x7fffffff) {
      t = (uint32_t)r / (uint32_t)s.heads;
    } else {
      t = r / s.heads;
    }
    h = r - t * s.heads;
  }
  oi = t * s.in_ts + h * s.in_hs;
  orr = t * s.res_ts + h * s.res_hs;
  os = t * s.sum_ts + h * s.sum_hs;
  oo = t * s.out_ts + h * s.out_hs;
}

// Rows per wave group in flight at once. 1 measured best on configuration 2 (steady state:
// 2 rows equal, 4 rows 6% slower: the extra registers cost more occupancy than they gain).
constexpr int kRowsPerGroup = 1;

// ---------------------------------------------------------------- W waves per row, VPL*512*W cols
// A row is held in registers by a group of W wavefronts (VPL 16-byte vectors per lane); lane l
// of wave g in the group owns vectors j*64*W + g*64 + l. W = 1 for long row lists (no barrier);
// W > 1 spreads short lists (decode batches) over the chip, combining the W partial sums of
// squares through LDS in a fixed order. The weight row stays in registers across rows.
template <int VPL, int RPG, bool ADD, bool GEMMA, bool NT>
__global__ __launch_bounds__(512) void rmsnorm_rows_reg(NormArgs a, int W) {
  prefetch_kernarg<(int)sizeof(NormArgs)>(a);
  __shared__ acc_t<GEMMA> part[RPG][8];
  const RowSet& s = a.set[0];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = wave / W, gsub = wave - grp * W;
  const int G = blockDim.x / (64 * W);  // row groups per block
  const int64_t stride = (int64_t)gridDim.x * G * RPG;
  const int vstep = 64 * W;
  const int v0 = gsub * 64 + lane;

  uint4 wv[VPL];  // loaded after each row's inputs are in flight (a hit in L2 after the first row)

  // A group handles RPG rows at once (rows base+grp, base+grp+G, ...): all their loads are in
  // flight before the first reduction. Block-uniform trip count: every thread reaches every
  // barrier.
  for (int64_t base = (int64_t)blockIdx.x * G * RPG; base < s.rows; base += stride) {
    int64_t oo[RPG];
    bool live[RPG];
    uint4 xv[RPG][VPL];
    acc_t<GEMMA> ss[RPG];
#pragma unroll
    for (int k = 0; k < RPG; ++k) {
      const int64_t r = base + grp + (int64_t)k * G;
      live[k] = r < s.rows;
      int64_t oi = 0, orr = 0, os = 0;
      oo[k] = 0;
      if (live[k]) row_offsets(s, r, oi, orr, os, oo[k]);
      ss[k] = 0;
      if (live[k]) {
        // both input streams in flight before either is used
        uint4 rv[VPL];
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
          xv[k][j] = row_ld<NT>(s.in + oi, v0 + j * vstep);
          if constexpr (ADD) rv[j] = row_ld<NT>(s.res + orr, v0 + j * vstep);
        }
#pragma unroll
        for (int j = 0; j < VPL; ++j) wv[j] = ld16(s.w + (int64_t)(v0 + j * vstep) * 8);
        __builtin_amdgcn_sched_barrier(0);  // keep the scheduler from pulling uses between the loads
        if constexpr (ADD) {
#pragma unroll
          for (int j = 0; j < VPL; ++j) {
            float xf[8], rf[8];
            unpack8(xv[k][j], xf);
            unpack8(rv[j], rf);
#pragma unroll
            for (int e = 0; e < 8; ++e) xf[e] = rf[e] + xf[e];
            xv[k][j] = pack8(xf);  // s rounded to bf16: the norm below reads the rounded values
            row_st<NT>(s.sum + os, v0 + j * vstep, xv[k][j]);
          }
        }
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
          float xf[8];
          unpack8(xv[k][j], xf);
          accum8<GEMMA>(ss[k], xf);
        }
      }
    }
    acc_t<GEMMA> tot[RPG];
#pragma unroll
    for (int k = 0; k < RPG; ++k) tot[k] = wave_sum(ss[k]);
    if (W > 1) {
      if (lane == 0) {
#pragma unroll
        for (int k = 0; k < RPG; ++k) part[k][wave] = tot[k];
      }
      __syncthreads();
#pragma unroll
      for (int k = 0; k < RPG; ++k) {
        tot[k] = 0;
        for (int q = 0; q < W; ++q) tot[k] += part[k][grp * W + q];
      }
      __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < RPG; ++k) {
      if (!live[k]) continue;
      const float rstd = nscale<GEMMA>(tot[k], (float)a.cols, a.eps);
#pragma unroll
      for (int j = 0; j < VPL; ++j) {
        float xf[8], wf[8];
        unpack8(xv[k][j], xf);
        unpack8(wprep8<GEMMA>(wv[j]), wf);
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[e] = napply<GEMMA>(xf[e], rstd, wf[e]);
        row_st<NT>(s.out + oo[k], v0 + j * vstep, pack8(xf));
      }
    }
  }
}

// ---------------------------------------------------------------- one row per 512-thread block
// Large residual-add row lists of 4096*VPL columns: a block of 8 waves takes one row (thread t owns vectors
// t + 512 j), with no loop over rows, so each block issues its loads at once and the grid is
// one row per block; non-temporal loads and stores. Same vector ownership and the same fixed
// order of the 8 wave partial sums as rmsnorm_rows_reg with W = 8, so results are identical.
// (Configuration 2 in one harness: 44.3 us for this shape against 48 us for the row-loop kernel.)
template <int VPL, bool ADD, bool GEMMA>
__global__ __launch_bounds__(512) void rmsnorm_row_block(NormArgs a) {
  prefetch_kernarg<(int)sizeof(NormArgs)>(a);
  __shared__ acc_t<GEMMA> part[8];
  const RowSet& s = a.set[0];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int64_t oi, orr, os, oo;
  row_offsets(s, blockIdx.x, oi, orr, os, oo);
  uint4 xv[VPL], rv[VPL], wv[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int64_t v = (int64_t)(threadIdx.x + 512 * j) * 8;
    xv[j] = ld_nt(s.in + oi + v);
    if constexpr (ADD) rv[j] = ld_nt(s.res + orr + v);
  }
#pragma unroll
  for (int j = 0; j < VPL; ++j) wv[j] = ld16(s.w + (int64_t)(threadIdx.x + 512 * j) * 8);
  acc_t<GEMMA> ss = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    float xf[8];
    unpack8(xv[j], xf);
    if constexpr (ADD) {
      float rf[8];
      unpack8(rv[j], rf);
#pragma unroll
      for (int e = 0; e < 8; ++e) xf[e] = rf[e] + xf[e];
      xv[j] = pack8(xf);  // s rounded to bf16: the norm below reads the rounded values
      row_st<true>(s.sum + os, threadIdx.x + 512 * j, xv[j]);
      unpack8(xv[j], xf);
    }
    accum8<GEMMA>(ss, xf);
  }
  const acc_t<GEMMA> wsum = wave_sum(ss);
  if (lane == 0) part[wave] = wsum;
  __syncthreads();
  acc_t<GEMMA> tot = 0;
#pragma unroll
  for (int q = 0; q < 8; ++q) tot += part[q];
  const float rstd = nscale<GEMMA>(tot, (float)a.cols, a.eps);
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    float xf[8], wf[8];
    unpack8(xv[j], xf);
    unpack8(wprep8<GEMMA>(wv[j]), wf);
#pragma unroll
    for (int e = 0; e < 8; ++e) xf[e] = napply<GEMMA>(xf[e], rstd, wf[e]);
    row_st<true>(s.out + oo, threadIdx.x + 512 * j, pack8(xf));
  }
}

// ---------------------------------------------------------------- one wave per row, rows prefetched
// Plain (no residual) norms of large row lists: each wave walks rows wave, wave + waves, ...
// holding a row in registers (VPL vectors per lane: lane l owns vectors l + 64 j) and issuing the
// next row's loads before it reduces and writes the current one, so the arithmetic of one row
// (Gemma's fp64 sum and roundings) overlaps the next row's loads. Two register buffers alternate
// (a copy between them would wait for the loads in flight). No LDS, no barrier.
template <int VPL, bool GEMMA>
__global__ __launch_bounds__(256) void rmsnorm_rows_pf(NormArgs a) {
  prefetch_kernarg<(int)sizeof(NormArgs)>(a);
  const RowSet& s = a.set[0];
  const int lane = threadIdx.x & 63;
  const int64_t nw = (int64_t)gridDim.x * 4;
  int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  uint4 wv[VPL];
#pragma unroll
  for (int j = 0; j < VPL; ++j) wv[j] = wprep8<GEMMA>(ld16(s.w + (int64_t)(lane + 64 * j) * 8));
  auto load = [&](uint4 (&x)[VPL], int64_t row) {
    int64_t oi, orr, os, oo;
    row_offsets(s, row, oi, orr, os, oo);
#pragma unroll
    for (int j = 0; j < VPL; ++j) x[j] = row_ld<true>(s.in + oi, lane + 64 * j);
  };
  auto finish = [&](const uint4 (&x)[VPL], int64_t row) {
    acc_t<GEMMA> ss = 0;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      float xf[8];
      unpack8(x[j], xf);
      accum8<GEMMA>(ss, xf);
    }
    const float rstd = nscale<GEMMA>(wave_sum(ss), (float)a.cols, a.eps);
    int64_t oi, orr, os, oo;
    row_offsets(s, row, oi, orr, os, oo);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      float xf[8], wf[8];
      unpack8(x[j], xf);
      unpack8(wv[j], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) xf[e] = napply<GEMMA>(xf[e], rstd, wf[e]);
      row_st<true>(s.out + oo, lane + 64 * j, pack8(xf));
    }
  };
  uint4 xa[VPL], xb[VPL];
  if (r < s.rows) load(xa, r);
  while (r < s.rows) {
    const int64_t r1 = r + nw;
    if (r1 < s.rows) load(xb, r1);
    finish(xa, r);
    if (r1 >= s.rows) break;
    const int64_t r2 = r1 + nw;
    if (r2 < s.rows) load(xa, r2);
    finish(xb, r1);
    r = r2;
  }
}

// ---------------------------------------------------------------- 16 lanes per row (D = 16*EPL)
// EPL elements per lane: 4 (D=64, 8-byte accesses), 8 (D=128), 16 (D=256, two vectors).
template <int EPL>
struct Chunk;
template <>
struct Chunk<4> {
  uint2 v;
  __device__ void load(const uint16_t* p) { v = *reinterpret_cast<const uint2*>(p); }
  __device__ void store(uint16_t* p) const { *reinterpret_cast<uint2*>(p) = v; }
  __device__ void get(float* f) const { f[0] = bf_lo(v.x); f[1] = bf_hi(v.x); f[2] = bf_lo(v.y); f[3] = bf_hi(v.y); }
  __device__ void set(const float* f) { v.x = pack_bf2(f[0], f[1]); v.y = pack_bf2(f[2], f[3]); }
};
template <>
struct Chunk<8> {
  uint4 v;
  __device__ void load(const uint16_t* p) { v = ld16(p); }
  __device__ void store(uint16_t* p) const { st16(p, v); }
  __device__ void get(float* f) const { unpack8(v, f); }
  __device__ void set(const float* f) { v = pack8(f); }
};
template <>
struct Chunk<16> {
  uint4 v0, v1;
  __device__ void load(const uint16_t* p) { v0 = ld16(p); v1 = ld16(p + 8); }
  __device__ void store(uint16_t* p) const { st16(p, v0); st16(p + 8, v1); }
  __device__ void get(float* f) const { unpack8(v0, f); unpack8(v1, f + 8); }
  __device__ void set(const float* f) { v0 = pack8(f); v1 = pack8(f + 8); }
};

template <int EPL, bool GEMMA>
__global__ __launch_bounds__(256) void rmsnorm_heads16(NormArgs a) {
  prefetch_kernarg<(int)sizeof(NormArgs)>(a);
  const int64_t g = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 4;  // 16-lane group
  const int sub = threadIdx.x & 15;
  const int64_t total = a.set[0].rows + a.set[1].rows;
  // Every lane of a wave must reach the DPP reduction: rows past the end compute on zeros.
  const bool live = g < total;
  const int which = (live && g >= a.set[0].rows) ? 1 : 0;
  const RowSet& s = a.set[which];
  const int64_t r = which ? g - a.set[0].rows : g;
  int64_t oi = 0, orr, os, oo = 0;
  if (live) row_offsets(s, r, oi, orr, os, oo);

  Chunk<EPL> c, wc;
  float f[EPL], wf[EPL];
  if (live) {
    c.load(s.in + oi + sub * EPL);
    wc.load(s.w + sub * EPL);
    c.get(f);
    wc.get(wf);
#pragma unroll
    for (int e = 0; e < EPL; ++e) wf[e] = wprep<GEMMA>(wf[e]);
  } else {
#pragma unroll
    for (int e = 0; e < EPL; ++e) f[e] = wf[e] = 0.f;
  }
  acc_t<GEMMA> ss = 0;
#pragma unroll
  for (int e = 0; e < EPL; ++e) ss += nsq<GEMMA>(f[e]);
  const float rstd = nscale<GEMMA>(row16_sum(ss), (float)a.cols, a.eps);
#pragma unroll
  for (int e = 0; e < EPL; ++e) f[e] = napply<GEMMA>(f[e], rstd, wf[e]);
  if (live) {
    c.set(f);
    c.store(s.out + oo + sub * EPL);
  }
}

// ---------------------------------------------------------------- generic: one wave per row
// VEC = 8: 16-byte accesses (cols % 8 == 0, all rows 16-byte aligned); VEC = 1: scalar.
// Pass 1 reads the row (and writes s), pass 2 re-reads it from cache and writes y.
template <int VEC, bool ADD, bool GEMMA>
__global__ __launch_bounds__(256) void rmsnorm_rows_generic(NormArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * (blockDim.x >> 6);
  const int64_t total = a.set[0].rows + a.set[1].rows;
  const int64_t nv = a.cols / VEC;
  for (int64_t g = wave0; g < total; g += nwaves) {
    const int which = g >= a.set[0].rows ? 1 : 0;
    const RowSet& s = a.set[which];
    const int64_t r = which ? g - a.set[0].rows : g;
    int64_t oi, orr, os, oo;
    row_offsets(s, r, oi, orr, os, oo);
    const uint16_t* src = ADD ? s.sum + os : s.in + oi;
    acc_t<GEMMA> ss = 0;
    for (int64_t j = lane; j < nv; j += 64) {
      float f[VEC];
      if constexpr (VEC == 8) {
        uint4 xv = ld16(s.in + oi + j * 8);
        unpack8(xv, f);
        if constexpr (ADD) {
          float rf[8];
          unpack8(ld16(s.res + orr + j * 8), rf);
#pragma unroll
          for (int e = 0; e < 8; ++e) f[e] = rf[e] + f[e];
          xv = pack8(f);
          unpack8(xv, f);
          st16(s.sum + os + j * 8, xv);
        }
      } else {
        f[0] = bf1(s.in[oi + j]);
        if constexpr (ADD) {
          const uint16_t sv = to_bf1(bf1(s.res[orr + j]) + f[0]);
          s.sum[os + j] = sv;
          f[0] = bf1(sv);
        }
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) ss += nsq<GEMMA>(f[e]);
    }
    const float rstd = nscale<GEMMA>(wave_sum(ss), (float)a.cols, a.eps);
    for (int64_t j = lane; j < nv; j += 64) {
      if constexpr (VEC == 8) {
        float f[8], wf[8];
        unpack8(ld16(src + j * 8), f);
        unpack8(wprep8<GEMMA>(ld16(s.w + j * 8)), wf);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = napply<GEMMA>(f[e], rstd, wf[e]);
        st16(s.out + oo + j * 8, pack8(f));
      } else {
        s.out[oo + j] = to_bf1(napply<GEMMA>(bf1(src[j]), rstd, wprep<GEMMA>(bf1(s.w[j]))));
      }
    }
  }
}

// ---------------------------------------------------------------- host side
int64_t wave_grid(int64_t rows) {
  // 4 waves per 256-thread block; cap the grid so waves loop over rows (weights stay in
  // registers) once the device is full many times over.
  const int64_t blocks = (rows + 3) / 4;
  const int64_t cap = (int64_t)num_cus() * 32;
  return blocks < cap ? blocks : cap;
}

bool rowset_vec_ok(const RowSet& s, bool add) {
  bool ok = aligned16(s.in) && aligned16(s.out) && aligned16(s.w) &&
            s.in_ts % 8 == 0 && s.in_hs % 8 == 0 && s.out_ts % 8 == 0 && s.out_hs % 8 == 0;
  if (add)
    ok = ok && aligned16(s.res) && aligned16(s.sum) && s.res_ts % 8 == 0 &&
         s.res_hs % 8 == 0 && s.sum_ts % 8 == 0 && s.sum_hs % 8 == 0;
  return ok;
}

// Large row lists (past 64 MB) take the non-temporal one-row-per-block kernel: on configuration
// 2 it measured 44.1 us per op against 47.8 us for the cached row-loop kernel.
template <bool ADD, bool GEMMA>
int launch_rows(const NormArgs& a, hipStream_t st, const char* name) {
  const int64_t rows = a.set[0].rows + a.set[1].rows;
  if (rows == 0) return PIE_HIP_OK;
  const bool vec = a.cols % 8 == 0 && rowset_vec_ok(a.set[0], ADD) &&
                   (a.set[1].rows == 0 || rowset_vec_ok(a.set[1], ADD));
  const dim3 blk(256);
  const int64_t in_bytes = rows * a.cols * 2;
  const bool large = in_bytes >= (int64_t)64 << 20;  // far larger than L2
  // (the residual-add form only: a plain norm, one input stream, keeps too few bytes in flight at
  // one vector per lane and stays on the row-loop kernel with 4 vectors per lane)
  if (ADD && vec && large && a.set[1].rows == 0 && a.cols % 4096 == 0 &&
      a.cols <= 3 * 4096 && rows < 0x7fffffff) {
    const dim3 grd((unsigned)rows), tb(512);
    switch (a.cols / 4096) {
      case 1: hipLaunchKernelGGL((rmsnorm_row_block<1, ADD, GEMMA>), grd, tb, 0, st, a); break;
      case 2: hipLaunchKernelGGL((rmsnorm_row_block<2, ADD, GEMMA>), grd, tb, 0, st, a); break;
      default: hipLaunchKernelGGL((rmsnorm_row_block<3, ADD, GEMMA>), grd, tb, 0, st, a); break;
    }
    return check_launch(name);
  }
  // Gemma's plain norm of large row lists: the row-prefetching kernel, 2 work groups per CU
  // ([8192, 4096]: 25.2 us against 26.6-28.5 for rows_reg; 1 per CU 26.4, 3 per CU 26.1; two
  // rows ahead 26.9). The standard plain norm measured the same either way (24.0-24.1 us) and
  // stays on rows_reg.
  const int pf_blocks = GEMMA ? 2 : 0;
  if (!ADD && vec && large && pf_blocks > 0 && a.set[1].rows == 0 && a.cols % 512 == 0 &&
      a.cols <= 8 * 512) {
    int64_t blocks = (int64_t)num_cus() * pf_blocks;
    const int64_t need = (rows + 3) / 4;
    if (blocks > need) blocks = need;
    const dim3 grd((unsigned)blocks), tb(256);
    switch (a.cols / 512) {
#define PIE_PF(n) case n: hipLaunchKernelGGL((rmsnorm_rows_pf<n, GEMMA>), grd, tb, 0, st, a); break;
      PIE_PF(1) PIE_PF(2) PIE_PF(3) PIE_PF(4) PIE_PF(5) PIE_PF(6) PIE_PF(7) default: PIE_PF(8)
#undef PIE_PF
    }
    return check_launch(name);
  }
  if (vec && a.set[1].rows == 0 && a.cols % 512 == 0 && a.cols <= 8 * 12 * 512) {
    const int64_t n512 = a.cols / 512;
    // Waves per row W (each lane then holds VPL = cols / (512 W) 16-byte vectors). Residual add:
    // as many waves as divide the row, up to 8 (two input streams already keep 2 KiB per wave in
    // flight; configuration 2: 8 waves 46.0 us, 1 wave 50.4 us). Plain norm: at least 4 vectors
    // per lane, since one stream at one vector per lane leaves too few bytes in flight per CU
    // ([8192, 4096]: 8 waves 31.6 us, 4 waves 26.6, 2 waves 26.0).
    int W = 0;
    for (int w = 8; w >= 1; w /= 2)
      if (n512 % w == 0 && n512 / w <= 12 && (ADD || n512 / w >= 4 || w == 1)) { W = w; break; }
    if (W > 0) {
      const int threads = W == 8 ? 512 : 256;
      const int64_t G = threads / (64 * W);
      int64_t blocks = (rows + G * kRowsPerGroup - 1) / (G * kRowsPerGroup);
      const int64_t cap = (int64_t)num_cus() * 64;
      if (blocks > cap) blocks = cap;
      const dim3 grd((unsigned)blocks), tb(threads);
      // Row lists far larger than L2 stream through non-temporal loads and stores (configuration
      // 2, 8 waves per row, steady state: x / r / s / y at 5.6 TB/s cached, 6.7 TB/s
      // non-temporal in a standalone model of this kernel); small lists (decode) keep their
      // outputs in L2 for the next kernel.
      // Non-temporal from 8 MB of input on (configuration 1, [2048, 2048] = 8 MiB, steady state:
      // 4.72 us against 6.05 us cached; W = 1 and 2 the same, W = 4 5.58 us; a plain copy of
      // the same bytes takes 3.79 us non-temporal, 4.42 cached). Decode-sized lists keep their
      // outputs in L2 for the next kernel.
      const bool nt = in_bytes >= (int64_t)8 << 20;
      switch ((n512 / W) * 2 + (nt ? 1 : 0)) {
#define PIE_NV(n)                                                                                      \
  case 2 * n: hipLaunchKernelGGL((rmsnorm_rows_reg<n, kRowsPerGroup, ADD, GEMMA, false>), grd, tb, 0, st, a, W); \
    break;                                                                                              \
  case 2 * n + 1: hipLaunchKernelGGL((rmsnorm_rows_reg<n, kRowsPerGroup, ADD, GEMMA, true>), grd, tb, 0, st, a, W); \
    break;
        PIE_NV(1) PIE_NV(2) PIE_NV(3) PIE_NV(4) PIE_NV(5) PIE_NV(6) PIE_NV(7) PIE_NV(8)
        PIE_NV(9) PIE_NV(10) PIE_NV(11) PIE_NV(12)
#undef PIE_NV
      }
      return check_launch(name);
    }
  }
  if (!ADD && vec && (a.cols == 64 || a.cols == 128 || a.cols == 256)) {
    const int64_t threads = rows * 16;
    const dim3 grd((unsigned)((threads + 255) / 256));
    if (a.cols == 64) hipLaunchKernelGGL((rmsnorm_heads16<4, GEMMA>), grd, blk, 0, st, a);
    else if (a.cols == 128) hipLaunchKernelGGL((rmsnorm_heads16<8, GEMMA>), grd, blk, 0, st, a);
    else hipLaunchKernelGGL((rmsnorm_heads16<16, GEMMA>), grd, blk, 0, st, a);
    return check_launch(name);
  }
  const dim3 grd((unsigned)wave_grid(rows));
  if (vec) hipLaunchKernelGGL((rmsnorm_rows_generic<8, ADD, GEMMA>), grd, blk, 0, st, a);
  else hipLaunchKernelGGL((rmsnorm_rows_generic<1, ADD, GEMMA>), grd, blk, 0, st, a);
  return check_launch(name);
}

}  // namespace
}  // namespace pie

using namespace pie;

namespace {
template <bool GEMMA>
int rmsnorm_impl(const pie_bf16* x, int64_t x_row_stride, const pie_bf16* w, pie_bf16* y,
                 int64_t y_row_stride, int64_t rows, int64_t cols, float eps, void* stream) {
  PIE_REQUIRE(rows >= 0 && cols > 0, "rmsnorm: bad shape rows=%lld cols=%lld", (long long)rows, (long long)cols);
  if (rows == 0) return PIE_HIP_OK;
  PIE_REQUIRE(x && w && y, "rmsnorm: null pointer");
  PIE_REQUIRE(x_row_stride >= cols && y_row_stride >= cols, "rmsnorm: row stride smaller than cols");
  NormArgs a{};
  a.set[0] = RowSet{x, nullptr, nullptr, y, w, x_row_stride, 0, 0, 0, 0, 0, y_row_stride, 0, 1, rows};
  a.cols = cols;
  a.eps = eps;
  return launch_rows<false, GEMMA>(a, (hipStream_t)stream, GEMMA ? "gemma_rmsnorm" : "rmsnorm");
}

template <bool GEMMA>
int add_rmsnorm_impl(const pie_bf16* x, int64_t x_row_stride, const pie_bf16* r,
                     int64_t r_row_stride, pie_bf16* s, int64_t s_row_stride, pie_bf16* y,
                     int64_t y_row_stride, const pie_bf16* w, int64_t rows, int64_t cols, float eps,
                     void* stream) {
  PIE_REQUIRE(rows >= 0 && cols > 0, "fused_add_rmsnorm: bad shape rows=%lld cols=%lld", (long long)rows, (long long)cols);
  if (rows == 0) return PIE_HIP_OK;
  PIE_REQUIRE(x && r && s && y && w, "fused_add_rmsnorm: null pointer");
  PIE_REQUIRE(x_row_stride >= cols && r_row_stride >= cols && s_row_stride >= cols && y_row_stride >= cols,
              "fused_add_rmsnorm: row stride smaller than cols");
  if (!GEMMA && group_is_open())
    return group_add_add_norm(AddNormRec{x, x_row_stride, r, r_row_stride, s, s_row_stride, y, y_row_stride,
                                         w, rows, cols, eps}, stream);
  NormArgs a{};
  a.set[0] = RowSet{x, r, s, y, w, x_row_stride, 0, r_row_stride, 0, s_row_stride, 0, y_row_stride, 0, 1, rows};
  a.cols = cols;
  a.eps = eps;
  return launch_rows<true, GEMMA>(a, (hipStream_t)stream, GEMMA ? "gemma_fused_add_rmsnorm" : "fused_add_rmsnorm");
}

template <bool GEMMA>
int qk_rmsnorm_impl(const pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride, pie_bf16* q_out,
                    int64_t qo_tok_stride, int64_t qo_head_stride, const pie_bf16* k,
                    int64_t k_tok_stride, int64_t k_head_stride, pie_bf16* k_out,
                    int64_t ko_tok_stride, int64_t ko_head_stride, const pie_bf16* qw,
                    const pie_bf16* kw, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, float eps,
                    void* stream) {
  PIE_REQUIRE(T >= 0 && Hq >= 0 && Hkv >= 0 && D > 0, "qk_rmsnorm: bad shape");
  if (T == 0 || Hq + Hkv == 0) return PIE_HIP_OK;
  PIE_REQUIRE(Hq == 0 || (q && q_out && qw), "qk_rmsnorm: null q pointer");
  PIE_REQUIRE(Hkv == 0 || (k && k_out && kw), "qk_rmsnorm: null k pointer");
  NormArgs a{};
  a.set[0] = RowSet{q, nullptr, nullptr, q_out, qw, q_tok_stride, q_head_stride, 0, 0, 0, 0,
                    qo_tok_stride, qo_head_stride, Hq ? Hq : 1, Hq ? T * Hq : 0};
  a.set[1] = RowSet{k, nullptr, nullptr, k_out, kw, k_tok_stride, k_head_stride, 0, 0, 0, 0,
                    ko_tok_stride, ko_head_stride, Hkv ? Hkv : 1, Hkv ? T * Hkv : 0};
  if (Hq == 0) { a.set[0] = a.set[1]; a.set[1] = RowSet{}; }
  a.cols = D;
  a.eps = eps;
  return launch_rows<false, GEMMA>(a, (hipStream_t)stream, GEMMA ? "gemma_qk_rmsnorm" : "qk_rmsnorm");
}
}  // namespace

#define PIE_NORM_ARGS x, x_row_stride, w, y, y_row_stride, rows, cols, eps, stream
extern "C" int pie_hip_rmsnorm(const pie_bf16* x, int64_t x_row_stride, const pie_bf16* w,
                               pie_bf16* y, int64_t y_row_stride, int64_t rows, int64_t cols,
                               float eps, void* stream) {
  return rmsnorm_impl<false>(PIE_NORM_ARGS);
}
extern "C" int pie_hip_gemma_rmsnorm(const pie_bf16* x, int64_t x_row_stride, const pie_bf16* w,
                                     pie_bf16* y, int64_t y_row_stride, int64_t rows, int64_t cols,
                                     float eps, void* stream) {
  return rmsnorm_impl<true>(PIE_NORM_ARGS);
}
#undef PIE_NORM_ARGS

#define PIE_ADD_ARGS x, x_row_stride, r, r_row_stride, s, s_row_stride, y, y_row_stride, w, rows, cols, eps, stream
extern "C" int pie_hip_fused_add_rmsnorm(const pie_bf16* x, int64_t x_row_stride,
                                         const pie_bf16* r, int64_t r_row_stride,
                                         pie_bf16* s, int64_t s_row_stride,
                                         pie_bf16* y, int64_t y_row_stride,
                                         const pie_bf16* w, int64_t rows, int64_t cols,
                                         float eps, void* stream) {
  return add_rmsnorm_impl<false>(PIE_ADD_ARGS);
}
extern "C" int pie_hip_gemma_fused_add_rmsnorm(const pie_bf16* x, int64_t x_row_stride,
                                               const pie_bf16* r, int64_t r_row_stride,
                                               pie_bf16* s, int64_t s_row_stride,
                                               pie_bf16* y, int64_t y_row_stride,
                                               const pie_bf16* w, int64_t rows, int64_t cols,
                                               float eps, void* stream) {
  return add_rmsnorm_impl<true>(PIE_ADD_ARGS);
}
#undef PIE_ADD_ARGS

#define PIE_QK_ARGS q, q_tok_stride, q_head_stride, q_out, qo_tok_stride, qo_head_stride, k, \
    k_tok_stride, k_head_stride, k_out, ko_tok_stride, ko_head_stride, qw, kw, T, Hq, Hkv, D, eps, stream
extern "C" int pie_hip_qk_rmsnorm(const pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride,
                                  pie_bf16* q_out, int64_t qo_tok_stride, int64_t qo_head_stride,
                                  const pie_bf16* k, int64_t k_tok_stride, int64_t k_head_stride,
                                  pie_bf16* k_out, int64_t ko_tok_stride, int64_t ko_head_stride,
                                  const pie_bf16* qw, const pie_bf16* kw, int64_t T, int64_t Hq,
                                  int64_t Hkv, int64_t D, float eps, void* stream) {
  return qk_rmsnorm_impl<false>(PIE_QK_ARGS);
}
extern "C" int pie_hip_gemma_qk_rmsnorm(const pie_bf16* q, int64_t q_tok_stride, int64_t q_head_stride,
                                        pie_bf16* q_out, int64_t qo_tok_stride, int64_t qo_head_stride,
                                        const pie_bf16* k, int64_t k_tok_stride, int64_t k_head_stride,
                                        pie_bf16* k_out, int64_t ko_tok_stride, int64_t ko_head_stride,
                                        const pie_bf16* qw, const pie_bf16* kw, int64_t T, int64_t Hq,
                                        int64_t Hkv, int64_t D, float eps, void* stream) {
  return qk_rmsnorm_impl<true>(PIE_QK_ARGS);
}
#undef PIE_QK_ARGS
