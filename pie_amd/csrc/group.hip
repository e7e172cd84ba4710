// Grouped launch: independent per-layer ops of one decode step in ONE kernel launch.
//
// A decode step at batch sizes of a few hundred tokens is latency-bound: each op moves a few MB,
// so launch gaps and each kernel's ramp-up and drain dominate. Between pie_hip_group_begin and
// pie_hip_group_end the groupable entry points (pie_hip_embedding, pie_hip_fused_add_rmsnorm,
// pie_hip_silu_and_mul, pie_hip_gelu_tanh_and_mul, pie_hip_qk_rmsnorm_rope_append) only validate
// and record their arguments; the group's end launches one kernel whose block ranges run the
// recorded ops side by side:
//   [ q/k prologue: one token per block | add + RMSNorm: one row per block | act: 2 KiB per block ]
// The longest dependent-load chain (position -> page table -> cache row) starts first.
// One producer/consumer pair is allowed: an embedding whose output is the x input of an
// add + RMSNorm in the same group (the decode chain's embedding gather feeding the residual
// add, qwen3.py:468-472 -> :571 -> :538) runs fused: the gathered table row goes straight
// into registers and is also stored to the embedding's output. Any other overlap between one
// op's output and another op's operands is rejected.
//
// Results are bit-identical to the standalone kernels: the same per-element arithmetic and, for
// the norm, the same order of partial sums (64-vector wave partials added in order).
#include <string.h>

#include <new>

#include "act_dev.h"
#include "norm_dev.h"
#include "rope_dev.h"

namespace pie {
namespace {

// Residual add + RMSNorm of one row per 256-thread block, the row's x optionally gathered from
// an embedding table. cols = 512 * n512 with n512 in {1, 2, 4, 8}: thread t owns vectors
// t + 256 j (j < NJ); the 64 vectors of "virtual wave" g = 4 j + wave form one wave partial,
// exactly the partials of rmsnorm_rows_reg with one vector per lane.
struct GatherNormArgs {
  const int32_t* ids;      // nullptr: x rows are read from x
  const uint16_t* table;   // embedding table [V, table_rs]
  int64_t V, table_rs;
  const uint16_t* x;
  int64_t x_rs;
  const uint16_t* r;
  int64_t r_rs;
  uint16_t* s;
  int64_t s_rs;
  uint16_t* y;
  int64_t y_rs;
  uint16_t* x_out;  // gathered rows (the embedding's output), or nullptr
  int64_t xo_rs;
  const uint16_t* w;
  int32_t cols, n512;
  float eps;
};

template <int NJ>
__device__ __forceinline__ void gather_add_norm_block(const GatherNormArgs& a, int row) {
  __shared__ float part[8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nvec = a.cols >> 3;
  uint4 rv[NJ], xv[NJ], wv[NJ];
  // the residual row does not wait for the id: request it first
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int v = threadIdx.x + 256 * j;
    if (v < nvec) rv[j] = ld16(a.r + (int64_t)row * a.r_rs + (int64_t)v * 8);
  }
  const uint16_t* xrow = a.x + (int64_t)row * a.x_rs;
  bool zero = false;
  if (a.ids) {
    const int id = a.ids[row];  // block-uniform
    zero = id < 0 || (int64_t)id >= a.V;
    xrow = a.table + (int64_t)(zero ? 0 : id) * a.table_rs;
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int v = threadIdx.x + 256 * j;
    if (v < nvec) {
      xv[j] = zero ? make_uint4(0, 0, 0, 0) : ld16(xrow + (int64_t)v * 8);
      wv[j] = ld16(a.w + (int64_t)v * 8);
    }
  }
  float ss[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int v = threadIdx.x + 256 * j;
    ss[j] = 0.f;
    if (v < nvec) {
      if (a.x_out) st16(a.x_out + (int64_t)row * a.xo_rs + (int64_t)v * 8, xv[j]);
      float xf[8], rf[8];
      unpack8(xv[j], xf);
      unpack8(rv[j], rf);
#pragma unroll
      for (int e = 0; e < 8; ++e) xf[e] = rf[e] + xf[e];
      xv[j] = pack8(xf);  // s rounded to bf16: the norm reads the rounded values
      st16(a.s + (int64_t)row * a.s_rs + (int64_t)v * 8, xv[j]);
      unpack8(xv[j], xf);
      accum8<false>(ss[j], xf);
    }
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const float p = wave_sum(ss[j]);
    const int g = 4 * j + wave;
    if (lane == 0 && g < a.n512) part[g] = p;
  }
  __syncthreads();
  float tot = 0.f;
  if (a.n512 == 1) {
    tot = part[0];
  } else {
    for (int g = 0; g < a.n512; ++g) tot += part[g];
  }
  const float rstd = nscale<false>(tot, (float)a.cols, a.eps);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int v = threadIdx.x + 256 * j;
    if (v < nvec) {
      float xf[8], wf[8];
      unpack8(xv[j], xf);
      unpack8(wv[j], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) xf[e] = napply<false>(xf[e], rstd, wf[e]);
      st16(a.y + (int64_t)row * a.y_rs + (int64_t)v * 8, pack8(xf));
    }
  }
}

struct GroupArgs {
  GatherNormArgs nm;
  SiluArgs act;
  int32_t qk_blocks, nm_blocks, act_blocks, act_gelu;
  QkNormArgs qk;  // last: its inverse-frequency array ends the block
};
constexpr int kGroupScalarBytes = (int)offsetof(GroupArgs, qk) + kQkScalarBytes;

template <int NJ, int AU>
__global__ __launch_bounds__(256) void decode_group_kernel(GroupArgs g) {
  prefetch_kernarg<kGroupScalarBytes>(g);
  int b = blockIdx.x;  // block-uniform dispatch: every branch below is taken by whole blocks
  if (b < g.qk_blocks) {
    qk_norm_rope_append_block(g.qk, b);
    return;
  }
  b -= g.qk_blocks;
  if (b < g.nm_blocks) {
    gather_add_norm_block<NJ>(g.nm, b);
    return;
  }
  b -= g.nm_blocks;
  if (g.act_gelu) act_and_mul_block<AU, kGeluTanh>(g.act, (uint32_t)b);
  else act_and_mul_block<AU, kSilu>(g.act, (uint32_t)b);
}

// 16-byte output vectors per thread in the activation's block range (2 and 4 measured slower).
constexpr int kActU = 1;

// ---------------------------------------------------------------- host: recording
enum { kOpEmbed = 0, kOpAddNorm = 1, kOpAct = 2, kOpQk = 3 };
constexpr int kMaxGroupOps = 8;

struct GroupOp {
  int kind;
  void* stream;
  EmbedRec e;
  AddNormRec n;
  ActRec a;
  QkRec q;
  float freq[kMaxPairs];  // the q/k op's inverse frequencies (the caller's array may be gone)
};

struct GroupState {
  bool open = false;
  int n = 0;
  GroupOp ops[kMaxGroupOps];
};

thread_local GroupState g_group;

int group_slot(GroupOp** op, int kind, void* stream) {
  if (g_group.n >= kMaxGroupOps)
    return set_error(PIE_HIP_EINVAL, "group: at most %d ops per group", kMaxGroupOps);
  GroupOp& o = g_group.ops[g_group.n++];
  o.kind = kind;
  o.stream = stream;
  *op = &o;
  return PIE_HIP_OK;
}

// ---------------------------------------------------------------- host: hazards
struct Span {
  uintptr_t lo, hi;
};
// Bytes spanned by a [n1, n2, n3] bf16 view with strides (s1, s2, 1); empty when any extent is 0.
Span span3(const void* p, int64_t n1, int64_t s1, int64_t n2, int64_t s2, int64_t n3, int64_t elem = 2) {
  if (!p || n1 <= 0 || n2 <= 0 || n3 <= 0) return Span{0, 0};
  const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
  return Span{lo, lo + (uintptr_t)(((n1 - 1) * s1 + (n2 - 1) * s2 + n3) * elem)};
}
Span span2(const void* p, int64_t rows, int64_t rs, int64_t cols, int64_t elem = 2) {
  return span3(p, rows, rs, 1, 0, cols, elem);
}
bool overlap(const Span& a, const Span& b) { return a.lo < b.hi && b.lo < a.hi && a.lo < a.hi && b.lo < b.hi; }

struct Spans {
  Span in[8], out[4];
  int nin = 0, nout = 0;
};

Spans op_spans(const GroupOp& o) {
  Spans s;
  switch (o.kind) {
    case kOpEmbed:
      s.in[s.nin++] = span2(o.e.ids, 1, 0, o.e.T, 4);
      s.in[s.nin++] = span2(o.e.W, o.e.V, o.e.w_rs, o.e.H);
      s.out[s.nout++] = span2(o.e.out, o.e.T, o.e.out_rs, o.e.H);
      break;
    case kOpAddNorm:
      s.in[s.nin++] = span2(o.n.x, o.n.rows, o.n.x_rs, o.n.cols);
      s.in[s.nin++] = span2(o.n.r, o.n.rows, o.n.r_rs, o.n.cols);
      s.in[s.nin++] = span2(o.n.w, 1, 0, o.n.cols);
      s.out[s.nout++] = span2(o.n.s, o.n.rows, o.n.s_rs, o.n.cols);
      s.out[s.nout++] = span2(o.n.y, o.n.rows, o.n.y_rs, o.n.cols);
      break;
    case kOpAct:
      s.in[s.nin++] = span2(o.a.in, o.a.rows, o.a.in_rs, 2 * o.a.I);
      s.out[s.nout++] = span2(o.a.out, o.a.rows, o.a.out_rs, o.a.I);
      break;
    default: {
      const QkRec& q = o.q;
      s.in[s.nin++] = span3(q.q, q.T, q.q_ts, q.Hq, q.q_hs, q.D);
      s.in[s.nin++] = span3(q.k, q.T, q.k_ts, q.Hkv, q.k_hs, q.D);
      s.in[s.nin++] = span3(q.v, q.T, q.v_ts, q.Hkv, q.v_hs, q.D);
      s.in[s.nin++] = span2(q.qw, 1, 0, q.D);
      s.in[s.nin++] = span2(q.kw, 1, 0, q.D);
      s.in[s.nin++] = span2(q.pos, 1, 0, q.T, 4);
      s.in[s.nin++] = span2(q.batch_indices, 1, 0, q.T, 4);
      s.in[s.nin++] = span2(q.positions, 1, 0, q.T, 4);
      s.out[s.nout++] = span3(q.q_out, q.T, q.qo_ts, q.Hq, q.qo_hs, q.D);
      s.out[s.nout++] = span3(q.k_out, q.T, q.ko_ts, q.Hkv, q.ko_hs, q.D);
      s.out[s.nout++] = span2(q.k_cache, q.num_pages, q.page_stride, q.page_stride);
      s.out[s.nout++] = span2(q.v_cache, q.num_pages, q.page_stride, q.page_stride);
      break;
    }
  }
  return s;
}

// Whether op j reads op i's output in the one allowed way: the fused embedding -> add + RMSNorm.
bool fused_pair(const GroupOp& e, const GroupOp& n) {
  return e.kind == kOpEmbed && n.kind == kOpAddNorm && n.n.x == e.e.out && n.n.x_rs == e.e.out_rs &&
         n.n.rows == e.e.T && n.n.cols == e.e.H;
}

int check_hazards(const GroupOp* ops, int n) {
  Spans sp[kMaxGroupOps];
  for (int i = 0; i < n; ++i) sp[i] = op_spans(ops[i]);
  for (int i = 0; i < n; ++i)
    for (int j = 0; j < n; ++j) {
      if (i == j) continue;
      const bool pair = fused_pair(ops[i], ops[j]);
      for (int a = 0; a < sp[i].nout; ++a) {
        for (int b = 0; b < sp[j].nout; ++b)
          if (overlap(sp[i].out[a], sp[j].out[b]))
            return set_error(PIE_HIP_EINVAL, "group: outputs of ops %d and %d overlap", i, j);
        for (int b = 0; b < sp[j].nin; ++b) {
          if (pair && b == 0) continue;  // the fused embedding output is the norm's x
          if (overlap(sp[i].out[a], sp[j].in[b]))
            return set_error(PIE_HIP_EINVAL,
                             "group: op %d writes memory op %d reads (only an embedding feeding an "
                             "add + RMSNorm's x may depend on another op)", i, j);
        }
      }
    }
  return PIE_HIP_OK;
}

// ---------------------------------------------------------------- host: launch
int launch_alone(const GroupOp& o) {
  switch (o.kind) {
    case kOpEmbed:
      return pie_hip_embedding(o.e.ids, o.e.T, o.e.W, o.e.V, o.e.H, o.e.w_rs, o.e.out, o.e.out_rs, o.stream);
    case kOpAddNorm:
      return pie_hip_fused_add_rmsnorm(o.n.x, o.n.x_rs, o.n.r, o.n.r_rs, o.n.s, o.n.s_rs, o.n.y, o.n.y_rs,
                                       o.n.w, o.n.rows, o.n.cols, o.n.eps, o.stream);
    case kOpAct:
      return (o.a.gelu ? pie_hip_gelu_tanh_and_mul : pie_hip_silu_and_mul)(
          o.a.in, o.a.in_rs, o.a.out, o.a.out_rs, o.a.rows, o.a.I, o.stream);
    default: {
      const QkRec& q = o.q;
      return pie_hip_qk_rmsnorm_rope_append(
          q.q, q.q_ts, q.q_hs, q.k, q.k_ts, q.k_hs, q.v, q.v_ts, q.v_hs, q.q_out, q.qo_ts, q.qo_hs,
          q.k_out, q.ko_ts, q.ko_hs, q.qw, q.kw, q.eps, q.pos, q.T, q.Hq, q.Hkv, q.D, o.freq,
          q.batch_indices, q.positions, q.kv_indices, q.kv_indptr, q.batch_size, q.k_cache,
          q.v_cache, q.num_pages, q.page_stride, q.slot_stride, q.head_stride, q.page_size, o.stream);
    }
  }
}

bool vec_rows(const void* p, int64_t rs) { return aligned16(p) && rs % 8 == 0; }

bool norm_fits(const AddNormRec& n) {
  const int64_t n512 = n.cols / 512;
  return n.cols % 512 == 0 && (n512 == 1 || n512 == 2 || n512 == 4 || n512 == 8) &&
         n.rows < (1ll << 31) && vec_rows(n.x, n.x_rs) && vec_rows(n.r, n.r_rs) &&
         vec_rows(n.s, n.s_rs) && vec_rows(n.y, n.y_rs) && aligned16(n.w);
}
bool embed_fits(const EmbedRec& e) {
  return e.H % 8 == 0 && (e.V == 0 || vec_rows(e.W, e.w_rs)) && vec_rows(e.out, e.out_rs);
}
bool act_fits(const ActRec& a) {
  return a.I % 8 == 0 && vec_rows(a.in, a.in_rs) && vec_rows(a.out, a.out_rs) &&
         a.rows * (a.I / 8) < (1ll << 31);
}

}  // namespace

bool group_is_open() { return g_group.open; }

int group_add_embedding(const EmbedRec& r, void* stream) {
  GroupOp* o;
  const int rc = group_slot(&o, kOpEmbed, stream);
  if (rc) return rc;
  o->e = r;
  return PIE_HIP_OK;
}
int group_add_add_norm(const AddNormRec& r, void* stream) {
  GroupOp* o;
  const int rc = group_slot(&o, kOpAddNorm, stream);
  if (rc) return rc;
  o->n = r;
  return PIE_HIP_OK;
}
int group_add_act(const ActRec& r, void* stream) {
  GroupOp* o;
  const int rc = group_slot(&o, kOpAct, stream);
  if (rc) return rc;
  o->a = r;
  return PIE_HIP_OK;
}
int group_add_qk(const QkRec& r, void* stream) {
  GroupOp* o;
  const int rc = group_slot(&o, kOpQk, stream);
  if (rc) return rc;
  o->q = r;
  memcpy(o->freq, r.inv_freq, sizeof(float) * (size_t)(r.D / 2));
  o->q.inv_freq = o->freq;
  return PIE_HIP_OK;
}

}  // namespace pie

using namespace pie;

extern "C" int pie_hip_group_begin(void) {
  PIE_REQUIRE(!g_group.open, "group_begin: a group is already open on this thread");
  g_group.open = true;
  g_group.n = 0;
  return PIE_HIP_OK;
}

// What a group launches: the grouped kernel (blocks > 0) and the ops that run standalone, in
// record order after it.
struct GroupLaunch {
  GroupArgs g{};
  int nj = 1;
  int64_t blocks = 0;
  int n_alone = 0;
  GroupOp alone[kMaxGroupOps];
};

static void keep_alone(GroupLaunch& L, const GroupOp& o) {
  GroupOp& c = L.alone[L.n_alone++];
  c = o;
  c.q.inv_freq = c.freq;  // the copy's own inverse frequencies
}

// Closes the open group and works out its launches (nothing is launched).
static int group_build(void* stream, GroupLaunch& L, const char* what) {
  PIE_REQUIRE(g_group.open, "%s: no group is open on this thread", what);
  // Close first: the standalone launches must not be recorded again.
  g_group.open = false;
  const int n = g_group.n;
  g_group.n = 0;
  GroupOp* ops = g_group.ops;
  for (int i = 0; i < n; ++i)
    PIE_REQUIRE(ops[i].stream == stream, "%s: op %d was recorded on another stream", what, i);
  int rc = check_hazards(ops, n);
  if (rc) return rc;

  // the fused embedding -> add + RMSNorm pair, if any
  int pe = -1, pn = -1;
  for (int i = 0; i < n && pe < 0; ++i)
    for (int j = 0; j < n; ++j)
      if (fused_pair(ops[i], ops[j])) { pe = i; pn = j; break; }

  // one op per block range: the first that fits it
  int iq = -1, in = -1, ia = -1;
  QkNormArgs qa{};
  for (int i = 0; i < n; ++i) {
    const GroupOp& o = ops[i];
    if (o.kind == kOpQk && iq < 0) {
      bool vec = false;
      if (qk_prepare(o.q, qa, vec) == PIE_HIP_OK && vec && o.q.T < (1ll << 31)) iq = i;
    } else if (o.kind == kOpAddNorm && in < 0 && norm_fits(o.n) && (i != pn || embed_fits(ops[pe].e))) {
      in = i;
    } else if (o.kind == kOpAct && ia < 0 && act_fits(o.a)) {
      ia = i;
    }
  }
  const bool pair_fused = pn >= 0 && in == pn;
  const int pieces = (iq >= 0) + (in >= 0) + (ia >= 0);
  if ((pn >= 0 && !pair_fused) || (pieces < 2 && !pair_fused)) {
    // nothing to gain, or the producer/consumer pair cannot run fused: record order
    for (int i = 0; i < n; ++i) keep_alone(L, ops[i]);
    return PIE_HIP_OK;
  }

  GroupArgs& g = L.g;
  int& nj = L.nj;
  if (iq >= 0) {
    g.qk = qa;
    g.qk.r.wpt = 4;  // one token per 256-thread block
    g.qk_blocks = (int32_t)ops[iq].q.T;
  }
  if (in >= 0) {
    const AddNormRec& r = ops[in].n;
    GatherNormArgs& m = g.nm;
    m.x = r.x;
    m.x_rs = r.x_rs;
    if (pair_fused) {
      const EmbedRec& e = ops[pe].e;
      m.ids = e.ids;
      m.table = e.W;
      m.V = e.V;
      m.table_rs = e.w_rs;
      m.x_out = e.out;
      m.xo_rs = e.out_rs;
    }
    m.r = r.r;
    m.r_rs = r.r_rs;
    m.s = r.s;
    m.s_rs = r.s_rs;
    m.y = r.y;
    m.y_rs = r.y_rs;
    m.w = r.w;
    m.cols = (int32_t)r.cols;
    m.n512 = (int32_t)(r.cols / 512);
    m.eps = r.eps;
    g.nm_blocks = (int32_t)r.rows;
    nj = m.n512 == 8 ? 2 : 1;
  }
  if (ia >= 0) {
    const ActRec& r = ops[ia].a;
    const int64_t nvec = r.rows * (r.I / 8);
    g.act = SiluArgs{r.in, r.out, r.in_rs, r.out_rs, r.rows, r.I, (uint32_t)nvec,
                     FastDiv::make((uint32_t)(r.I / 8))};
    g.act_blocks = (int32_t)((nvec + 256 * kActU - 1) / (256 * kActU));
    g.act_gelu = r.gelu;
  }
  L.blocks = (int64_t)g.qk_blocks + g.nm_blocks + g.act_blocks;
  PIE_REQUIRE(L.blocks < (1ll << 31), "%s: %lld blocks", what, (long long)L.blocks);
  for (int i = 0; i < n; ++i) {
    if (i == iq || i == in || i == ia || (pair_fused && i == pe)) continue;
    keep_alone(L, ops[i]);
  }
  return PIE_HIP_OK;
}

static int group_launch(const GroupLaunch& L, void* stream, const char* what) {
  int rc;
  if (L.blocks > 0) {
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (L.nj == 2)
      hipLaunchKernelGGL((decode_group_kernel<2, kActU>), dim3((unsigned)L.blocks), dim3(256), 0, st, L.g);
    else
      hipLaunchKernelGGL((decode_group_kernel<1, kActU>), dim3((unsigned)L.blocks), dim3(256), 0, st, L.g);
    if ((rc = check_launch(what))) return rc;
  }
  for (int i = 0; i < L.n_alone; ++i) {
    GroupOp o = L.alone[i];
    o.q.inv_freq = o.freq;
    o.stream = stream;
    if ((rc = launch_alone(o))) return rc;
  }
  return PIE_HIP_OK;
}


extern "C" int pie_hip_group_end(void* stream) {
  GroupLaunch L;
  int rc = group_build(stream, L, "group_end");
  return rc ? rc : group_launch(L, stream, "group_end");
}

extern "C" int pie_hip_group_save(void* stream, void** group) {
  PIE_REQUIRE(group, "group_save: null handle pointer");
  *group = nullptr;
  GroupLaunch* L = new (std::nothrow) GroupLaunch();
  if (!L) {
    g_group.open = false;
    g_group.n = 0;
    return set_error(PIE_HIP_EINVAL, "group_save: out of host memory");
  }
  const int rc = group_build(stream, *L, "group_save");
  if (rc) {
    delete L;
    return rc;
  }
  *group = L;
  return PIE_HIP_OK;
}

extern "C" int pie_hip_group_launch(const void* group, void* stream) {
  PIE_REQUIRE(group, "group_launch: null group");
  return group_launch(*static_cast<const GroupLaunch*>(group), stream, "group_launch");
}

extern "C" void pie_hip_group_free(void* group) { delete static_cast<GroupLaunch*>(group); }
