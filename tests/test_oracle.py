"""Pins the CPU oracle (oracle/oracle.c) to independent sources of truth. CPU only.

a1/a2/a3 RMSNorm, a2 residual add, a4 SiLU-and-mul, a5 embedding: the reference runs these as
torch ops (pie/src/pie_worker/model/llama3.py:555, :586, :569-572, :471), so torch-CPU running
the very same expressions is the reference implementation; it is compared here.
a6/a7 RoPE: flashinfer is absent (an external wheel, no network), so the frequency rule is
pinned to transformers' Llama-3 rope parameters and the rotation to HF's rotate-half form in
float64, plus closed-form invariants. a8 append and a9 index helpers: brute-force Python loops
restating pie/src/flashinfer_metal/ops.py:392-436 and metal_append_paged_kv_cache.metal:51-103.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from pie_amd import workloads as wl
from tests._util import assert_bf16_close, assert_bits_equal, ulp_diff

N, T_ = oracle.to_np, oracle.to_torch


# ----------------------------------------------------------------------------- bf16 rounding
def test_bf16_rounding_matches_torch():
    g = torch.Generator().manual_seed(0)
    x = torch.cat([torch.randn(100000, generator=g) * 10 ** torch.randint(-30, 30, (100000,), generator=g),
                   torch.tensor([0.0, -0.0, float("inf"), -float("inf"), 1e-40, 3.4e38, 65504.0])])
    want = x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert_bits_equal(oracle.f32_to_bf16(x.numpy()), want, "vectorised f32->bf16")
    lib = oracle._load()
    got = np.array([lib.oracle_f32_to_bf16(float(v)) for v in x.numpy()[:2000]], dtype=np.uint16)
    assert_bits_equal(got, want[:2000], "C f32->bf16")


def test_f64_to_bf16_single_rounding():
    lib = oracle._load()
    # 1 + 2^-8 is a bf16 tie; a hair above must round up even though fp32 would land on the tie
    assert lib.oracle_f64_to_bf16(1.0 + 2.0 ** -8 + 2.0 ** -40) == 0x3F81
    assert lib.oracle_f64_to_bf16(1.0 + 2.0 ** -8 - 2.0 ** -40) == 0x3F80
    assert lib.oracle_f64_to_bf16(1.0 + 2.0 ** -8) == 0x3F80  # exact tie: to even


# ----------------------------------------------------------------------------- RMSNorm
@pytest.mark.parametrize("T,H,eps", [(64, 2048, 1e-5), (17, 4096, 1e-6), (5, 896, 1e-6), (9, 100, 1e-5)])
def test_rmsnorm_vs_torch(T, H, eps):
    x, w = wl.normal((T, H), 1), wl.normal((H,), 2, 1.0, 0.1)
    want = F.rms_norm(x, [H], w, eps)
    got = oracle.rmsnorm(N(x), N(w), eps)
    assert ulp_diff(got, N(want)).max() <= 1
    assert_bf16_close(got, N(want), what="rmsnorm")


def test_rmsnorm_invariants():
    H = 512
    x = wl.normal((8, H), 3)
    w = wl.normal((H,), 4, 1.0, 0.1)
    y = oracle.bf16_to_f32(oracle.rmsnorm(N(x), N(w), 1e-6))
    # scale invariance: y(4x) == y(x) when eps << mean square (4 is exact in bf16)
    y4 = oracle.bf16_to_f32(oracle.rmsnorm(N(x * 4), N(w), 1e-6))
    np.testing.assert_allclose(y4, y, rtol=1e-2, atol=1e-2)
    # constant row c -> w * sign(c)
    c = torch.full((1, H), -3.0).to(torch.bfloat16)
    yc = oracle.bf16_to_f32(oracle.rmsnorm(N(c), N(w), 1e-6))
    np.testing.assert_allclose(yc[0], -oracle.bf16_to_f32(N(w)), rtol=1e-2)
    # zero row -> zeros
    z = torch.zeros((1, H), dtype=torch.bfloat16)
    assert (oracle.bf16_to_f32(oracle.rmsnorm(N(z), N(w), 1e-6)) == 0).all()
    # rows are independent
    y_first = oracle.rmsnorm(N(x[:1]), N(w), 1e-6)
    assert_bits_equal(y_first, oracle.rmsnorm(N(x), N(w), 1e-6)[:1])
    # mean of squares of the normalised row (w = 1) is 1
    ones = torch.ones(H, dtype=torch.bfloat16)
    yn = oracle.bf16_to_f32(oracle.rmsnorm(N(x), N(ones), 0.0)).astype(np.float64)
    np.testing.assert_allclose((yn ** 2).mean(-1), 1.0, rtol=1e-2)


def test_per_head_rmsnorm_vs_torch():
    c = wl.cfg5(B=16, V=64)
    q, k, _ = wl.split_qkv(c["qkv"], 32, 8, 128)
    want_q = F.rms_norm(q, [128], c["q_norm"], 1e-6)
    got = oracle.rmsnorm(N(q), N(c["q_norm"]), 1e-6)
    assert ulp_diff(got, N(want_q)).max() <= 1
    want_k = F.rms_norm(k, [128], c["k_norm"], 1e-6)
    assert ulp_diff(oracle.rmsnorm(N(k), N(c["k_norm"]), 1e-6), N(want_k)).max() <= 1


def test_add_rmsnorm_vs_torch():
    c = wl.cfg2(T=48, H=4096, I=64)
    s_want = c["r"] + c["x"]
    y_want = F.rms_norm(s_want, [4096], c["w"], 1e-5)
    y, s = oracle.add_rmsnorm(N(c["x"]), N(c["r"]), N(c["w"]), 1e-5)
    assert_bits_equal(s, N(s_want), "residual sum (bit-exact)")
    assert ulp_diff(y, N(y_want)).max() <= 1


# ----------------------------------------------------------------------------- SiLU-and-mul
def test_silu_and_mul_vs_torch():
    c = wl.cfg2(T=32, H=8, I=1536)
    g, u = torch.split(c["gate_up"], [1536, 1536], -1)
    want = F.silu(g) * u
    got = oracle.silu_and_mul(N(c["gate_up"]), mode=0)
    assert ulp_diff(got, N(want)).max() <= 1
    assert (got == N(want)).mean() > 0.999
    # single-rounding form stays inside the stated tolerance of torch's double rounding
    assert_bf16_close(oracle.silu_and_mul(N(c["gate_up"]), mode=1), N(want), what="silu 1-round")


def test_silu_special_values():
    g = torch.tensor([0.0, 20.0, -20.0, 1.0], dtype=torch.bfloat16)
    u = torch.tensor([3.0, 2.0, 5.0, 1.0], dtype=torch.bfloat16)
    out = oracle.bf16_to_f32(oracle.silu_and_mul(N(torch.cat([g, u])[None])))[0]
    assert out[0] == 0.0
    assert out[1] == 40.0          # silu(g) == g for g >> 0
    assert abs(out[2]) < 1e-6      # silu(g) ~ 0 for g << 0
    assert abs(out[3] - 1.0 / (1.0 + math.exp(-1.0))) < 4e-3


# ----------------------------------------------------------------------------- embedding
def test_embedding_vs_torch():
    c = wl.cfg4(V=1000, H=64, T=300)
    got, bad = oracle.embedding(N(c["ids"]), N(c["W"]))
    assert bad == 0
    assert_bits_equal(got, N(F.embedding(c["ids"], c["W"])), "embedding")


def test_embedding_out_of_range_rows_are_zero():
    W = wl.normal((10, 16), 1)
    ids = torch.tensor([0, 10, -1, 9], dtype=torch.int32)
    got, bad = oracle.embedding(N(ids), N(W))
    assert bad == 2
    assert (got[1] == 0).all() and (got[2] == 0).all()
    assert_bits_equal(got[[0, 3]], N(W)[[0, 9]])


# ----------------------------------------------------------------------------- RoPE
def _hf_llama3_inv_freq(D, theta, factor, lo, hi, L):
    from transformers import LlamaConfig
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    cfg = LlamaConfig(hidden_size=D * 4, num_attention_heads=4, head_dim=D,
                      rope_parameters=dict(rope_type="llama3", rope_theta=theta, factor=factor,
                                           low_freq_factor=lo, high_freq_factor=hi,
                                           original_max_position_embeddings=L))
    f, _ = ROPE_INIT_FUNCTIONS["llama3"](cfg, "cpu")
    return f.double().numpy()


@pytest.mark.parametrize("theta,factor", [(5e5, 8.0), (5e5, 32.0), (1e4, 4.0)])
def test_llama31_inv_freq_vs_transformers(theta, factor):
    want = _hf_llama3_inv_freq(128, theta, factor, 1.0, 4.0, 8192)
    got = oracle.inv_freq_llama31(128, factor, theta, 1.0, 4.0, 8192)
    np.testing.assert_allclose(got, want, rtol=2e-6)  # transformers evaluates in fp32
    # all three bands occur for the Llama-3 constants
    base = oracle.inv_freq_std(128, 1.0, theta)
    assert (got == base).any() and np.isclose(got, base / factor).any()


def test_llama31_reduces_to_standard_when_unscaled():
    np.testing.assert_allclose(oracle.inv_freq_llama31(128, 1.0, 5e5, 1.0, 4.0, 8192),
                               oracle.inv_freq_std(128, 1.0, 5e5), rtol=1e-15)


def test_standard_inv_freq_closed_form():
    f = oracle.inv_freq_std(64, 2.0, 1e6)
    assert f[0] == 0.5
    np.testing.assert_allclose(f, 0.5 * 1e6 ** (-np.arange(0, 64, 2) / 64), rtol=1e-14)


def _hf_rotate_half(x, pos, inv_freq, interleave=False):
    """HF apply_rotary_pos_emb in float64 on [T,H,D] (rotate_half; interleaved via reshape)."""
    x = x.double()
    ang = pos.double()[:, None] * torch.from_numpy(inv_freq)[None, :]
    cos, sin = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]
    if interleave:
        x1, x2 = x[..., 0::2], x[..., 1::2]
        out = torch.empty_like(x)
        out[..., 0::2] = x1 * cos - x2 * sin
        out[..., 1::2] = x2 * cos + x1 * sin
        return out
    cos, sin = torch.cat([cos, cos], -1), torch.cat([sin, sin], -1)
    x1, x2 = x[..., : x.shape[-1] // 2], x[..., x.shape[-1] // 2:]
    return x * cos + torch.cat([-x2, x1], -1) * sin


@pytest.mark.parametrize("interleave", [False, True])
def test_rope_vs_hf_rotate_half(interleave):
    T, Hq, Hkv, D = 40, 4, 2, 128
    q, k = wl.normal((T, Hq, D), 1), wl.normal((T, Hkv, D), 2)
    pos = torch.randint(0, 8192, (T,), generator=torch.Generator().manual_seed(3)).to(torch.int32)
    f = oracle.inv_freq_llama31(D, 8.0, 5e5, 1.0, 4.0, 8192)
    gq, gk = oracle.rope(N(q), N(k), N(pos), f, interleave=interleave)
    wq = _hf_rotate_half(q, pos, f, interleave).float().to(torch.bfloat16)
    wk = _hf_rotate_half(k, pos, f, interleave).float().to(torch.bfloat16)
    assert ulp_diff(gq, N(wq)).max() <= 1
    assert ulp_diff(gk, N(wk)).max() <= 1


def test_rope_partial_rotary_dim_leaves_tail():
    T, H, D, rd = 6, 2, 128, 64
    q, k = wl.normal((T, H, D), 4), wl.normal((T, H, D), 5)
    pos = torch.arange(T, dtype=torch.int32) * 100
    f = oracle.inv_freq_std(rd, 1.0, 1e4)
    gq, _ = oracle.rope(N(q), N(k), N(pos), f, rotary_dim=rd)
    assert_bits_equal(gq[..., rd:], N(q)[..., rd:], "tail untouched")
    wq = _hf_rotate_half(q[..., :rd], pos, f).float().to(torch.bfloat16)
    assert ulp_diff(gq[..., :rd], N(wq)).max() <= 1


def test_rope_invariants():
    T, H, D = 16, 3, 128
    q, k = wl.normal((T, H, D), 6), wl.normal((T, H, D), 7)
    f = oracle.inv_freq_std(D, 1.0, 1e6)
    # pos = 0 is the identity, bit for bit
    z = np.zeros(T, np.int32)
    gq, gk = oracle.rope(N(q), N(k), z, f)
    assert_bits_equal(gq, N(q))
    # each rotated pair keeps its norm
    pos = np.arange(T, dtype=np.int32) * 37
    gq, _ = oracle.rope(N(q), N(k), pos, f)
    a, b = oracle.bf16_to_f32(N(q)).astype(np.float64), oracle.bf16_to_f32(gq).astype(np.float64)
    na = a[..., :64] ** 2 + a[..., 64:] ** 2
    nb = b[..., :64] ** 2 + b[..., 64:] ** 2
    np.testing.assert_allclose(nb, na, rtol=2e-2, atol=1e-2)
    # composition R(a) R(b) = R(a + b) in float64 (via the HF form, no bf16 in between)
    x = torch.randn(T, H, D, dtype=torch.float64, generator=torch.Generator().manual_seed(8))
    p1 = torch.arange(T, dtype=torch.int32) * 3
    p2 = torch.arange(T, dtype=torch.int32) * 5
    two = _hf_rotate_half(_hf_rotate_half(x, p1, f), p2, f)
    one = _hf_rotate_half(x, p1 + p2, f)
    torch.testing.assert_close(two, one, rtol=1e-9, atol=1e-9)


# ----------------------------------------------------------------------------- paged append
def _brute_append(k, v, bidx, pos, cache, kv_indices, kv_indptr, P):
    """Loop restatement of metal_append_paged_kv_cache.metal:51-103 (NHD)."""
    B = len(kv_indptr) - 1
    for t in range(k.shape[0]):
        b, p = int(bidx[t]), int(pos[t])
        if b < 0 or b >= B or p < 0:
            continue
        logical = int(kv_indptr[b]) + p // P
        if logical >= int(kv_indptr[b + 1]):
            continue
        page = int(kv_indices[logical])
        if page < 0 or page >= cache.shape[0]:
            continue
        cache[page, 0, p % P] = k[t]
        cache[page, 1, p % P] = v[t]


def test_append_vs_brute_force():
    pb = wl.paged_batch(torch.tensor([0, 5, 31, 16], dtype=torch.int32),
                        torch.tensor([3, 20, 1, 0], dtype=torch.int32), 16, 24, 1)
    T, Hkv, D = int(pb.lens.sum()), 2, 16
    k, v = N(wl.normal((T, Hkv, D), 1)), N(wl.normal((T, Hkv, D), 2))
    bidx, pos = N(pb.batch_indices), N(pb.positions)
    # poison: one token with an out-of-range batch index, one past its pages
    bidx[0] = 7
    pos[4] = 10_000
    c1 = N(wl.sentinel_cache((24, 2, 16, Hkv, D)))
    c2 = c1.copy()
    n = oracle.append(k, v, bidx, pos, c1, N(pb.kv_indices), N(pb.kv_indptr))
    _brute_append(k, v, bidx, pos, c2, N(pb.kv_indices), N(pb.kv_indptr), 16)
    assert n == T - 2
    assert_bits_equal(c1, c2, "append")
    assert (c1 == wl.SENTINEL_BITS).any()  # untouched pages keep the sentinel


def test_append_hnd_matches_nhd_transposed():
    pb = wl.paged_batch(torch.tensor([3, 0], dtype=torch.int32), torch.tensor([9, 17], dtype=torch.int32), 8, 10, 2)
    T, Hkv, D = int(pb.lens.sum()), 3, 8
    k, v = N(wl.normal((T, Hkv, D), 3)), N(wl.normal((T, Hkv, D), 4))
    nhd = N(wl.sentinel_cache((10, 2, 8, Hkv, D)))
    hnd = N(wl.sentinel_cache((10, 2, Hkv, 8, D)))
    args = (N(pb.batch_indices), N(pb.positions))
    oracle.append(k, v, *args, nhd, N(pb.kv_indices), N(pb.kv_indptr), "NHD")
    oracle.append(k, v, *args, hnd, N(pb.kv_indices), N(pb.kv_indptr), "HND")
    assert_bits_equal(hnd.transpose(0, 1, 3, 2, 4), nhd)


# ----------------------------------------------------------------------------- index helpers
def _brute_seq_lens(indptr, last, P):
    """flashinfer_metal/ops.py:392-407."""
    out = []
    for i in range(len(indptr) - 1):
        n = indptr[i + 1] - indptr[i]
        out.append((n - 1) * P + last[i] if n > 0 else 0)
    return np.array(out, np.int32)


def _brute_batch_pos(indptr, seq_lens, nnz):
    """flashinfer_metal/ops.py:410-436."""
    b = np.full(nnz, -1, np.int32)
    p = np.full(nnz, -1, np.int32)
    for i in range(len(indptr) - 1):
        s, e = indptr[i], indptr[i + 1]
        b[s:e] = i
        p[s:e] = np.arange(seq_lens[i] - (e - s), seq_lens[i])
    return b, p


def test_index_helpers_vs_brute_force():
    rng = np.random.default_rng(5)
    npages = rng.integers(0, 6, 40)
    npages[3] = 0
    indptr = np.concatenate([[0], np.cumsum(npages)]).astype(np.int32)
    last = rng.integers(1, 17, 40).astype(np.int32)
    assert_bits_equal(oracle.seq_lens(indptr, last, 16), _brute_seq_lens(indptr, last, 16))
    sl = oracle.seq_lens(indptr, last, 16)
    newtok = np.minimum(rng.integers(0, 5, 40), sl)
    qo = np.concatenate([[0], np.cumsum(newtok)]).astype(np.int32)
    nnz = int(qo[-1]) + 3  # padded tail stays untouched
    got_b, got_p = oracle.batch_indices_positions(qo, sl, nnz)
    want_b, want_p = _brute_batch_pos(qo, sl, nnz)
    assert_bits_equal(got_b, want_b)
    assert_bits_equal(got_p, want_p)
    assert (got_b[-3:] == -1).all()


def test_workload_positions_match_index_helpers():
    """The workload builder's positions equal what get_batch_indices_positions derives."""
    c = wl.cfg5(B=32, V=16)
    pb = c["batch"]
    sl = oracle.seq_lens(N(pb.kv_indptr), N(pb.kv_last_page_len), pb.page_size)
    assert_bits_equal(sl, N(pb.seq_lens))
    b, p = oracle.batch_indices_positions(N(pb.qo_indptr), sl, int(pb.qo_indptr[-1]))
    assert_bits_equal(b, N(pb.batch_indices))
    assert_bits_equal(p, N(pb.positions))


# ----------------------------------------------------------------------------- variant ops
def _gemma_torch(x, w, eps):
    """The reference's expression (gemma2.py:514-526), run by torch-CPU. One substitution:
    torch-CPU's bf16 rsqrt kernel is not correctly rounded (rsqrt(1.0234375) gives 0.9921875;
    the fp32 value 0.98848 rounds to 0.98828125), while torch's GPU elementwise kernels compute
    bf16 rsqrt in fp32 and round once, so the rsqrt is taken in fp32 and rounded here."""
    variance = x.pow(2).mean(-1, keepdim=True)
    x_normed = x * torch.rsqrt((variance + eps).float()).to(x.dtype)
    return x_normed * (1.0 + w)


def _assert_gemma_rows(got, x, w, eps, what):
    """Rows whose bf16 variance (exact sum, one rounding) equals torch's must match torch bit for
    bit; a row where torch's fp32 summation order rounds the variance one ulp the other way may
    differ by the propagated amount (<= 2.5e-2 relative) and must differ in variance by exactly
    one ulp."""
    want = N(_gemma_torch(x, w, eps))
    v_torch = N(x.pow(2).mean(-1, keepdim=True)).reshape(-1)
    sq = oracle.bf16_to_f32(oracle.f32_to_bf16(oracle.bf16_to_f32(N(x)) ** 2)).astype(np.float64)
    v_exact = oracle.f32_to_bf16((sq.sum(-1) / x.shape[-1]).astype(np.float32)).reshape(-1)
    g2, w2 = got.reshape(-1, x.shape[-1]), want.reshape(-1, x.shape[-1])
    same = v_exact == v_torch
    assert same.mean() > 0.8, f"{what}: variance agreement {same.mean()}"
    assert_bits_equal(g2[same], w2[same], f"{what} (rows with equal variance)")
    if (~same).any():
        assert ulp_diff(v_exact[~same], v_torch[~same]).max() == 1
        assert_bf16_close(g2[~same], w2[~same], rtol=2.5e-2, what=f"{what} (variance 1 ulp apart)")


@pytest.mark.parametrize("T,H", [(32, 3584), (16, 2304), (8, 256)])
def test_gemma_rmsnorm_vs_torch(T, H):
    x, w = wl.normal((T, H), 31), wl.normal((H,), 32, 0.0, 0.5)
    _assert_gemma_rows(oracle.gemma_rmsnorm(N(x), N(w), 1e-6), x, w, 1e-6, "gemma rmsnorm")
    # per-head form (gemma3 _qk_norm on [T, H, D])
    q = wl.normal((4, 8, 256), 33)
    wq = wl.normal((256,), 34, 0.0, 0.5)
    _assert_gemma_rows(oracle.gemma_rmsnorm(N(q), N(wq), 1e-6), q, wq, 1e-6, "gemma per-head")


def test_gemma_add_rmsnorm_vs_torch():
    x, r, w = wl.normal((8, 3584), 35), wl.normal((8, 3584), 36), wl.normal((3584,), 37, 0.0, 0.5)
    y, s = oracle.gemma_add_rmsnorm(N(x), N(r), N(w), 1e-6)
    assert_bits_equal(s, N(r + x), "residual")
    _assert_gemma_rows(y, r + x, w, 1e-6, "gemma add+norm")


def test_gemma_rmsnorm_differs_from_standard():
    """A dropped (1 + w) or a missing step rounding would make gemma equal standard*w."""
    x, w = wl.normal((4, 512), 38), wl.normal((512,), 39, 0.0, 0.5)
    g = oracle.bf16_to_f32(oracle.gemma_rmsnorm(N(x), N(w), 1e-6))
    s1 = oracle.bf16_to_f32(oracle.rmsnorm(N(x), N((1.0 + w.float()).to(torch.bfloat16)), 1e-6))
    np.testing.assert_allclose(g, s1, rtol=2e-2, atol=2e-2)  # same function up to roundings
    assert not np.array_equal(g, oracle.bf16_to_f32(oracle.rmsnorm(N(x), N(w), 1e-6)))


def test_gelu_tanh_and_mul_vs_torch():
    gu = wl.normal((32, 2 * 1536), 40, 0.0, 2 ** 0.5)
    g, u = torch.split(gu, [1536, 1536], -1)
    want = F.gelu(g, approximate="tanh") * u
    got = oracle.gelu_tanh_and_mul(N(gu))
    assert_bf16_close(got, N(want), what="gelu*up")
    # torch's fp32 1 + tanh(u) cancels for gate << 0 (values ~1e-6); elsewhere <= 1 ulp
    big = np.abs(oracle.bf16_to_f32(N(want))) > 1e-3
    assert ulp_diff(got, N(want))[big].max() <= 1
    assert (got == N(want)).mean() > 0.99


def test_gelu_special_values():
    g = torch.tensor([0.0, 10.0, -10.0], dtype=torch.bfloat16)
    u = torch.tensor([5.0, 2.0, 3.0], dtype=torch.bfloat16)
    out = oracle.bf16_to_f32(oracle.gelu_tanh_and_mul(N(torch.cat([g, u])[None])))[0]
    assert out[0] == 0.0 and out[1] == 20.0 and abs(out[2]) < 1e-6


def test_embedding_scaled_vs_torch():
    c = wl.cfg4(V=300, H=2304, T=64)
    scale = math.sqrt(2304)
    want = F.embedding(c["ids"], c["W"]) * scale
    got, bad = oracle.embedding_scaled(N(c["ids"]), N(c["W"]), scale)
    assert bad == 0
    assert_bits_equal(got, N(want), "scaled embedding")


def _yarnless_cache(rows, rd, theta):
    f = oracle.inv_freq_std(rd, 1.0, theta)
    ang = np.arange(rows, dtype=np.float64)[:, None] * f[None, :]
    return np.concatenate([np.cos(ang), np.sin(ang)], -1).astype(np.float32), f


@pytest.mark.parametrize("interleave", [False, True])
def test_rope_cos_sin_table_matches_frequency_rope(interleave):
    T, Hq, Hkv, D = 20, 4, 2, 64
    q, k = wl.normal((T, Hq, D), 41), wl.normal((T, Hkv, D), 42)
    pos = torch.randint(0, 500, (T,), generator=torch.Generator().manual_seed(43)).to(torch.int32)
    cs, f = _yarnless_cache(512, D, 1.5e5)
    gq, gk = oracle.rope_cos_sin(N(q), N(k), N(pos), cs, interleave)
    wq, wk = oracle.rope(N(q), N(k), N(pos), f, interleave=interleave)
    assert ulp_diff(gq, wq).max() <= 1 and ulp_diff(gk, wk).max() <= 1
    # partial rotary dim: dims past the table's width are untouched
    cs32, _ = _yarnless_cache(512, 32, 1.5e5)
    pq, _ = oracle.rope_cos_sin(N(q), N(k), N(pos), cs32, interleave)
    assert_bits_equal(pq[..., 32:], N(q)[..., 32:])
    # a position outside the table leaves the token unchanged
    pos2 = N(pos).copy()
    pos2[0] = 600
    oq, _ = oracle.rope_cos_sin(N(q), N(k), pos2, cs, interleave)
    assert_bits_equal(oq[0], N(q)[0])


# ----------------------------------------------------------------------------- paged attention
def _gather_kv(cache, pb, b, layout="NHD"):
    """Request b's k, v as float64 [kv_len, Hkv, D], read page by page (brute force)."""
    P = pb.page_size
    kv_len = int(pb.seq_lens[b])
    pages = pb.kv_indices[int(pb.kv_indptr[b]):int(pb.kv_indptr[b + 1])].tolist()
    c = cache.to(torch.float64)
    rows_k, rows_v = [], []
    for t in range(kv_len):
        pg, sl = pages[t // P], t % P
        if layout == "NHD":
            rows_k.append(c[pg, 0, sl]); rows_v.append(c[pg, 1, sl])
        else:
            rows_k.append(c[pg, 0, :, sl]); rows_v.append(c[pg, 1, :, sl])
    return torch.stack(rows_k), torch.stack(rows_v)


def _sdpa_reference(a, custom=None, window_left=-1):
    """torch-CPU scaled_dot_product_attention in float64, one request at a time, with the
    causal window written as an explicit boolean mask (or the custom mask)."""
    pb, q = a["batch"], a["q"].to(torch.float64)
    G = a["Hq"] // a["Hkv"]
    out = torch.zeros_like(q)
    moff = 0
    for b in range(pb.seq_lens.numel()):
        q0, q1 = int(pb.qo_indptr[b]), int(pb.qo_indptr[b + 1])
        kv_len, qo_len = int(pb.seq_lens[b]), q1 - q0
        if qo_len == 0 or kv_len == 0:
            continue
        k, v = _gather_kv(a["cache"], pb, b, a["layout"])
        if custom is None:
            m = torch.tensor([[t <= kv_len - qo_len + i for t in range(kv_len)] for i in range(qo_len)])
        else:
            m = torch.as_tensor(custom[moff:moff + qo_len * kv_len]).view(qo_len, kv_len).bool()
            moff += qo_len * kv_len
        if window_left >= 0:
            m = m & torch.tensor([[t >= kv_len - qo_len + i - window_left for t in range(kv_len)]
                                  for i in range(qo_len)])
        k = k.repeat_interleave(G, dim=1).transpose(0, 1)  # [Hq, kv, D]
        v = v.repeat_interleave(G, dim=1).transpose(0, 1)
        o = F.scaled_dot_product_attention(q[q0:q1].transpose(0, 1), k, v, attn_mask=m)
        o = torch.where(m.any(1)[None, :, None], o, torch.zeros_like(o))  # empty rows -> 0
        out[q0:q1] = o.transpose(0, 1)
    return out


def _oracle_attn(a, custom=None, **kw):
    pb = a["batch"]
    return oracle.attention(N(a["q"]), N(a["cache"]), N(pb.qo_indptr), N(pb.kv_indptr),
                            N(pb.kv_indices), N(pb.kv_last_page_len), custom_mask=custom,
                            layout=a["layout"], **kw)


@pytest.mark.parametrize("layout", ["NHD", "HND"])
def test_attention_vs_torch_sdpa(layout):
    # decode rows, a chunked prefill over cached context, a fresh prefill, an empty request
    a = wl.attn_batch([37, 0, 5, 60, 0], [1, 19, 12, 3, 0], Hq=8, Hkv=2, D=64, page_size=16,
                      seed=3, layout=layout)
    want = _sdpa_reference(a).to(torch.float32)
    got = oracle.bf16_to_f32(_oracle_attn(a))
    assert np.abs(got - want.numpy()).max() <= 2 ** -8 * np.abs(want.numpy()).max() + 1e-6


def test_attention_square_causal_is_torch_is_causal():
    # kv_len == qo_len: the window t <= i is torch's own is_causal definition
    a = wl.attn_batch([0], [23], Hq=4, Hkv=4, D=32, page_size=4, seed=5)
    k, v = _gather_kv(a["cache"], a["batch"], 0)
    q = a["q"].to(torch.float64).transpose(0, 1)
    want = F.scaled_dot_product_attention(q, k.transpose(0, 1), v.transpose(0, 1), is_causal=True)
    got = oracle.bf16_to_f32(_oracle_attn(a))
    np.testing.assert_allclose(got, want.transpose(0, 1).numpy(), rtol=2 ** -8, atol=1e-6)


def test_attention_custom_mask_vs_sdpa_and_causal():
    a = wl.attn_batch([9, 30], [7, 4], Hq=4, Hkv=2, D=32, page_size=8, seed=7)
    pb = a["batch"]
    g = torch.Generator().manual_seed(8)
    blocks, causal = [], []
    for b in range(2):
        qo, kv = int(pb.lens[b]), int(pb.seq_lens[b])
        blocks.append((torch.rand(qo, kv, generator=g) < 0.6).flatten())
        causal.append(torch.tensor([[t <= kv - qo + i for t in range(kv)] for i in range(qo)]).flatten())
    mask = torch.cat(blocks)
    mask[:5] = False  # row 0 of request 0 partly masked; fully-masked rows give 0
    want = _sdpa_reference(a, mask.numpy()).to(torch.float32)
    got = oracle.bf16_to_f32(_oracle_attn(a, mask.numpy()))
    np.testing.assert_allclose(got, want.numpy(), rtol=2 ** -8, atol=1e-6)
    # the causal window written as a custom mask is the default behaviour, bit for bit
    assert_bits_equal(_oracle_attn(a, torch.cat(causal).numpy()), _oracle_attn(a), "causal mask")


@pytest.mark.parametrize("window_left", [0, 5, 40])
def test_attention_sliding_window_vs_torch_sdpa(window_left):
    a = wl.attn_batch([37, 0, 5, 60], [1, 19, 12, 3], Hq=8, Hkv=2, D=64, page_size=16, seed=13)
    want = _sdpa_reference(a, window_left=window_left).to(torch.float32)
    got = oracle.bf16_to_f32(_oracle_attn(a, window_left=window_left))
    assert np.abs(got - want.numpy()).max() <= 2 ** -8 * np.abs(want.numpy()).max() + 1e-6
    if window_left == 0:  # each query sees only its own position: output = its v row, exactly
        pb = a["batch"]
        for b in range(4):
            _, v = _gather_kv(a["cache"], pb, b)
            q0, q1 = int(pb.qo_indptr[b]), int(pb.qo_indptr[b + 1])
            L = int(pb.seq_lens[b])
            for i in range(q1 - q0):
                row = v[L - (q1 - q0) + i].repeat_interleave(4, 0).float().numpy()
                assert (got[q0 + i] == row).all(), f"request {b} token {i}"


def test_attention_closed_forms():
    # one visible position: output is that v row exactly; lse is the scaled score
    a = wl.attn_batch([0], [1], Hq=2, Hkv=1, D=16, page_size=4, seed=9)
    out, lse = _oracle_attn(a, return_lse=True)
    k, v = _gather_kv(a["cache"], a["batch"], 0)
    assert_bits_equal(out[0], N(v[0].to(torch.bfloat16).repeat(2, 1)), "single position")
    s = (a["q"][0].to(torch.float64) * k[0]).sum(-1) / 4.0
    np.testing.assert_allclose(lse[0], s.numpy(), rtol=1e-12)
    # identical keys: uniform weights, output = mean of v, lse = s + log(n)
    a = wl.attn_batch([40], [1], Hq=1, Hkv=1, D=16, page_size=8, seed=10)
    pb = a["batch"]
    for pg in pb.kv_indices.tolist():
        a["cache"][pg, 0] = a["cache"][pb.kv_indices[0], 0, 0]
    out, lse = _oracle_attn(a, return_lse=True)
    k, v = _gather_kv(a["cache"], pb, 0)
    want = v[:, 0].mean(0)
    np.testing.assert_allclose(oracle.bf16_to_f32(out[0, 0]), want.numpy(), rtol=2 ** -8, atol=1e-7)
    s = float((a["q"][0, 0].to(torch.float64) * k[0, 0]).sum()) / 4.0
    assert abs(lse[0, 0] - (s + math.log(41))) < 1e-9


def test_attention_page_permutation_invariant():
    # moving pages (data and table entry together) does not change the result
    a = wl.attn_batch([50, 17], [3, 2], Hq=4, Hkv=2, D=32, page_size=4, seed=11)
    pb = a["batch"]
    base = _oracle_attn(a)
    perm = torch.randperm(a["cache"].shape[0], generator=torch.Generator().manual_seed(12))
    cache2 = torch.empty_like(a["cache"])
    cache2[perm] = a["cache"]
    a2 = dict(a, cache=cache2)
    pb.kv_indices = perm[pb.kv_indices.long()].to(torch.int32)
    assert_bits_equal(_oracle_attn(a2), base, "page permutation")


# ----------------------------------------------------------------------------- sampling path
def _hf_kept(scores: torch.Tensor, mode: str, k=None, p=None, m=None) -> torch.Tensor:
    """Kept sets from transformers' logits warpers (a local library routine): top-p keeps the
    smallest most-probable set reaching p, top-k the k best (ties at the k-th value stay), min-p
    tokens with prob >= m * max."""
    from transformers.generation.logits_process import (MinPLogitsWarper, TopKLogitsWarper,
                                                        TopPLogitsWarper)
    lg = torch.log(scores)
    if mode == "top_p":
        lg = TopPLogitsWarper(top_p=p)(None, lg)
    elif mode == "top_k":
        lg = TopKLogitsWarper(top_k=k)(None, lg)
    elif mode == "min_p":
        lg = MinPLogitsWarper(min_p=m)(None, lg)
    return torch.isfinite(lg)


@pytest.mark.parametrize("mode", ["top_p", "top_k", "min_p"])
def test_sample_kept_sets_vs_transformers_warpers(mode):
    g = torch.Generator().manual_seed(31)
    for trial in range(20):
        V = int(torch.randint(5, 300, (1,), generator=g))
        probs = torch.rand(1, V, generator=g, dtype=torch.float64) ** 3
        probs /= probs.sum()
        k = int(torch.randint(1, V + 3, (1,), generator=g))
        p = float(torch.rand(1, generator=g)) * 0.98 + 0.01
        m = float(torch.rand(1, generator=g)) * 0.9
        want = _hf_kept(probs, mode, k=k, p=p, m=m)[0].numpy()
        _, kept = oracle.sample(probs.float().numpy(), mode, [0.5], top_k=[k], top_p=[p], min_p=[m])
        assert (kept[0] == want).all(), f"{mode} trial {trial}: V={V} k={k} p={p} m={m}"


def test_sample_closed_forms():
    probs = np.array([[0.1, 0.4, 0.2, 0.3]], np.float32)
    # plain inverse CDF in index order: cumulative 0.1, 0.5, 0.7, 1.0
    for u, want in ((0.0, 0), (0.05, 0), (0.1, 1), (0.49, 1), (0.5, 2), (0.69, 2), (0.7, 3), (0.99, 3)):
        assert oracle.sample(probs, "plain", [u])[0][0] == want, u
    # top_k = 1 and tiny top_p are greedy; top_k >= V and top_p = 1 keep everything
    for u in (0.0, 0.3, 0.99):
        assert oracle.sample(probs, "top_k", [u], top_k=[1])[0][0] == 1
        assert oracle.sample(probs, "top_p", [u], top_p=[1e-6])[0][0] == 1
    assert oracle.sample(probs, "top_k", [0.5], top_k=[9])[1].all()
    assert oracle.sample(probs, "top_p", [0.5], top_p=[1.0])[1].all()
    # top_p 0.6: 0.4 (mass above 0 < 0.6) and 0.3 (above 0.4 < 0.6) stay, 0.2 (above 0.7) goes
    assert (oracle.sample(probs, "top_p", [0.5], top_p=[0.6])[1][0] == [False, True, False, True]).all()
    # min_p 0.6: threshold 0.24 keeps 0.4 and 0.3
    assert (oracle.sample(probs, "min_p", [0.5], min_p=[0.6])[1][0] == [False, True, False, True]).all()
    # top_k 3 then top_p 0.5 inside {0.4, 0.3, 0.2} (mass 0.9, threshold 0.45): 0.4 and 0.3 stay
    assert (oracle.sample(probs, "top_k_top_p", [0.5], top_k=[3], top_p=[0.5])[1][0]
            == [False, True, False, True]).all()
    # ties at the k-th value all stay
    tied = np.array([[0.3, 0.2, 0.2, 0.2, 0.1]], np.float32)
    assert (oracle.sample(tied, "top_k", [0.5], top_k=[2])[1][0] == [True, True, True, True, False]).all()


def test_scaled_softmax_vs_torch_reference():
    """Against Pie's own torch form (_safe_scaled_softmax_impl_torch, common.py:38-59) in fp64."""
    g = torch.Generator().manual_seed(32)
    x = torch.randn(4, 500, generator=g) * 4
    x[1, :300] = -float("inf")  # masked logits (padding, banned tokens): probability 0
    x[2, ::2] = -float("inf")
    x[0, :10] = -float("inf")
    temps = torch.tensor([0.0, 0.5, 1.0, 2.5])
    safe = torch.where(temps[:, None] < 1e-5, 1.0, temps[:, None].double())
    soft = torch.softmax(x.double() / safe, -1)
    greedy = F.one_hot(x.argmax(-1), 500).double()
    want = torch.where(temps[:, None] < 1e-5, greedy, soft)
    np.testing.assert_allclose(oracle.scaled_softmax(x.numpy(), temps.numpy()), want.numpy(),
                               rtol=1e-12, atol=1e-300)


def _sink_reference(a, sinks, window_left=-1):
    """The published gpt-oss form, in torch float64: the head's sink logit appended as one more
    score column, softmax over the row, the sink column dropped, then the product with v."""
    pb, q = a["batch"], a["q"].to(torch.float64)
    G, D = a["Hq"] // a["Hkv"], a["D"]
    out = torch.zeros_like(q)
    for b in range(pb.seq_lens.numel()):
        q0, q1 = int(pb.qo_indptr[b]), int(pb.qo_indptr[b + 1])
        kv_len, qo_len = int(pb.seq_lens[b]), q1 - q0
        if qo_len == 0:
            continue
        k, v = _gather_kv(a["cache"], pb, b, a["layout"])
        k = k.repeat_interleave(G, dim=1).transpose(0, 1)  # [Hq, kv, D]
        v = v.repeat_interleave(G, dim=1).transpose(0, 1)
        s = q[q0:q1].transpose(0, 1) @ k.transpose(1, 2) / math.sqrt(D)  # [Hq, qo, kv]
        m = torch.tensor([[t <= kv_len - qo_len + i and (window_left < 0 or t >= kv_len - qo_len + i - window_left)
                           for t in range(kv_len)] for i in range(qo_len)], dtype=torch.bool)
        s = s.masked_fill(~m, -math.inf)
        col = torch.as_tensor(sinks, dtype=torch.float64)[:, None, None].expand(-1, qo_len, 1)
        w = torch.softmax(torch.cat([s, col], -1), -1)[..., :-1]
        out[q0:q1] = (w @ v).transpose(0, 1)
    return out


@pytest.mark.parametrize("window_left", [-1, 7])
def test_attention_sinks_vs_gpt_oss_form(window_left):
    a = wl.attn_batch([37, 0, 5, 60], [1, 19, 12, 3], Hq=8, Hkv=2, D=64, page_size=16, seed=21)
    sinks = np.linspace(-3, 6, 8).astype(np.float32)
    want = _sink_reference(a, sinks, window_left).to(torch.float32).numpy()
    got = oracle.bf16_to_f32(_oracle_attn(a, sinks=sinks, window_left=window_left))
    assert np.abs(got - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-6
    # the sinks change the result (by up to a factor e^6 / (sum of the row's weights))
    assert np.abs(got - oracle.bf16_to_f32(_oracle_attn(a, window_left=window_left))).max() > 0.05


def test_attention_sink_limits_and_closed_form():
    a = wl.attn_batch([12, 30], [3, 1], Hq=4, Hkv=2, D=32, page_size=8, seed=22)
    plain = _oracle_attn(a)
    # a sink of -inf adds nothing: plain attention, bit for bit
    assert_bits_equal(_oracle_attn(a, sinks=np.full(4, -np.inf, np.float32)), plain, "sink -inf")
    # a dominant sink takes all the mass: the output vanishes
    assert not oracle.bf16_to_f32(_oracle_attn(a, sinks=np.full(4, 1e4, np.float32))).any()
    # one visible position with score s: out = v / (1 + e^(sink - s))
    a = wl.attn_batch([0], [1], Hq=2, Hkv=1, D=16, page_size=4, seed=23)
    k, v = _gather_kv(a["cache"], a["batch"], 0)
    s = ((a["q"][0].to(torch.float64) * k[0]).sum(-1) / 4.0).numpy()
    sk = np.array([0.5, -1.0], np.float32)
    want = v[0, 0].numpy()[None, :] / (1 + np.exp(sk.astype(np.float64) - s))[:, None]
    got = oracle.bf16_to_f32(_oracle_attn(a, sinks=sk))[0]
    np.testing.assert_allclose(got, want, rtol=2 ** -8, atol=1e-6)
