"""GPU parity: RoPE (standard and Llama-3.1; tolerance 1e-2 rel / 2e-2 abs of the float64
oracle), the paged KV append (bit-exact, untouched pages keep a sentinel), the fused
RoPE + append (bit-identical to the two separate calls) and the index helpers (exact)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from pie_amd import ops
from pie_amd import workloads as wl
from tests._util import assert_bf16_close, assert_bf16_close_rows, assert_bits_equal

pytestmark = pytest.mark.gpu
N = oracle.to_np
L31 = dict(rope_scale=8.0, rope_theta=5e5, low_freq_factor=1.0, high_freq_factor=4.0,
           old_context_len=8192)


def _small_batch(seed=0, B=5, max_len=40, ctx_max=50, page_size=16, Hq=4, Hkv=2, D=128):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(1, max_len + 1, (B,), generator=g).to(torch.int32)
    ctx = torch.randint(0, ctx_max + 1, (B,), generator=g).to(torch.int32)
    need = int(((ctx + lens + page_size - 1) // page_size).sum())
    pb = wl.paged_batch(ctx, lens, page_size, need + 7, seed + 1)
    T = int(lens.sum())
    qkv = wl.normal((T, (Hq + 2 * Hkv) * D), seed + 2)
    return pb, qkv, T


def _oracle_rope(q, k, pos, freqs, rd=None, interleave=False):
    return oracle.rope(N(q), N(k), N(pos), freqs, rotary_dim=rd, interleave=interleave)


@pytest.mark.parametrize("interleave", [False, True])
@pytest.mark.parametrize("D,rd", [(128, None), (64, None), (128, 64), (256, None)])
def test_llama31_rope(dev, interleave, D, rd):
    print(f"llama31 rope D={D} rd={rd} interleave={interleave}", flush=True)
    pb, qkv, T = _small_batch(D=D)
    qkv_d = qkv.to(dev)
    q, k, _ = wl.split_qkv(qkv_d, 4, 2, D)
    q0, k0, _ = wl.split_qkv(qkv, 4, 2, D)
    ops.apply_llama31_rope_pos_ids_inplace(q, k, pb.positions.to(dev), rotary_dim=rd,
                                           interleave=interleave, **L31)
    torch.cuda.synchronize()
    f = oracle.inv_freq_llama31(rd or D, 8.0, 5e5, 1.0, 4.0, 8192)
    wq, wk = _oracle_rope(q0, k0, pb.positions, f, rd, interleave)
    assert_bf16_close(N(q), wq, what="q")
    assert_bf16_close(N(k), wk, what="k")
    # v columns of the projection are untouched
    assert_bits_equal(N(qkv_d)[:, (4 + 2) * D:], N(qkv)[:, (4 + 2) * D:], "v untouched")


def test_standard_rope_scalar_path(dev):
    """rd = 24 is not a multiple of 16: the scalar kernel runs."""
    pb, qkv, T = _small_batch(D=32, Hq=3, Hkv=1)
    q, k, _ = wl.split_qkv(qkv.to(dev), 3, 1, 32)
    q0, k0, _ = wl.split_qkv(qkv, 3, 1, 32)
    ops.apply_rope_pos_ids_inplace(q, k, pb.positions.to(dev), rotary_dim=24, rope_theta=1e4)
    wq, wk = _oracle_rope(q0, k0, pb.positions, oracle.inv_freq_std(24, 1.0, 1e4), 24)
    assert_bf16_close(N(q), wq, what="q scalar")
    assert_bf16_close(N(k), wk, what="k scalar")


def test_rope_position_zero_identity(dev):
    q = wl.normal((9, 4, 128), 1)
    k = wl.normal((9, 2, 128), 2)
    qd, kd = q.to(dev), k.to(dev)
    ops.apply_rope_pos_ids_inplace(qd, kd, torch.zeros(9, dtype=torch.int32, device=dev), rope_theta=1e6)
    assert_bits_equal(N(qd), N(q), "pos 0 q")
    assert_bits_equal(N(kd), N(k), "pos 0 k")


def test_rope_large_positions(dev):
    """Positions up to 128k: fp32 angles stay within tolerance of the float64 oracle."""
    q, k = wl.normal((64, 2, 128), 3), wl.normal((64, 1, 128), 4)
    pos = torch.randint(0, 131072, (64,), generator=torch.Generator().manual_seed(5)).to(torch.int32)
    qd, kd = q.to(dev), k.to(dev)
    ops.apply_llama31_rope_pos_ids_inplace(qd, kd, pos.to(dev), **L31)
    wq, wk = _oracle_rope(q, k, pos, oracle.inv_freq_llama31(128, 8.0, 5e5, 1.0, 4.0, 8192))
    assert_bf16_close(N(qd), wq, what="q long ctx")
    assert_bf16_close(N(kd), wk, what="k long ctx")


def _cache(shape, layout, dev):
    return wl.sentinel_cache(shape).to(dev)


@pytest.mark.parametrize("layout", ["NHD", "HND"])
def test_append(dev, layout):
    print(f"append layout={layout}", flush=True)
    pb, qkv, T = _small_batch()
    _, k, v = wl.split_qkv(qkv, 4, 2, 128)
    shape = (pb.num_pages, 2, 16, 2, 128) if layout == "NHD" else (pb.num_pages, 2, 2, 16, 128)
    cache = _cache(shape, layout, dev)
    kd, vd = wl.split_qkv(qkv.to(dev), 4, 2, 128)[1:]
    ops.append_paged_kv_cache(kd, vd, pb.batch_indices.to(dev), pb.positions.to(dev), cache,
                              pb.kv_indices.to(dev), pb.kv_indptr.to(dev),
                              pb.kv_last_page_len.to(dev), kv_layout=layout)
    want = N(wl.sentinel_cache(shape))
    n = oracle.append(N(k), N(v), N(pb.batch_indices), N(pb.positions), want,
                      N(pb.kv_indices), N(pb.kv_indptr), layout)
    assert n == T
    assert_bits_equal(N(cache), want, f"cache {layout}")
    assert (want == wl.SENTINEL_BITS).any()


def test_append_tuple_cache_and_skips(dev):
    pb, qkv, T = _small_batch(seed=3)
    _, k, v = wl.split_qkv(qkv, 4, 2, 128)
    bidx, pos = pb.batch_indices.clone(), pb.positions.clone()
    bidx[0] = 99             # batch index out of range -> skipped
    pos[1] = 100000          # beyond the request's pages -> skipped
    kc = _cache((pb.num_pages, 16, 2, 128), "NHD", dev)
    vc = _cache((pb.num_pages, 16, 2, 128), "NHD", dev)
    ops.append_paged_kv_cache(k.to(dev), v.to(dev), bidx.to(dev), pos.to(dev), (kc, vc),
                              pb.kv_indices.to(dev), pb.kv_indptr.to(dev),
                              pb.kv_last_page_len.to(dev))
    want = N(wl.sentinel_cache((pb.num_pages, 2, 16, 2, 128)))
    n = oracle.append(N(k), N(v), N(bidx), N(pos), want, N(pb.kv_indices), N(pb.kv_indptr))
    assert n == T - 2
    assert_bits_equal(N(kc), want[:, 0], "k cache")
    assert_bits_equal(N(vc), want[:, 1], "v cache")


@pytest.mark.parametrize("interleave", [False, True])
@pytest.mark.parametrize("rd", [None, 64])
def test_fused_rope_append_equals_separate(dev, interleave, rd):
    print(f"fused rope+append interleave={interleave} rd={rd}", flush=True)
    pb, qkv, T = _small_batch(seed=5)
    shape = (pb.num_pages, 2, 16, 2, 128)
    args = lambda d: (pb.batch_indices.to(d), pb.positions.to(d))
    # separate calls
    a = qkv.to(dev)
    qa, ka, va = wl.split_qkv(a, 4, 2, 128)
    ca = _cache(shape, "NHD", dev)
    ops.apply_llama31_rope_pos_ids_inplace(qa, ka, pb.positions.to(dev), rotary_dim=rd,
                                           interleave=interleave, **L31)
    ops.append_paged_kv_cache(ka, va, *args(dev), ca, pb.kv_indices.to(dev), pb.kv_indptr.to(dev),
                              pb.kv_last_page_len.to(dev))
    # fused
    b = qkv.to(dev)
    qb, kb, vb = wl.split_qkv(b, 4, 2, 128)
    cb = _cache(shape, "NHD", dev)
    ops.apply_llama31_rope_pos_ids_and_append_paged_kv_cache(
        qb, kb, vb, pb.positions.to(dev), *args(dev), cb, pb.kv_indices.to(dev),
        pb.kv_indptr.to(dev), pb.kv_last_page_len.to(dev), rotary_dim=rd, interleave=interleave,
        **L31)
    assert_bits_equal(N(b), N(a), "q/k/v buffers")
    assert_bits_equal(N(cb), N(ca), "cache")
    # and against the oracle
    q0, k0, v0 = wl.split_qkv(qkv, 4, 2, 128)
    f = oracle.inv_freq_llama31(rd or 128, 8.0, 5e5, 1.0, 4.0, 8192)
    wq, wk = _oracle_rope(q0, k0, pb.positions, f, rd, interleave)
    assert_bf16_close(N(qb), wq, what="fused q")
    want = N(wl.sentinel_cache(shape))
    oracle.append(N(kb), N(v0), N(pb.batch_indices), N(pb.positions), want, N(pb.kv_indices),
                  N(pb.kv_indptr))
    assert_bits_equal(N(cb), want, "fused cache holds rotated k")


def test_config3_full(dev):
    """Llama-3 prefill batch (64 ragged requests, T ~ 65k): append bit-exact on the whole
    8192-page pool; RoPE vs the oracle on every token; fused == separate."""
    c = wl.cfg3()
    pb, T = c["batch"], c["qkv"].shape[0]
    q0, k0, v0 = wl.split_qkv(c["qkv"], 32, 8, 128)
    a = c["qkv"].to(dev)
    q, k, v = wl.split_qkv(a, 32, 8, 128)
    cache = _cache(c["cache_shape"], "NHD", dev)
    dv = {n: getattr(pb, n).to(dev) for n in ("batch_indices", "positions", "kv_indices",
                                              "kv_indptr", "kv_last_page_len")}
    ops.apply_llama31_rope_pos_ids_inplace(q, k, dv["positions"], **c["rope"])
    ops.append_paged_kv_cache(k, v, dv["batch_indices"], dv["positions"], cache, dv["kv_indices"],
                              dv["kv_indptr"], dv["kv_last_page_len"])
    kr = N(k)
    want = N(wl.sentinel_cache(c["cache_shape"]))
    assert oracle.append(kr, N(v0), N(pb.batch_indices), N(pb.positions), want,
                         N(pb.kv_indices), N(pb.kv_indptr)) == T
    assert_bits_equal(N(cache), want, "cfg3 cache")
    f = oracle.inv_freq_llama31(128, 8.0, 5e5, 1.0, 4.0, 8192)
    wq, wk = _oracle_rope(q0, k0, pb.positions, f)  # every token
    assert_bf16_close_rows(N(q), wq, chunk=4096, what="cfg3 q")
    assert_bf16_close_rows(kr, wk, chunk=4096, what="cfg3 k")
    del wq, wk
    b = c["qkv"].to(dev)
    qb, kb, vb = wl.split_qkv(b, 32, 8, 128)
    cb = _cache(c["cache_shape"], "NHD", dev)
    ops.apply_llama31_rope_pos_ids_and_append_paged_kv_cache(
        qb, kb, vb, dv["positions"], dv["batch_indices"], dv["positions"], cb, dv["kv_indices"],
        dv["kv_indptr"], dv["kv_last_page_len"], **c["rope"])
    assert torch.equal(b.view(torch.int16), a.view(torch.int16))
    assert torch.equal(cb.view(torch.int16), cache.view(torch.int16))


def test_index_helpers(dev):
    rng = np.random.default_rng(5)
    npages = rng.integers(0, 6, 300)
    npages[[3, 77]] = 0
    indptr = np.concatenate([[0], np.cumsum(npages)]).astype(np.int32)
    last = rng.integers(1, 17, 300).astype(np.int32)
    sl = ops.get_seq_lens(torch.from_numpy(indptr).to(dev), torch.from_numpy(last).to(dev), 16)
    want_sl = oracle.seq_lens(indptr, last, 16)
    assert_bits_equal(N(sl), want_sl, "seq_lens")
    newtok = np.minimum(rng.integers(0, 9, 300), want_sl)
    qo = np.concatenate([[0], np.cumsum(newtok)]).astype(np.int32)
    nnz = int(qo[-1])
    b, p = ops.get_batch_indices_positions(torch.from_numpy(qo).to(dev), sl, nnz)
    wb, wp = oracle.batch_indices_positions(qo, want_sl, nnz)
    assert_bits_equal(N(b), wb, "batch_indices")
    assert_bits_equal(N(p), wp, "positions")


def test_index_helpers_feed_append(dev):
    """get_seq_lens -> get_batch_indices_positions -> append, as transform() chains them
    (llama3.py:745-755, :675)."""
    c = wl.cfg5(B=64, V=16)
    pb = c["batch"]
    sl = ops.get_seq_lens(pb.kv_indptr.to(dev), pb.kv_last_page_len.to(dev), 16)
    b, p = ops.get_batch_indices_positions(pb.qo_indptr.to(dev), sl, 64)
    assert_bits_equal(N(b), N(pb.batch_indices))
    assert_bits_equal(N(p), N(pb.positions))


@pytest.mark.parametrize("D", [128, 64])
def test_qk_norm_rope_append_equals_separate(dev, D):
    """One-pass q/k norm + RoPE + append (qwen3.py:651-684) == the three calls, bit for bit;
    and the cache holds the oracle's append of the normalised, rotated k."""
    print(f"qk_rms_norm_rope_append D={D}", flush=True)
    pb, qkv, T = _small_batch(seed=9, D=D, ctx_max=300)
    qkv_d = qkv.to(dev)
    q, k, v = wl.split_qkv(qkv_d, 4, 2, D)
    qw, kw = wl.normal((D,), 1, 1.0, 0.1).to(dev), wl.normal((D,), 2, 1.0, 0.1).to(dev)
    shape = (pb.num_pages, 2, 16, 2, D)
    d = {n: getattr(pb, n).to(dev) for n in ("batch_indices", "positions", "kv_indices",
                                             "kv_indptr", "kv_last_page_len")}
    ca = _cache(shape, "NHD", dev)
    qa, ka = ops.qk_rms_norm_rope_append(q, k, v, qw, kw, 1e-6, d["positions"], d["batch_indices"],
                                         d["positions"], ca, d["kv_indices"], d["kv_indptr"],
                                         d["kv_last_page_len"], rope_theta=1e6)
    qb, kb = ops.qk_rms_norm(q, k, qw, kw, 1e-6)
    cb = _cache(shape, "NHD", dev)
    ops.apply_rope_pos_ids_inplace(qb, kb, d["positions"], rope_theta=1e6)
    ops.append_paged_kv_cache(kb, v, d["batch_indices"], d["positions"], cb, d["kv_indices"],
                              d["kv_indptr"], d["kv_last_page_len"])
    assert_bits_equal(N(qa), N(qb), "q")
    assert_bits_equal(N(ka), N(kb), "k")
    assert_bits_equal(N(ca), N(cb), "cache")
    q0, k0, v0 = wl.split_qkv(qkv, 4, 2, D)
    wq, wk = oracle.rope(oracle.rmsnorm(N(q0), N(qw), 1e-6), oracle.rmsnorm(N(k0), N(kw), 1e-6),
                         N(pb.positions), oracle.inv_freq_std(D, 1.0, 1e6))
    assert_bf16_close(N(qa), wq, what="q vs oracle")
    assert_bf16_close(N(ka), wk, what="k vs oracle")
