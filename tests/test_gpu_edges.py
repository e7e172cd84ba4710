"""GPU: edge cases across the entry points — empty batches (no tokens, no requests, no rows),
requests that append no tokens inside a ragged batch, and a one-entry vocabulary. Each call must
return without error, leave memory it does not own untouched, and agree with the oracle where
there is anything to compute."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from pie_amd import attention, ops, sampling
from pie_amd import workloads as wl

pytestmark = pytest.mark.gpu


def test_empty_token_batches(dev):
    """T = 0 everywhere: RoPE, the append, the fused pass, the embedding and the index ops."""
    bf = torch.bfloat16
    q = torch.empty((0, 4, 128), dtype=bf, device=dev)
    k = torch.empty((0, 2, 128), dtype=bf, device=dev)
    v = torch.empty((0, 2, 128), dtype=bf, device=dev)
    pos = torch.empty(0, dtype=torch.int32, device=dev)
    cache = wl.sentinel_cache((4, 2, 16, 2, 128)).to(dev)
    before = cache.clone()
    ind = torch.tensor([0, 1], dtype=torch.int32, device=dev)
    indptr = torch.tensor([0, 1], dtype=torch.int32, device=dev)
    last = torch.tensor([3], dtype=torch.int32, device=dev)
    ops.apply_rope_pos_ids_inplace(q, k, pos)
    ops.apply_llama31_rope_pos_ids_inplace(q, k, pos)
    ops.append_paged_kv_cache(k, v, pos, pos, cache, ind, indptr, last)
    ops.apply_llama31_rope_pos_ids_and_append_paged_kv_cache(q, k, v, pos, pos, pos, cache, ind,
                                                              indptr, last)
    torch.cuda.synchronize()
    assert torch.equal(cache.view(torch.int16), before.view(torch.int16))  # bits (NaN sentinel)
    W = wl.normal((10, 64), 1).to(dev)
    assert ops.embedding(torch.empty(0, dtype=torch.int32, device=dev), W).shape == (0, 64)
    seq = ops.get_seq_lens(indptr, last, 16)
    bidx, bpos = ops.get_batch_indices_positions(torch.tensor([0, 0], dtype=torch.int32, device=dev),
                                                 seq, 0)
    assert bidx.numel() == 0 and bpos.numel() == 0


def test_empty_sampling_batches(dev):
    probs = torch.empty((0, 100), dtype=torch.float32, device=dev)
    for fn, kw in ((sampling.sampling_from_probs, {}), (sampling.top_p_sampling_from_probs, {"top_p": 0.5}),
                   (sampling.top_k_sampling_from_probs, {"top_k": 3}),
                   (sampling.min_p_sampling_from_probs, {"min_p": 0.1}),
                   (sampling.top_k_top_p_sampling_from_probs, {"top_k": 3, "top_p": 0.5})):
        assert fn(probs, **kw).shape == (0,)
    logits = torch.empty((0, 100), dtype=torch.bfloat16, device=dev)
    assert sampling.safe_scaled_softmax(logits, torch.empty(0, device=dev)).shape == (0, 100)


def test_one_entry_vocabulary(dev):
    """V = 1: every sampler draws token 0 and the softmax is exactly 1."""
    probs = torch.ones((3, 1), dtype=torch.float32, device=dev)
    for fn, kw in ((sampling.sampling_from_probs, {}), (sampling.top_p_sampling_from_probs, {"top_p": 0.5}),
                   (sampling.top_k_sampling_from_probs, {"top_k": 1}),
                   (sampling.min_p_sampling_from_probs, {"min_p": 0.1}),
                   (sampling.top_k_top_p_sampling_from_probs, {"top_k": 1, "top_p": 0.9})):
        assert fn(probs, **kw).tolist() == [0, 0, 0]
    g = torch.Generator().manual_seed(5)
    logits = (torch.randn(64, 1, generator=g) * 30).to(dev)
    out = sampling.safe_scaled_softmax(logits, torch.linspace(0, 2, 64).to(dev))
    assert out.flatten().tolist() == [1.0] * 64  # exp(x - max) = exp(0), as torch computes it


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_softmax_rows_shorter_than_a_vector(dev, dtype):
    """Rows of 3 entries in a 16-byte-aligned padded layout (stride 8): shorter than one 16-byte
    vector, they take the streaming softmax; against the oracle, greedy rows one-hot."""
    g = torch.Generator().manual_seed(9)
    full = (torch.randn(16, 8, generator=g) * 3).to(dtype)
    temps = torch.linspace(0, 2, 16)
    out = sampling.safe_scaled_softmax(full.to(dev)[:, :3], temps.to(dev))
    want = oracle.scaled_softmax(full[:, :3].float().numpy(), temps.numpy())
    got = out.float().cpu().numpy().astype(np.float64)
    rel = 2 ** -7 if dtype == torch.bfloat16 else 1e-5
    assert np.all(np.abs(got - want) <= rel * np.abs(want) + 1e-30)


def test_prefill_with_requests_appending_nothing(dev):
    """A ragged prefill batch where some requests have no query tokens (cached context only) and
    one holds no context at all: the others match the oracle, and the empty ones write nothing."""
    ctx = torch.tensor([40, 0, 17, 5], dtype=torch.int32)
    new = torch.tensor([0, 9, 0, 23], dtype=torch.int32)
    a = wl.attn_batch(ctx, new, Hq=4, Hkv=2, D=128, seed=70)
    pb = a["batch"]
    q, cache = a["q"].to(dev), a["cache"].to(dev)
    ws = torch.zeros(16 << 20, dtype=torch.uint8, device=dev)
    w = attention.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(pb.qo_indptr.to(dev), pb.kv_indptr.to(dev), pb.kv_indices.to(dev),
           pb.kv_last_page_len.to(dev), 4, 2, 128, 16, causal=True)
    out = w.run(q, cache)
    N = oracle.to_np
    want = oracle.attention(N(a["q"]), N(a["cache"]), N(pb.qo_indptr), N(pb.kv_indptr),
                            N(pb.kv_indices), N(pb.kv_last_page_len), layout="NHD", causal=True)
    g = oracle.bf16_to_f32(N(out)).astype(np.float64)
    wv = oracle.bf16_to_f32(want).astype(np.float64)
    assert out.shape == q.shape
    assert (np.abs(g - wv) / (1 / 256 + np.abs(wv) / 128)).max() <= 1.0


def test_decode_with_empty_contexts(dev):
    """Decode requests with no cached tokens at all produce zero rows (nothing to attend to)."""
    ctx = torch.tensor([0, 30, 0], dtype=torch.int32)
    pb = wl.paged_batch(ctx, torch.zeros(3, dtype=torch.int32), 16, 8, 71)
    cache = wl.normal((8, 2, 16, 2, 128), 72).to(dev)
    q = wl.normal((3, 4, 128), 73).to(dev)
    ws = torch.zeros(16 << 20, dtype=torch.uint8, device=dev)
    w = attention.BatchDecodeWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(pb.kv_indptr.to(dev), pb.kv_indices.to(dev), pb.kv_last_page_len.to(dev), 4, 2, 128, 16)
    out = w.run(q, cache)
    assert bool(torch.isfinite(out.float()).all())
    assert float(out[0].float().abs().max()) == 0.0 and float(out[2].float().abs().max()) == 0.0
