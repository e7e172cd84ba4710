"""GPU parity of paged attention (flashinfer's decode and prefill wrappers) against the float64
oracle: bf16 outputs within 1e-2 relative / 2e-2 absolute (RTOL/ATOL in tests/_util.py), plus
tighter structural checks (uniform keys give the exact mean of the visible v rows, so a dropped
or extra position shows), graph capture with re-planned page tables, and the decode
configuration at full size (Qwen3-8B, 256 sequences, contexts U[128, 4096])."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from pie_amd import _lib, attention
from pie_amd import workloads as wl
from tests._util import assert_bf16_close

pytestmark = pytest.mark.gpu
N = oracle.to_np
WS_BYTES = 128 * 1024 * 1024  # Pie's workspace (llama3.py:230-232)


def _workspace(dev):
    return torch.zeros(WS_BYTES, dtype=torch.uint8, device=dev)


def _decode(dev, a, splits=None, out=None, window_left=-1):
    pb, lay = a["batch"], a["layout"]
    w = attention.BatchDecodeWithPagedKVCacheWrapper(_workspace(dev), lay)
    w.plan(pb.kv_indptr.to(dev), pb.kv_indices.to(dev), pb.kv_last_page_len.to(dev),
           a["Hq"], a["Hkv"], a["D"], pb.page_size, pos_encoding_mode="NONE",
           q_data_type=torch.bfloat16, window_left=window_left)
    if splits is not None:
        w._plan["splits"] = splits
    o = w.run(a["q"].to(dev), a["cache"].to(dev), out=out)
    torch.cuda.synchronize()
    return o


def _want(a, custom=None, window_left=-1, causal=True):
    pb = a["batch"]
    return oracle.attention(N(a["q"]), N(a["cache"]), N(pb.qo_indptr), N(pb.kv_indptr),
                            N(pb.kv_indices), N(pb.kv_last_page_len), custom_mask=custom,
                            layout=a["layout"], window_left=window_left, causal=causal)


def _tight(got, want, what):
    """|err| <= 1/256 + |want|/128: averages of N(0,1) rows rounded once to bf16."""
    g = oracle.bf16_to_f32(N(got) if isinstance(got, torch.Tensor) else got).astype(np.float64)
    w = oracle.bf16_to_f32(want).astype(np.float64)
    r = np.abs(g - w) / (1 / 256 + np.abs(w) / 128)
    assert r.max() <= 1.0, f"{what}: worst error {r.max():.3f} of the bound at {np.unravel_index(r.argmax(), r.shape)}"


@pytest.mark.parametrize("layout", ["NHD", "HND"])
@pytest.mark.parametrize("Hq,Hkv,D,P", [(32, 8, 128, 16), (8, 8, 64, 16), (16, 2, 256, 8),
                                        (28, 4, 128, 5), (16, 1, 128, 32)])
@pytest.mark.parametrize("splits", [None, 1, 3])
def test_decode_vs_oracle(dev, layout, Hq, Hkv, D, P, splits):
    print(f"decode Hq={Hq} Hkv={Hkv} D={D} P={P} layout={layout} splits={splits}", flush=True)
    g = torch.Generator().manual_seed(Hq * 7 + D + P)
    ctx = torch.randint(0, 700, (9,), generator=g).to(torch.int32)
    ctx[0] = 0  # a request whose only kv token is the new one
    a = wl.attn_batch(ctx, torch.ones(9, dtype=torch.int32), Hq=Hq, Hkv=Hkv, D=D, page_size=P,
                      pool_pages=int(((ctx + P) // P).sum()) + 3, seed=int(ctx.sum()) % 1000,
                      layout=layout)
    got = _decode(dev, a, splits)
    want = _want(a)
    assert_bf16_close(N(got), want, what="decode")
    _tight(got, want, "decode")


@pytest.mark.parametrize("B", [256, 257])
def test_decode_request_order(dev, B):
    """Batches of at most 256 requests are worked on longest first (ranked on the device, ties by
    request index), larger ones in request order: tied and distinct lengths against the oracle,
    and the same requests given in another order give the same rows bit for bit."""
    print(f"decode request order B={B}", flush=True)
    g = torch.Generator().manual_seed(B)
    ctx = torch.tensor([0, 1, 15, 16, 17, 40, 95])[torch.randint(0, 7, (B,), generator=g)].to(torch.int32)
    ctx[: B // 4] = torch.randint(0, 200, (B // 4,), generator=g).to(torch.int32)
    a = wl.attn_batch(ctx, torch.ones(B, dtype=torch.int32), Hq=8, Hkv=2, D=128, page_size=16,
                      seed=B + 7)
    want = _want(a)
    perm = torch.randperm(B, generator=g)
    ap = wl.attn_batch(ctx[perm], torch.ones(B, dtype=torch.int32), Hq=8, Hkv=2, D=128,
                       page_size=16, seed=B + 7)
    # the same k/v rows and q rows per request: copy them over into the permuted layout
    pb, pbp = a["batch"], ap["batch"]
    for i in range(B):
        b = int(perm[i])
        src = pb.kv_indices[int(pb.kv_indptr[b]):int(pb.kv_indptr[b + 1])].long()
        dst = pbp.kv_indices[int(pbp.kv_indptr[i]):int(pbp.kv_indptr[i + 1])].long()
        ap["cache"][dst] = a["cache"][src]
    ap["q"] = a["q"][perm].clone()
    for splits in (None, 2):
        got = _decode(dev, a, splits)
        assert_bf16_close(N(got), want, what=f"decode B={B} splits {splits}")
        _tight(got, want, f"decode B={B} splits {splits}")
        gotp = _decode(dev, ap, splits)
        assert torch.equal(gotp.cpu(), got.cpu()[perm]), f"B={B} splits {splits}: permuted batch differs"


def test_decode_page_size_one_long_context(dev):
    """Page size 1: a 1500-token context spans several 510-page windows of the staged table."""
    a = wl.attn_batch(torch.tensor([1499, 700, 3]), torch.ones(3, dtype=torch.int32), Hq=8, Hkv=2,
                      D=128, page_size=1, seed=90)
    for splits in (1, 2):
        got = _decode(dev, a, splits)
        want = _want(a)
        assert_bf16_close(N(got), want, what=f"P=1 splits {splits}")
        _tight(got, want, f"P=1 splits {splits}")


def test_decode_uniform_keys_average_visible_rows(dev):
    """Every key equal: the output is the plain mean of exactly the request's kv_len v rows."""
    a = wl.attn_batch(torch.tensor([0, 15, 16, 17, 300, 511]), torch.ones(6, dtype=torch.int32),
                      Hq=8, Hkv=2, D=128, page_size=16, seed=60)
    pb = a["batch"]
    a["cache"][:, 0] = a["cache"][0, 0, 0, 0]  # one k row everywhere
    a["cache"][:, 1] = wl.normal(a["cache"][:, 1].shape, 61, 0.0, 1.0)
    for splits in (1, 4):
        got = oracle.bf16_to_f32(N(_decode(dev, a, splits))).astype(np.float64)
        for b in range(6):
            L = int(pb.seq_lens[b])
            pages = pb.kv_indices[int(pb.kv_indptr[b]):int(pb.kv_indptr[b + 1])].long()
            v = a["cache"][pages, 1].to(torch.float64).reshape(-1, 2, 128)[:L]  # [L, Hkv, D]
            mean = v.mean(0).repeat_interleave(4, 0).numpy()
            assert np.abs(got[b] - mean).max() <= 1 / 256 + np.abs(mean).max() / 128, \
                f"request {b} (kv_len {L}) splits {splits}"


def test_decode_graph_replay_with_new_tables(dev):
    """Pie's graph mode: plan once on dummy one-page tables, capture, then replay after copying
    new page tables and lengths into the fixed buffers (llama3.py:340-414, :905-950)."""
    B, Hq, Hkv, D, P = 16, 32, 8, 128, 16
    pool = 16 * 64
    cache = wl.normal((pool + 1, 2, P, Hkv, D), 70).to(dev)
    ib = torch.zeros(B + 1, dtype=torch.int32, device=dev)
    xb = torch.zeros(pool + 1, dtype=torch.int32, device=dev)
    lb = torch.zeros(B, dtype=torch.int32, device=dev)
    w = attention.BatchDecodeWithPagedKVCacheWrapper(_workspace(dev), "NHD", use_cuda_graph=True,
                                                     paged_kv_indptr_buffer=ib,
                                                     paged_kv_indices_buffer=xb,
                                                     paged_kv_last_page_len_buffer=lb)
    ib.copy_(torch.arange(B + 1, dtype=torch.int32))
    lb.fill_(1)
    xb[:B].fill_(pool)
    w.plan(ib, xb, lb, Hq, Hkv, D, P, q_data_type=torch.bfloat16)
    q = torch.zeros((B, Hq, D), dtype=torch.bfloat16, device=dev)
    out = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=dev)
    w.run(q, cache, out=out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        w.run(q, cache, out=out)
    g = torch.Generator().manual_seed(71)
    for rep in range(3):
        ctx = torch.randint(1, 64 * P - 1, (B,), generator=g).to(torch.int32)
        pb = wl.paged_batch(ctx, torch.ones(B, dtype=torch.int32), P, pool, 72 + rep)
        ib.copy_(pb.kv_indptr)
        xb[: pb.kv_indices.numel()].copy_(pb.kv_indices)
        lb.copy_(pb.kv_last_page_len)
        q.copy_(wl.normal((B, Hq, D), 73 + rep))
        graph.replay()
        torch.cuda.synchronize()
        a = {"q": q.cpu(), "cache": cache.cpu(), "batch": pb, "layout": "NHD"}
        want = _want(a)
        assert_bf16_close(N(out), want, what=f"replay {rep}")
        _tight(out, want, f"replay {rep}")
        # eager work between replays
        torch.cuda.synchronize()


def test_decode_full_config_sampled(dev):
    """Configuration: Qwen3-8B decode attention, 256 sequences, contexts U[128, 4096] (+1 new
    token), cache ~2.2 GB. The oracle checks 24 sampled requests against the full output."""
    a = wl.attn_decode_cfg()
    pb = a["batch"]
    got = N(_decode(dev, a))
    cache = N(a["cache"])
    pick = np.random.default_rng(0).choice(pb.seq_lens.numel(), 24, replace=False)
    for b in pick:
        b = int(b)
        ind = pb.kv_indices[int(pb.kv_indptr[b]):int(pb.kv_indptr[b + 1])]
        want = oracle.attention(N(a["q"][b:b + 1]), cache, np.array([0, 1], np.int32),
                                np.array([0, ind.numel()], np.int32), N(ind),
                                N(pb.kv_last_page_len[b:b + 1]))
        assert_bf16_close(got[b:b + 1], want, what=f"request {b}")
        _tight(got[b:b + 1], want, f"request {b}")


def test_decode_rejects_bad_input(dev):
    a = wl.attn_batch([5], [1], Hq=8, Hkv=2, D=128, page_size=16, seed=80)
    pb = a["batch"]
    w = attention.BatchDecodeWithPagedKVCacheWrapper(_workspace(dev), "NHD")
    with pytest.raises(RuntimeError):
        w.run(a["q"].to(dev), a["cache"].to(dev))  # before plan
    w.plan(pb.kv_indptr.to(dev), pb.kv_indices.to(dev), pb.kv_last_page_len.to(dev), 8, 2, 128, 16)
    with pytest.raises(ValueError):
        w.run(a["q"].to(dev)[:, :4], a["cache"].to(dev))  # wrong head count
    with pytest.raises(ValueError):
        w.run(a["q"].to(dev).float(), a["cache"].to(dev))
    with pytest.raises(NotImplementedError):
        w.plan(pb.kv_indptr.to(dev), pb.kv_indices.to(dev), pb.kv_last_page_len.to(dev), 8, 2,
               128, 16, pos_encoding_mode="ROPE_LLAMA")


# ----------------------------------------------------------------------------- prefill
def _prefill(dev, a, causal=True, custom=None, out=None, window_left=-1):
    pb = a["batch"]
    w = attention.BatchPrefillWithPagedKVCacheWrapper(_workspace(dev), a["layout"])
    w.plan(pb.qo_indptr.to(dev), pb.kv_indptr.to(dev), pb.kv_indices.to(dev),
           pb.kv_last_page_len.to(dev), a["Hq"], a["Hkv"], a["D"], pb.page_size,
           custom_mask=None if custom is None else torch.as_tensor(custom).to(dev), causal=causal,
           q_data_type=torch.bfloat16, window_left=window_left)
    o = w.run(a["q"].to(dev), a["cache"].to(dev), out=out)
    torch.cuda.synchronize()
    return o


def _brle_causal_mask(pb):
    """The mask Pie builds for plain causal requests (batching.py:335-386 with one true run of
    position+1): per request a [qo_len, kv_len] block, row i true for t <= kv_len - qo_len + i."""
    blocks = []
    for b in range(pb.seq_lens.numel()):
        qo, kv = int(pb.lens[b]), int(pb.seq_lens[b])
        t = torch.arange(kv)[None, :]
        i = torch.arange(qo)[:, None]
        blocks.append((t <= kv - qo + i).flatten())
    return torch.cat(blocks) if blocks else torch.zeros(0, dtype=torch.bool)


@pytest.mark.parametrize("layout", ["NHD", "HND"])
@pytest.mark.parametrize("Hq,Hkv,D,P", [(32, 8, 128, 16), (8, 8, 64, 16), (8, 2, 256, 8),
                                        (28, 4, 128, 5), (12, 4, 128, 1)])
@pytest.mark.parametrize("mode", ["causal", "full", "custom"])
def test_prefill_vs_oracle(dev, layout, Hq, Hkv, D, P, mode):
    print(f"prefill Hq={Hq} Hkv={Hkv} D={D} P={P} layout={layout} mode={mode}", flush=True)
    g = torch.Generator().manual_seed(Hq + D * 3 + P)
    B = 5
    ctx = torch.randint(0, 300, (B,), generator=g).to(torch.int32)
    qo = torch.randint(1, 90, (B,), generator=g).to(torch.int32)
    ctx[0], qo[1] = 0, 0  # a fresh prefill and a request with no query tokens
    a = wl.attn_batch(ctx, qo, Hq=Hq, Hkv=Hkv, D=D, page_size=P, seed=int(qo.sum()) % 997,
                      layout=layout)
    custom = None
    if mode == "custom":
        pb = a["batch"]
        n = int((pb.lens.to(torch.int64) * pb.seq_lens.to(torch.int64)).sum())
        custom = (torch.rand(n, generator=g) < 0.5)
        custom[:7] = False
    got = _prefill(dev, a, causal=mode == "causal", custom=custom)
    pb = a["batch"]
    want = oracle.attention(N(a["q"]), N(a["cache"]), N(pb.qo_indptr), N(pb.kv_indptr),
                            N(pb.kv_indices), N(pb.kv_last_page_len),
                            custom_mask=None if custom is None else custom.numpy(),
                            causal=mode == "causal", layout=layout)
    assert_bf16_close(N(got), want, what=mode)
    _tight(got, want, mode)


def test_prefill_pie_causal_mask_equals_causal_mode(dev):
    """Pie always passes a custom mask (batching.py:226-228); for plain causal requests it is the
    causal window, and the result is bit-identical to causal=True."""
    a = wl.attn_batch(torch.tensor([0, 40, 333, 7]), torch.tensor([130, 5, 64, 1]), Hq=32, Hkv=8,
                      D=128, page_size=16, seed=100)
    by_mask = _prefill(dev, a, custom=_brle_causal_mask(a["batch"]))
    by_mode = _prefill(dev, a, causal=True)
    assert torch.equal(by_mask.view(torch.int16), by_mode.view(torch.int16))


@pytest.mark.parametrize("D", [128, 64])
def test_prefill_nearly_causal_masks(dev, D):
    """Causal masks with a few bits changed (a hidden past position, a visible future one, a row
    cut short): work groups whose rows are all exactly causal take the causal path, the others
    read the mask; every row matches the oracle under the mask as given."""
    print(f"nearly causal D={D}", flush=True)
    a = wl.attn_batch(torch.tensor([0, 40, 333, 7, 0]), torch.tensor([130, 5, 64, 1, 70]), Hq=16,
                      Hkv=4, D=D, page_size=16, seed=101)
    pb = a["batch"]
    mask = _brle_causal_mask(pb).clone()
    starts = torch.cat([torch.zeros(1, dtype=torch.int64),
                        torch.cumsum(pb.lens.to(torch.int64) * pb.seq_lens.to(torch.int64), 0)])
    kv = [int(x) for x in pb.seq_lens]
    mask[int(starts[0]) + 97 * kv[0] + 3] = False            # request 0, row 97: a hidden past position
    mask[int(starts[2]) + 0 * kv[2] + kv[2] - 1] = True      # request 2, row 0: a visible future one
    r4 = int(starts[4]) + 40 * kv[4]
    mask[r4 + 20: r4 + 41] = False                            # request 4, row 40: cut short
    want = _want(a, custom=mask.numpy(), causal=False)
    got = _prefill(dev, a, custom=mask)
    assert_bf16_close(N(got), want, what="nearly causal")
    _tight(got, want, "nearly causal")
    exact = _prefill(dev, a, custom=_brle_causal_mask(pb))
    _tight(exact, _want(a), "exactly causal")


def test_prefill_decode_rows_match_decode_wrapper(dev):
    """One query token per request: prefill (causal) and decode agree within bf16 rounding."""
    a = wl.attn_batch(torch.randint(0, 900, (7,), generator=torch.Generator().manual_seed(3)),
                      torch.ones(7, dtype=torch.int32), Hq=32, Hkv=8, D=128, page_size=16, seed=101)
    p = _prefill(dev, a, causal=True)
    d = _decode(dev, a)
    _tight(p, N(d), "prefill vs decode")


def test_prefill_config3_sampled(dev):
    """Configuration 3's ragged batch (64 requests, lengths U[1, 2048], fresh causal prefill,
    Llama-3-8B heads): the full batch runs in one call; four requests are checked against the
    oracle (each request's rows depend only on its own pages)."""
    a = wl.attn_prefill_cfg()
    pb = a["batch"]
    got = N(_prefill(dev, a, causal=True))
    cache = N(a["cache"])
    lens = pb.lens.tolist()
    pick = [b for b in np.random.default_rng(1).permutation(len(lens)) if lens[b] <= 1100][:4]
    for b in pick:
        b = int(b)
        q0, q1 = int(pb.qo_indptr[b]), int(pb.qo_indptr[b + 1])
        ind = pb.kv_indices[int(pb.kv_indptr[b]):int(pb.kv_indptr[b + 1])]
        want = oracle.attention(N(a["q"][q0:q1]), cache, np.array([0, q1 - q0], np.int32),
                                np.array([0, ind.numel()], np.int32), N(ind),
                                N(pb.kv_last_page_len[b:b + 1]))
        assert_bf16_close(got[q0:q1], want, what=f"request {b} (len {q1 - q0})")
        _tight(got[q0:q1], want, f"request {b}")


@pytest.mark.parametrize("custom", [False, True])
def test_prefill_repeated_runs_and_graph_replays(dev, custom):
    """One plan, many runs: the head-dim-128 kernel counts its work in the plan's header and
    leaves the counters at zero, so every eager run and every replay of a captured run gives the
    first run's output bit for bit (with eager work between replays)."""
    print(f"prefill repeated runs custom={custom}", flush=True)
    a = wl.attn_batch([30, 0, 200, 5], [90, 64, 300, 40], Hq=32, Hkv=8, D=128, page_size=16, seed=121)
    pb = a["batch"]
    w = attention.BatchPrefillWithPagedKVCacheWrapper(_workspace(dev), a["layout"])
    mask = _brle_causal_mask(pb).to(dev) if custom else None
    w.plan(pb.qo_indptr.to(dev), pb.kv_indptr.to(dev), pb.kv_indices.to(dev), pb.kv_last_page_len.to(dev),
           32, 8, 128, 16, custom_mask=mask, causal=not custom)
    q, cache = a["q"].to(dev), a["cache"].to(dev)
    out = torch.empty_like(q)
    w.run(q, cache, out=out)
    torch.cuda.synchronize()
    first = out.clone()
    for i in range(3):
        out.zero_()
        w.run(q, cache, out=out)
        torch.cuda.synchronize()
        assert torch.equal(out, first), f"eager run {i + 1} differs"
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            w.run(q, cache, out=out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for i in range(3):
        out.zero_()
        junk = torch.randn(1 << 20, device=dev).sum()  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first), f"replay {i} differs"
        del junk
    want = _want(a, custom=_brle_causal_mask(pb).numpy() if custom else None, causal=not custom)
    assert_bf16_close(N(first), want, what="first run vs oracle")


def test_prefill_plan_in_use_on_another_stream_is_refused(dev):
    """The head-dim-128 kernel counts its work in the device plan, so two runs sharing a plan
    must not overlap: an eager run while the plan is still in use on another stream is refused
    (PIE_HIP_EBUSY), runs on the same stream queue as usual, and after a synchronisation the
    other stream runs and gives the same output bit for bit."""
    a = wl.attn_batch([0, 0, 0, 0], [4096, 4096, 4096, 4096], Hq=32, Hkv=8, D=128, page_size=16, seed=131)
    pb = a["batch"]
    w = attention.BatchPrefillWithPagedKVCacheWrapper(_workspace(dev), "NHD")
    w.plan(pb.qo_indptr.to(dev), pb.kv_indptr.to(dev), pb.kv_indices.to(dev), pb.kv_last_page_len.to(dev),
           32, 8, 128, 16, causal=True)
    q, cache = a["q"].to(dev), a["cache"].to(dev)
    out1, out2 = torch.empty_like(q), torch.empty_like(q)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(s1):
        for _ in range(4):  # ~1 ms of queued work on s1
            w.run(q, cache, out=out1)
    with torch.cuda.stream(s2):
        with pytest.raises(_lib.PieHipError, match="another stream"):
            w.run(q, cache, out=out2)
    s1.synchronize()
    with torch.cuda.stream(s2):
        w.run(q, cache, out=out2)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)


def test_prefill_plan_for_another_head_dim_gives_nan(dev):
    """A device plan made for head_dim 256 (other rows per item) driving the head-dim-128 kernel
    through the C ABI: the kernel cannot use it and fills the whole output with NaN instead of
    returning with the output unwritten."""
    a = wl.attn_batch([20, 3], [40, 9], Hq=8, Hkv=2, D=128, page_size=16, seed=132)
    pb = a["batch"]
    w = attention.BatchPrefillWithPagedKVCacheWrapper(_workspace(dev), "NHD")
    w.plan(pb.qo_indptr.to(dev), pb.kv_indptr.to(dev), pb.kv_indices.to(dev), pb.kv_last_page_len.to(dev),
           8, 2, 256, 16, causal=True)
    w._plan["D"] = 128  # bypass the wrapper's own shape check to reach the kernel
    out = torch.zeros_like(a["q"], device=dev)
    w.run(a["q"].to(dev), a["cache"].to(dev), out=out)
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()


def test_prefill_rejects_bad_input(dev):
    a = wl.attn_batch([5, 0], [3, 4], Hq=8, Hkv=2, D=128, page_size=16, seed=102)
    pb = a["batch"]
    w = attention.BatchPrefillWithPagedKVCacheWrapper(_workspace(dev), "NHD")
    with pytest.raises(RuntimeError):
        w.run(a["q"].to(dev), a["cache"].to(dev))
    w.plan(pb.qo_indptr.to(dev), pb.kv_indptr.to(dev), pb.kv_indices.to(dev),
           pb.kv_last_page_len.to(dev), 8, 2, 128, 16, causal=True)
    with pytest.raises(ValueError):
        w.run(a["q"].to(dev)[:3], a["cache"].to(dev))  # wrong token count
    with pytest.raises(ValueError):
        w.plan(pb.qo_indptr.to(dev), pb.kv_indptr.to(dev), pb.kv_indices.to(dev),
               pb.kv_last_page_len.to(dev), 8, 2, 128, 16,
               custom_mask=torch.ones(3, dtype=torch.bool, device=dev))  # mask too short
    with pytest.raises(NotImplementedError):
        w.plan(pb.qo_indptr.to(dev), pb.kv_indptr.to(dev), pb.kv_indices.to(dev),
               pb.kv_last_page_len.to(dev), 8, 2, 128, 16, logits_soft_cap=30.0)


# ----------------------------------------------------------------------------- sliding window
@pytest.mark.parametrize("window_left", [0, 31, 200, 4096])
@pytest.mark.parametrize("splits", [1, 3])
def test_decode_sliding_window(dev, window_left, splits):
    """flashinfer's window_left (OLMo-3 plans it per layer, olmo3.py:973-1005): the query sees
    positions >= kv_len - 1 - window_left."""
    g = torch.Generator().manual_seed(window_left + splits)
    ctx = torch.randint(0, 900, (7,), generator=g).to(torch.int32)
    a = wl.attn_batch(ctx, torch.ones(7, dtype=torch.int32), Hq=16, Hkv=4, D=128, page_size=16,
                      seed=110 + splits)
    got = _decode(dev, a, splits, window_left=window_left)
    want = _want(a, window_left=window_left)
    assert_bf16_close(N(got), want, what=f"window {window_left}")
    _tight(got, want, f"window {window_left}")


@pytest.mark.parametrize("window_left", [0, 50, 300])
@pytest.mark.parametrize("mode", ["causal", "full", "custom"])
def test_prefill_sliding_window(dev, window_left, mode):
    g = torch.Generator().manual_seed(window_left * 3 + len(mode))
    ctx = torch.randint(0, 400, (4,), generator=g).to(torch.int32)
    qo = torch.randint(1, 200, (4,), generator=g).to(torch.int32)
    a = wl.attn_batch(ctx, qo, Hq=32, Hkv=8, D=128, page_size=16, seed=120)
    custom = None
    if mode == "custom":
        pb = a["batch"]
        n = int((pb.lens.to(torch.int64) * pb.seq_lens.to(torch.int64)).sum())
        custom = torch.rand(n, generator=g) < 0.6
    got = _prefill(dev, a, causal=mode == "causal", custom=custom, window_left=window_left)
    want = _want(a, custom=None if custom is None else custom.numpy(), window_left=window_left,
                 causal=mode == "causal")
    assert_bf16_close(N(got), want, what=f"{mode} window {window_left}")
    _tight(got, want, f"{mode} window {window_left}")


def test_decode_graph_with_window_like_olmo(dev):
    """OLMo-3 captures decode graphs with window_left in the plan (olmo3.py:381-391)."""
    B, P, window = 8, 16, 100
    pool = B * 40
    cache = wl.normal((pool + 1, 2, P, 8, 128), 130).to(dev)
    ib = torch.arange(B + 1, dtype=torch.int32, device=dev)
    xb = torch.full((pool + 1,), pool, dtype=torch.int32, device=dev)
    lb = torch.ones(B, dtype=torch.int32, device=dev)
    w = attention.BatchDecodeWithPagedKVCacheWrapper(_workspace(dev), "NHD", use_cuda_graph=True,
                                                     paged_kv_indptr_buffer=ib,
                                                     paged_kv_indices_buffer=xb,
                                                     paged_kv_last_page_len_buffer=lb)
    w.plan(ib, xb, lb, 32, 8, 128, P, q_data_type=torch.bfloat16, window_left=window)
    q = torch.zeros((B, 32, 128), dtype=torch.bfloat16, device=dev)
    out = torch.empty_like(q)
    w.run(q, cache, out=out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        w.run(q, cache, out=out)
    ctx = torch.randint(1, 40 * P - 1, (B,), generator=torch.Generator().manual_seed(131)).to(torch.int32)
    pb = wl.paged_batch(ctx, torch.ones(B, dtype=torch.int32), P, pool, 132)
    ib.copy_(pb.kv_indptr)
    xb[: pb.kv_indices.numel()].copy_(pb.kv_indices)
    lb.copy_(pb.kv_last_page_len)
    q.copy_(wl.normal((B, 32, 128), 133))
    graph.replay()
    torch.cuda.synchronize()
    a = {"q": q.cpu(), "cache": cache.cpu(), "batch": pb, "layout": "NHD"}
    want = _want(a, window_left=window)
    _tight(out, want, "graph replay with window")


def _ramp_batch(slope, D, Hq=8, Hkv=2, page_size=16):
    """One fresh prefill (qo 200 tokens, no cached context) and one request with 300 cached
    tokens and 1 query token, where token t's key is a_t in every dimension and every query
    entry is 1: row scores rise (slope > 0) or fall (slope < 0) by |slope| log2 units per
    token. Rising scores move each row's maximum on every tile, by less or more than the
    kernels' lazy-maximum headroom (2^8) depending on the slope."""
    a = wl.attn_batch(torch.tensor([0, 300]), torch.tensor([200, 1]), Hq=Hq, Hkv=Hkv, D=D,
                      page_size=page_size, seed=131)
    pb = a["batch"]
    unit = D / np.sqrt(D) * np.log2(np.e)  # log2 units per unit of a_t (q = 1, scale 1/sqrt(D))
    cache = a["cache"].clone()
    for b in range(2):
        kv = int(pb.seq_lens[b])
        pages = pb.kv_indices[int(pb.kv_indptr[b]):int(pb.kv_indptr[b + 1])].long()
        for t in range(kv):
            cache[pages[t // page_size], 0, t % page_size] = slope * t / unit
    a["cache"] = cache
    a["q"] = torch.ones_like(a["q"])
    return a


@pytest.mark.parametrize("D", [128, 64])
@pytest.mark.parametrize("slope", [0.1, 0.3, 1.5, -1.5])
def test_prefill_and_decode_with_rising_scores(dev, D, slope):
    """Scores that rise steadily along the row (the running maximum grows inside the lazy
    headroom, past it, or on every tile) or fall (it never grows) match the oracle."""
    print(f"ramp D={D} slope={slope}", flush=True)
    a = _ramp_batch(slope, D)
    want = _want(a)
    got = _prefill(dev, a)
    assert_bf16_close(N(got), want, what=f"prefill slope {slope}")
    _tight(got, want, f"prefill slope {slope}")
    d = wl.attn_batch(torch.tensor([300]), torch.tensor([1]), Hq=8, Hkv=2, D=D, seed=131)
    d["cache"], d["q"] = a["cache"], a["q"][200:201]
    pb = a["batch"]
    d["batch"] = wl.paged_batch(torch.tensor([300]), torch.tensor([1]), 16, pb.kv_indices.numel(), 0)
    d["batch"].kv_indices[:] = pb.kv_indices[int(pb.kv_indptr[1]):]
    for splits in (1, 3):
        got = _decode(dev, d, splits=splits)
        _tight(got, _want(d), f"decode slope {slope} splits {splits}")


@pytest.mark.parametrize("sm_scale", [-0.09, 0.0])
def test_prefill_negative_and_zero_scale(dev, sm_scale):
    """A negative scale (the row maximum is the smallest raw score) and a zero scale (uniform
    weights over the visible tokens) match the oracle."""
    a = wl.attn_batch(torch.tensor([0, 70]), torch.tensor([90, 33]), Hq=8, Hkv=2, D=128, seed=133)
    pb = a["batch"]
    w = attention.BatchPrefillWithPagedKVCacheWrapper(_workspace(dev), "NHD")
    w.plan(pb.qo_indptr.to(dev), pb.kv_indptr.to(dev), pb.kv_indices.to(dev),
           pb.kv_last_page_len.to(dev), 8, 2, 128, pb.page_size, causal=True, sm_scale=sm_scale)
    got = w.run(a["q"].to(dev), a["cache"].to(dev))
    want = oracle.attention(N(a["q"]), N(a["cache"]), N(pb.qo_indptr), N(pb.kv_indptr),
                            N(pb.kv_indices), N(pb.kv_last_page_len), causal=True,
                            sm_scale=sm_scale)
    _tight(got, want, f"sm_scale {sm_scale}")


# ----------------------------------------------------------------------------- attention sinks
def _sink_run(dev, a, sinks, window_left=-1):
    """gpt-oss's calls: BatchAttentionWithAttentionSinkWrapper construction, plan (causal, with the
    layer's window), run(q, kv_cache_layer, sinks, scaling) (gpt_oss.py:420-438, :839-870, :693-697)."""
    pb = a["batch"]
    w = attention.BatchAttentionWithAttentionSinkWrapper(_workspace(dev), kv_layout=a["layout"],
                                                         window_left=window_left,
                                                         head_dim_qk=a["D"], head_dim_vo=a["D"])
    w.plan(pb.qo_indptr.to(dev), pb.kv_indptr.to(dev), pb.kv_indices.to(dev),
           pb.kv_last_page_len.to(dev), a["Hq"], a["Hkv"], a["D"], pb.page_size, causal=True,
           window_left=window_left, q_data_type=torch.bfloat16, non_blocking=True)
    o = w.run(a["q"].to(dev), a["cache"].to(dev), torch.as_tensor(sinks).to(dev), a["D"] ** -0.5)
    torch.cuda.synchronize()
    return o, w._use


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("window_left", [-1, 100])
def test_sink_wrapper_decode_batch(dev, D, window_left):
    print(f"sinks decode D={D} window={window_left}", flush=True)
    g = torch.Generator().manual_seed(31 + D)
    ctx = torch.randint(0, 900, (12,), generator=g).to(torch.int32)
    a = wl.attn_batch(ctx, torch.ones(12, dtype=torch.int32), Hq=16, Hkv=2, D=D, page_size=16, seed=33)
    sinks = torch.linspace(-3, 7, 16, dtype=torch.float32)
    got, used = _sink_run(dev, a, sinks, window_left)
    assert isinstance(used, attention.BatchDecodeWithPagedKVCacheWrapper)
    pb = a["batch"]
    want = oracle.attention(N(a["q"]), N(a["cache"]), N(pb.qo_indptr), N(pb.kv_indptr), N(pb.kv_indices),
                            N(pb.kv_last_page_len), window_left=window_left, sinks=sinks.numpy())
    assert_bf16_close(N(got), want, what="sink decode")
    _tight(got, want, "sink decode")


@pytest.mark.parametrize("D", [64, 128])
def test_sink_wrapper_prefill_batch(dev, D):
    print(f"sinks prefill D={D}", flush=True)
    a = wl.attn_batch([37, 0, 5, 160], [1, 90, 12, 33], Hq=8, Hkv=2, D=D, page_size=16, seed=35)
    sinks = torch.linspace(-2, 6, 8, dtype=torch.float32)
    got, used = _sink_run(dev, a, sinks)
    assert isinstance(used, attention.BatchPrefillWithPagedKVCacheWrapper)
    pb = a["batch"]
    want = oracle.attention(N(a["q"]), N(a["cache"]), N(pb.qo_indptr), N(pb.kv_indptr), N(pb.kv_indices),
                            N(pb.kv_last_page_len), sinks=sinks.numpy())
    assert_bf16_close(N(got), want, what="sink prefill")
    _tight(got, want, "sink prefill")
    plain = _want(a)
    assert (oracle.bf16_to_f32(N(got)) != oracle.bf16_to_f32(plain)).mean() > 0.5  # the sinks matter
