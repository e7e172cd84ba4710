"""GPU: a small Llama-3 style model run the way Pie's forward pass runs it, with `flashinfer`
served by this package (pie_amd.integration.install), against a float32 torch restatement of
the same model.

The bf16 path follows pie/src/pie_worker/model/llama3.py: `transform` (:712-790: get_seq_lens,
get_batch_indices_positions, the prefill wrapper's plan with a custom mask, or the decode
wrapper's plan), `attention` (:588-710: rms_norm, qkv projection, q/k/v views, Llama-3.1 RoPE in
place, paged append, wrapper.run, output projection, residual) and `mlp` (:543-586: rms_norm,
gate_up projection, silu * mul, down projection, residual), with each residual add fused into the
next norm as fused_add_rmsnorm does; GEMMs are torch's. The sampling step follows common.py
(safe_scaled_softmax, then a sampler). Prefill of three ragged requests, then one decode step per
request on the same cache. Tolerance: bf16 activations through two layers against float32, the
last-token logits of every request within 4% of the logits' range and cosine similarity above
0.999 (measured: 1.2-1.4%, 0.99965); the greedy token agrees where the top-2 margin exceeds the
error. A skipped RoPE or a dropped residual add measured 56-76% of the range, cosine below 0.2.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import oracle
from pie_amd import integration, ops
from pie_amd import sampling as pie_sampling
from pie_amd import workloads as wl

pytestmark = pytest.mark.gpu

H, HQ, HKV, D, I, V, LAYERS, EPS, P = 1024, 8, 2, 128, 2048, 2000, 2, 1e-5, 16
ROPE = dict(rope_scale=8.0, rope_theta=5e5, low_freq_factor=1.0, high_freq_factor=4.0,
            old_context_len=8192)


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return torch.device("cuda:0")


def _weights(seed=60):
    g = torch.Generator().manual_seed(seed)
    n = lambda *s, std=0.02: (torch.randn(*s, generator=g) * std).to(torch.bfloat16)
    nw = lambda *s: (1.0 + torch.randn(*s, generator=g) * 0.1).to(torch.bfloat16)
    w = {"emb": n(V, H, std=1.0), "final": nw(H), "lm": n(V, H)}
    for l in range(LAYERS):
        w[f"{l}.attn"], w[f"{l}.mlp"] = nw(H), nw(H)
        # projections large enough that attention and the MLP move the residual stream (with
        # std 0.02 the logits barely depend on them, and a skipped RoPE went unnoticed)
        w[f"{l}.qkv"] = n((HQ + 2 * HKV) * D, H, std=0.08)
        w[f"{l}.o"] = n(H, HQ * D, std=0.06)
        w[f"{l}.gu"] = n(2 * I, H, std=0.06)  # [gate; up] rows, as the loader fuses them
        w[f"{l}.down"] = n(H, I, std=0.06)
    return w


def _ref_logits(tokens, w, dev):
    """float32 restatement for one request's whole sequence: logits of every position."""
    f = lambda k: w[k].to(dev).float()
    L = len(tokens)
    inv = torch.tensor(oracle.inv_freq_llama31(D, ROPE["rope_scale"], ROPE["rope_theta"],
                                               ROPE["low_freq_factor"], ROPE["high_freq_factor"],
                                               ROPE["old_context_len"]), dtype=torch.float64)
    ang = torch.arange(L, dtype=torch.float64)[:, None] * inv[None, :]
    cos, sin = ang.cos().float().to(dev), ang.sin().float().to(dev)

    def rope(x):  # [L, h, D], half-split pairs
        a, b = x[..., : D // 2], x[..., D // 2:]
        c, s = cos[:, None, :], sin[:, None, :]
        return torch.cat([a * c - b * s, a * s + b * c], -1)

    norm = lambda x, wk: F.rms_norm(x, [H], f(wk), EPS)
    h = f("emb")[torch.as_tensor(tokens, device=dev).long()]
    for l in range(LAYERS):
        qkv = norm(h, f"{l}.attn") @ f(f"{l}.qkv").T
        q = rope(qkv[:, : HQ * D].view(L, HQ, D))
        k = rope(qkv[:, HQ * D: (HQ + HKV) * D].view(L, HKV, D))
        v = qkv[:, (HQ + HKV) * D:].view(L, HKV, D)
        rep = HQ // HKV
        k, v = k.repeat_interleave(rep, 1), v.repeat_interleave(rep, 1)
        att = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1),
                                             is_causal=True)
        h = h + att.transpose(0, 1).reshape(L, HQ * D) @ f(f"{l}.o").T
        gu = norm(h, f"{l}.mlp") @ f(f"{l}.gu").T
        h = h + (F.silu(gu[:, :I]) * gu[:, I:]) @ f(f"{l}.down").T
    return norm(h, "final") @ f("lm").T


class _PieModel:
    """The bf16 path through the installed `flashinfer` namespace."""

    def __init__(self, w, dev, pool_pages=64):
        self.w = {k: v.to(dev) for k, v in w.items()}
        self.dev = dev
        self.cache = [wl.sentinel_cache((pool_pages, 2, P, HKV, D)).to(dev) for _ in range(LAYERS)]
        self.ws = torch.zeros(64 << 20, dtype=torch.uint8, device=dev)

    def forward(self, fi, ids, pos, qo_indptr, kv_indptr, kv_indices, last_len, custom_mask, decode):
        n = ids.numel()
        seq_lens = fi.get_seq_lens(kv_indptr, last_len, P)
        bidx, bpos = fi.get_batch_indices_positions(qo_indptr, seq_lens, n)
        if decode:
            wrapper = fi.BatchDecodeWithPagedKVCacheWrapper(self.ws, "NHD")
            wrapper.plan(indptr=kv_indptr, indices=kv_indices, last_page_len=last_len,
                         num_qo_heads=HQ, num_kv_heads=HKV, head_dim=D, page_size=P,
                         pos_encoding_mode="NONE", q_data_type=torch.bfloat16)
        else:
            wrapper = fi.BatchPrefillWithPagedKVCacheWrapper(self.ws, "NHD")
            kw = dict(custom_mask=custom_mask) if custom_mask is not None else dict(causal=True)
            wrapper.plan(qo_indptr=qo_indptr, paged_kv_indptr=kv_indptr, paged_kv_indices=kv_indices,
                         paged_kv_last_page_len=last_len, num_qo_heads=HQ, num_kv_heads=HKV,
                         head_dim_qk=D, page_size=P, q_data_type=torch.bfloat16, **kw)
        w = self.w
        h = ops.embedding(ids, w["emb"])
        down = None
        for l in range(LAYERS):
            if down is None:
                normed = ops.rmsnorm(h, w[f"{l}.attn"], EPS)
            else:
                normed, h = ops.add_rms_norm(down, h, w[f"{l}.attn"], EPS)  # h + down, then norm
            qkv = F.linear(normed, w[f"{l}.qkv"])
            q, k, v = torch.split(qkv, [HQ * D, HKV * D, HKV * D], dim=-1)
            q, k, v = q.view(n, HQ, D), k.view(n, HKV, D), v.view(n, HKV, D)
            fi.apply_llama31_rope_pos_ids_inplace(q=q, k=k, pos_ids=pos, **ROPE)
            fi.append_paged_kv_cache(append_key=k, append_value=v, batch_indices=bidx,
                                     positions=bpos, paged_kv_cache=self.cache[l],
                                     kv_indices=kv_indices, kv_indptr=kv_indptr,
                                     kv_last_page_len=last_len, kv_layout="NHD")
            att = wrapper.run(q, self.cache[l]).reshape(n, -1)
            o = F.linear(att, w[f"{l}.o"])
            normed, h = ops.add_rms_norm(o, h, w[f"{l}.mlp"], EPS)
            down = F.linear(fi.silu_and_mul(F.linear(normed, w[f"{l}.gu"])), w[f"{l}.down"])
        hn, h = ops.add_rms_norm(down, h, w["final"], EPS)
        return F.linear(hn, w["lm"])


def _causal_custom_mask(qo_lens, ctx_before):
    """Pie's flattened per-request boolean masks (query i sees kv positions <= ctx + i)."""
    parts = []
    for ql, cb in zip(qo_lens, ctx_before):
        kv = cb + ql
        parts.append((torch.arange(kv)[None, :] <= (cb + torch.arange(ql))[:, None]).flatten())
    return torch.cat(parts)


def _check(got_rows, want_rows, what):
    got, want = got_rows.float(), want_rows.float()
    span = float(want.max() - want.min())
    err = float((got - want).abs().max())
    cos = F.cosine_similarity(got, want, dim=-1)
    print(f"  {what}: max |err| {err:.4f}, logits span {span:.3f}, min cosine {float(cos.min()):.6f}")
    assert err <= 0.04 * span, f"{what}: max |err| {err:.4f} vs logits span {span:.3f}"
    assert float(cos.min()) > 0.999, f"{what}: cosine {cos.tolist()}"
    # greedy choice: equal wherever the reference's top-2 margin is beyond the error
    top2 = want.topk(2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 2 * err
    assert torch.equal(got.argmax(-1)[clear], want.argmax(-1)[clear]), what


@pytest.mark.parametrize("masking", ["causal", "custom_mask"])
def test_prefill_then_decode_matches_fp32_model(dev, masking):
    print(f"e2e layers masking={masking}", flush=True)
    fi = integration.install()
    try:
        w = _weights()
        model = _PieModel(w, dev)
        g = torch.Generator().manual_seed(61)
        prompts = [torch.randint(0, V, (L,), generator=g).tolist() for L in (37, 70, 5)]
        lens = torch.tensor([len(p) for p in prompts], dtype=torch.int32)
        zero = torch.zeros_like(lens)
        # prefill: pages for the prompt plus one decode token
        pb = wl.paged_batch(zero, lens + 1, P, 64, 62)
        npg = (lens + P - 1) // P
        kv_indptr = torch.zeros(len(prompts) + 1, dtype=torch.int32)
        kv_indptr[1:] = torch.cumsum(npg, 0)
        kv_indices = torch.cat([pb.kv_indices[int(pb.kv_indptr[b]): int(pb.kv_indptr[b]) + int(npg[b])]
                                for b in range(len(prompts))])
        last = (lens - P * (npg - 1)).to(torch.int32)
        qo = torch.zeros(len(prompts) + 1, dtype=torch.int32)
        qo[1:] = torch.cumsum(lens, 0)
        ids = torch.tensor(sum(prompts, []), dtype=torch.int32)
        pos = torch.cat([torch.arange(L, dtype=torch.int32) for L in lens.tolist()])
        mask = _causal_custom_mask(lens.tolist(), [0] * len(prompts)) if masking == "custom_mask" else None
        to = lambda t: t.to(dev)
        logits = model.forward(fi, to(ids), to(pos), to(qo), to(kv_indptr), to(kv_indices), to(last),
                               None if mask is None else to(mask), decode=False)
        last_rows = logits[(qo[1:] - 1).long().to(dev)]
        want = torch.stack([_ref_logits(p, w, dev)[-1] for p in prompts])
        _check(last_rows, want, "prefill last-token logits")

        # the sampling path on these logits (common.py:226-344): safe_scaled_softmax, then a
        # sampler from the `flashinfer.sampling` Pie imports; a greedy row (temperature 0) is the
        # one-hot of its argmax
        temps = torch.tensor([0.0, 0.7, 1.0], device=dev)
        probs = pie_sampling.safe_scaled_softmax(last_rows.contiguous(), temps).float()
        assert int(probs[0].argmax()) == int(last_rows[0].float().argmax()) and float(probs[0].max()) == 1.0
        tok = fi.sampling.top_k_top_p_sampling_from_probs(probs, 20, 0.9, seed=3, offset=0)
        assert tok.shape == (3,) and int(tok[0]) == int(probs[0].argmax())
        assert bool(((tok >= 0) & (tok < V)).all())

        # decode: one new token per request (its page table now covers prompt + 1)
        nxt = torch.randint(0, V, (len(prompts),), generator=g).to(torch.int32)
        logits_d = model.forward(fi, to(nxt), to(lens.clone()), to(torch.arange(len(prompts) + 1,
                                 dtype=torch.int32)), to(pb.kv_indptr), to(pb.kv_indices),
                                 to(pb.kv_last_page_len), None, decode=True)
        want_d = torch.stack([_ref_logits(p + [int(t)], w, dev)[-1] for p, t in zip(prompts, nxt)])
        _check(logits_d, want_d, "decode logits")
    finally:
        integration.uninstall()
