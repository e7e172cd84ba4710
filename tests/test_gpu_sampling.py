"""GPU parity of the sampling path: Pie's safe_scaled_softmax (fp32 and bf16 logits, greedy
rows) against the float64 oracle, and the five flashinfer samplers. With caller-given uniforms
and probabilities on a 2^-30 grid (exact in the kernel's fixed point and in float64) every draw
must equal the oracle's exactly; with the kernel's own Philox numbers the draws must follow the
kept-set distribution (chi-square over 40k draws with a fixed seed) and stay inside the kept set
at full vocabulary size (Llama-3 128256, Qwen3 151936)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from pie_amd import sampling
from tests._util import assert_bf16_close

pytestmark = pytest.mark.gpu
N = oracle.to_np
SAMPLERS = {
    "plain": lambda p, **kw: sampling.sampling_from_probs(p, **kw),
    "top_p": lambda p, top_p, **kw: sampling.top_p_sampling_from_probs(p, top_p, **kw),
    "top_k": lambda p, top_k, **kw: sampling.top_k_sampling_from_probs(p, top_k, **kw),
    "min_p": lambda p, min_p, **kw: sampling.min_p_sampling_from_probs(p, min_p, **kw),
    "top_k_top_p": lambda p, top_k, top_p, **kw: sampling.top_k_top_p_sampling_from_probs(
        p, top_k, top_p, **kw),
}


def _grid_probs(B, V, seed, ties=True):
    g = torch.Generator().manual_seed(seed)
    w = torch.randint(0, 4097, (B, V), generator=g).double() ** 2
    if ties:
        w[1::3, ::7] = w[1::3, :1]  # many tokens tied with one value
        w[2::4, 3] = 0
    p = w / w.sum(-1, keepdim=True)
    return (torch.floor(p * 2**30) / 2**30).float()


def _params(B, V, seed):
    g = torch.Generator().manual_seed(seed)
    k = torch.randint(1, V + 3, (B,), generator=g).to(torch.int32)
    k[0] = 0
    return dict(top_k=k, top_p=torch.rand(B, generator=g) * 0.98 + 0.01,
                min_p=torch.rand(B, generator=g) * 0.5,
                u=torch.rand(B, generator=g, dtype=torch.float64))


def _call(mode, probs, prm, **kw):
    args = {"plain": {}, "top_p": {"top_p": prm["top_p"]}, "top_k": {"top_k": prm["top_k"]},
            "min_p": {"min_p": prm["min_p"]},
            "top_k_top_p": {"top_k": prm["top_k"], "top_p": prm["top_p"]}}[mode]
    return SAMPLERS[mode](probs, **args, **kw)


@pytest.mark.parametrize("mode", list(SAMPLERS))
@pytest.mark.parametrize("V", [301, 4099, 32000])
def test_sample_exact_vs_oracle(dev, mode, V):
    print(f"sample mode={mode} V={V}", flush=True)
    B = 24
    probs = _grid_probs(B, V, V + len(mode))
    prm = _params(B, V, V)
    dp = {k: v.to(dev) for k, v in prm.items()}
    got = _call(mode, probs.to(dev), dp, uniforms=dp["u"]).cpu().numpy()
    want, kept = oracle.sample(probs.numpy(), mode, prm["u"].numpy(), top_k=prm["top_k"].numpy(),
                               top_p=prm["top_p"].numpy(), min_p=prm["min_p"].numpy())
    assert (got == want).all(), f"rows {np.nonzero(got != want)[0][:5]}: {got[got != want][:5]} vs {want[got != want][:5]}"
    assert kept[np.arange(B), got].all()


@pytest.mark.parametrize("scale", [1.0, 3.0, 6.0, 0.0])
def test_top_p_regimes_exact(dev, scale):
    """top_p at Llama-3 vocabulary over rows whose kept sets range from 60% of the vocabulary
    (logits N(0, 1)) to a few tokens (N(0, 6)) and all-equal rows (scale 0: one histogram bin
    holds the whole row), with p from 0.001 (one to three tokens kept) to 0.999, exact against
    the oracle with given uniforms; min_p near 1 and tiny top_p on the same rows (candidate lists
    of one to three elements)."""
    print(f"top_p regimes scale={scale}", flush=True)
    B, V = 12, 128256
    g = torch.Generator().manual_seed(int(scale * 10) + 5)
    logits = torch.randn(B, V, generator=g, dtype=torch.float64) * scale
    p = torch.softmax(logits, -1)
    probs = (torch.floor(p * 2**30) / 2**30).float()
    prm = _params(B, V, 90)
    prm["top_p"] = torch.tensor([0.001, 0.01, 0.1, 0.3, 0.5, 0.7, 0.8, 0.9, 0.95, 0.99, 0.999, 1.0])
    prm["min_p"] = torch.tensor([0.99, 0.9, 0.5, 0.3, 0.1, 0.05, 0.01, 0.001, 0.0, 0.999, 0.7, 0.2])
    dp = {k: v.to(dev) for k, v in prm.items()}
    for mode in ("top_p", "min_p", "top_k_top_p"):
        got = _call(mode, probs.to(dev), dp, uniforms=dp["u"]).cpu().numpy()
        want, kept = oracle.sample(probs.numpy(), mode, prm["u"].numpy(), top_k=prm["top_k"].numpy(),
                                   top_p=prm["top_p"].numpy(), min_p=prm["min_p"].numpy())
        assert (got == want).all(), f"{mode}: rows {np.nonzero(got != want)[0][:5]}: {got[got != want][:5]} vs {want[got != want][:5]}"
        assert kept[np.arange(B), got].all()


@pytest.mark.parametrize("mode", list(SAMPLERS))
def test_sample_long_rows(dev, mode):
    """Rows of more than 256 tiles of 4096 (the draw's chunks then span several tiles), one with
    a length that is not a multiple of 4 (scalar loads)."""
    for V in (1_100_000, 1_048_583):
        print(f"sample mode={mode} V={V}", flush=True)
        B = 4
        probs = _grid_probs(B, V, V + 1)
        prm = _params(B, V, V + 2)
        dp = {k: v.to(dev) for k, v in prm.items()}
        got = _call(mode, probs.to(dev), dp, uniforms=dp["u"]).cpu().numpy()
        want, _ = oracle.sample(probs.numpy(), mode, prm["u"].numpy(), top_k=prm["top_k"].numpy(),
                                top_p=prm["top_p"].numpy(), min_p=prm["min_p"].numpy())
        assert (got == want).all(), f"V={V}: {got} vs {want}"


@pytest.mark.parametrize("mode", list(SAMPLERS))
@pytest.mark.parametrize("V", [4099, 128256])
def test_sample_uniform_edges(dev, mode, V):
    """u = 0 draws the first kept token and u = 1 (target = the whole kept mass, which no running
    sum exceeds) the last one, as in the oracle; rows whose last kept token is not in the row's
    last chunk (trailing zeros) exercise the draw's search for the last chunk with kept mass."""
    print(f"sample edges mode={mode} V={V}", flush=True)
    B = 8
    probs = _grid_probs(B, V, V + 5, ties=False)
    probs[4:, V // 2:] = 0  # trailing zeros: the last kept token sits mid-row
    probs = probs / probs.sum(-1, keepdim=True)
    probs = (torch.floor(probs.double() * 2**30) / 2**30).float()
    prm = _params(B, V, V + 6)
    prm["top_k"] = torch.randint(1, 300, (B,), generator=torch.Generator().manual_seed(V)).to(torch.int32)
    prm["u"] = torch.tensor([0.0, 1.0] * (B // 2), dtype=torch.float64)
    dp = {k: v.to(dev) for k, v in prm.items()}
    got = _call(mode, probs.to(dev), dp, uniforms=dp["u"]).cpu().numpy()
    want, kept = oracle.sample(probs.numpy(), mode, prm["u"].numpy(), top_k=prm["top_k"].numpy(),
                               top_p=prm["top_p"].numpy(), min_p=prm["min_p"].numpy())
    assert (got == want).all(), f"rows {np.nonzero(got != want)[0][:5]}: {got[got != want][:5]} vs {want[got != want][:5]}"
    assert kept[np.arange(B), got].all()


@pytest.mark.parametrize("mode", list(SAMPLERS))
def test_sample_padded_rows(dev, mode):
    """16-byte aligned rows whose length is not a multiple of 4 (a padded row stride): the
    vector passes and the candidate lists' last elements."""
    B, V, pad = 16, 128253, 3
    g = torch.Generator().manual_seed(77)
    full = torch.softmax(torch.randn(B, V + pad, generator=g, dtype=torch.float64) * 3, -1).float()
    full[:, V:] = 0.9  # never read: beyond each row's V entries
    probs = full[:, :V]
    prm = _params(B, V, 78)
    prm["top_k"] = torch.randint(1, 300, (B,), generator=g).to(torch.int32)
    dp = {k: v.to(dev) for k, v in prm.items()}
    got = _call(mode, full.to(dev)[:, :V], dp, uniforms=dp["u"]).cpu().numpy()
    want, kept = oracle.sample(probs.contiguous().numpy(), mode, prm["u"].numpy(),
                               top_k=prm["top_k"].numpy(), top_p=prm["top_p"].numpy(),
                               min_p=prm["min_p"].numpy())
    assert kept[np.arange(B), got].all()
    assert (got == want).all(), f"{got} vs {want}"


def test_sample_scalar_params_and_row_indices(dev):
    B, V = 16, 1000
    probs = _grid_probs(B, V, 5)
    u = torch.rand(12, generator=torch.Generator().manual_seed(6), dtype=torch.float64)
    idx = torch.tensor([3, 3, 0, 15, 7, 7, 7, 1, 2, 9, 11, 4], dtype=torch.int32)
    got = sampling.top_k_top_p_sampling_from_probs(probs.to(dev), 50, 0.7, indices=idx.to(dev),
                                                   uniforms=u.to(dev)).cpu().numpy()
    want, _ = oracle.sample(probs[idx.long()].numpy(), "top_k_top_p", u.numpy(), top_k=50, top_p=0.7)
    assert (got == want).all()


def test_sample_distribution_with_philox(dev):
    """40k draws of one 8-token distribution per mode, fixed seed: chi-square against the
    renormalised kept set (p-value above 1e-4 for every mode)."""
    from scipy.stats import chisquare
    p = torch.tensor([0.02, 0.3, 0.05, 0.2, 0.13, 0.1, 0.15, 0.05])
    n = 40000
    probs = p.repeat(n, 1).to(dev)
    for mode in SAMPLERS:
        prm = dict(top_k=4, top_p=0.6, min_p=0.3, u=None)
        got = _call(mode, probs, prm, seed=1234, offset=7).cpu().numpy()
        _, kept = oracle.sample(p[None].numpy(), mode, [0.5], top_k=4, top_p=0.6, min_p=0.3)
        kept = kept[0]
        assert kept[got].all(), mode
        counts = np.bincount(got, minlength=8)[kept]
        expect = p.numpy()[kept].astype(np.float64)
        expect = expect / expect.sum() * n
        pv = chisquare(counts, expect).pvalue
        assert pv > 1e-4, f"{mode}: p-value {pv}, counts {counts}, expected {expect}"


def test_sample_reproducible_by_seed_and_offset(dev):
    probs = _grid_probs(64, 5000, 9).to(dev)
    a = sampling.sampling_from_probs(probs, seed=42, offset=3)
    b = sampling.sampling_from_probs(probs, seed=42, offset=3)
    c = sampling.sampling_from_probs(probs, seed=42, offset=4)
    assert torch.equal(a, b) and not torch.equal(a, c)
    g = torch.Generator().manual_seed(77)
    d, e = sampling.sampling_from_probs(probs, generator=g), sampling.sampling_from_probs(probs, generator=g)
    assert not torch.equal(d, e)  # the generator advances
    g2 = torch.Generator().manual_seed(77)  # the same seed replays the same sequence of draws
    assert torch.equal(sampling.sampling_from_probs(probs, generator=g2), d)
    assert torch.equal(sampling.sampling_from_probs(probs, generator=g2), e)
    gg = torch.Generator(device=probs.device).manual_seed(5)  # a GPU generator: its offset advances
    off0 = gg.get_offset()
    f1, f2 = sampling.sampling_from_probs(probs, generator=gg), sampling.sampling_from_probs(probs, generator=gg)
    assert not torch.equal(f1, f2) and gg.get_offset() > off0


@pytest.mark.parametrize("V", [128256, 151936])
def test_sample_full_vocab_kept_sets(dev, V):
    """Full vocabulary, softmax of N(0, 3) logits (as after the LM head): every mode's draws stay
    in the oracle's kept set, and with given uniforms equal the oracle's draw except where the
    fp32 probabilities' 2^-40 rounding moves a boundary (none expected here)."""
    B = 32
    g = torch.Generator().manual_seed(V)
    logits = torch.randn(B, V, generator=g) * 3
    probs = torch.softmax(logits.double(), -1).float()
    prm = _params(B, V, 11)
    prm["top_k"] = torch.randint(1, 200, (B,), generator=g).to(torch.int32)
    dp = {k: v.to(dev) for k, v in prm.items()}
    for mode in SAMPLERS:
        got = _call(mode, probs.to(dev), dp, uniforms=dp["u"]).cpu().numpy()
        want, kept = oracle.sample(probs.numpy(), mode, prm["u"].numpy(), top_k=prm["top_k"].numpy(),
                                   top_p=prm["top_p"].numpy(), min_p=prm["min_p"].numpy())
        assert kept[np.arange(B), got].all(), mode
        assert (got == want).mean() >= 0.9, f"{mode}: {(got == want).mean()}"
        free = _call(mode, probs.to(dev), dp, seed=5, offset=0).cpu().numpy()
        assert kept[np.arange(B), free].all(), f"{mode} (Philox)"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("V,pad", [(128256, 0), (151936, 0), (50257, 7), (70001, 3), (200003, 0)])
def test_safe_scaled_softmax(dev, dtype, V, pad):
    """Row lengths that run the register-resident kernel at each of its sizes (with and without
    tail elements, padded row strides) and the streaming one (200003: too long for registers;
    unpadded odd lengths: rows not 16-byte aligned)."""
    print(f"safe_scaled_softmax V={V} pad={pad} {dtype}", flush=True)
    B = 8
    g = torch.Generator().manual_seed(21)
    full = (torch.randn(B, V + pad, generator=g) * 4)
    full[0, 5] = full[0, V - 1] = full[0].max() + 1  # tied maxima: the first one wins
    full = full.to(dtype)
    logits = full[:, :V]
    temps = torch.tensor([0.0, 1e-6, 0.3, 0.7, 1.0, 1.0, 1.7, 5.0])
    got = sampling.safe_scaled_softmax(full.to(dev)[:, :V], temps.to(dev))
    want = oracle.scaled_softmax(logits.float().numpy(), temps.numpy())
    gotf = got.float().cpu().numpy().astype(np.float64)
    assert gotf[0, 5] == 1.0, "first of tied maxima"
    assert (gotf[:2] == want[:2]).all(), "greedy rows are exact one-hots"
    rel = 2 ** -7 if dtype == torch.bfloat16 else 1e-5
    bad = np.abs(gotf - want) > rel * np.abs(want) + 1e-30
    assert not bad.any(), f"{bad.sum()} entries off, first {np.argwhere(bad)[:3]}"
    np.testing.assert_allclose(gotf[2:].sum(-1), 1.0, rtol=2e-2 if dtype == torch.bfloat16 else 1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("V", [4096, 128256, 151936, 200003])
def test_safe_scaled_softmax_masked_logits(dev, dtype, V):
    """-inf logits (padding, banned tokens) get probability 0, as in the reference's Triton
    kernel and torch.softmax: whole leading 16-byte groups of a thread masked (row 1: the first
    3/4 of the row), every other 16-byte group (row 2), everything but one token (row 3, which
    must come out exactly 1), a greedy row with masked entries (row 0). Register-resident sizes
    and the streaming kernel (200003)."""
    print(f"safe_scaled_softmax masked V={V} {dtype}", flush=True)
    B, E = 6, (8 if dtype == torch.bfloat16 else 4)
    g = torch.Generator().manual_seed(22)
    x = torch.randn(B, V, generator=g) * 4
    col = torch.arange(V)
    x[0, : V // 2] = -float("inf")
    x[1, : 3 * V // 4] = -float("inf")
    x[2, (col // E) % 2 == 0] = -float("inf")
    x[3, :] = -float("inf")
    x[3, V // 3] = 1.5
    x[4, -E * 3:] = -float("inf")
    x = x.to(dtype)
    temps = torch.tensor([0.0, 0.7, 1.0, 1.3, 0.5, 2.0])
    got = sampling.safe_scaled_softmax(x.to(dev), temps.to(dev)).float().cpu().numpy().astype(np.float64)
    want = oracle.scaled_softmax(x.float().numpy(), temps.numpy())
    assert np.isfinite(got).all(), f"{(~np.isfinite(got)).sum()} non-finite entries"
    assert (got[x.float().numpy() == -np.inf] == 0).all(), "masked logits must get probability 0"
    assert got[3, V // 3] == 1.0 and got[3].sum() == 1.0
    assert (got[0] == want[0]).all(), "greedy row"
    rel = 2 ** -7 if dtype == torch.bfloat16 else 1e-5
    bad = np.abs(got - want) > rel * np.abs(want) + 1e-30
    assert not bad.any(), f"{bad.sum()} entries off, first {np.argwhere(bad)[:3]}"


def test_sampling_chain_like_pie(dev):
    """Pie's order (common.py:226-283): softmax with temperatures, then a sampler per group."""
    B, V = 6, 32000
    logits = torch.randn(B, V, generator=torch.Generator().manual_seed(3)).to(dev) * 2
    temps = torch.tensor([0.0, 0.8, 0.8, 1.0, 1.2, 0.5], device=dev)
    probs = sampling.safe_scaled_softmax(logits, temps)
    tok = sampling.top_k_top_p_sampling_from_probs(probs, 40, 0.9, seed=1, offset=0)
    assert tok.dtype == torch.int32 and tok.shape == (B,)
    assert int(tok[0]) == int(logits[0].argmax())  # greedy row
    assert ((tok >= 0) & (tok < V)).all()


def _sample_positions(V):
    """The entries the one-read paths sample for their floor: the first three batches of 256
    16-byte vectors of each of the 16 wave segments of the row."""
    nv = V // 4
    seg = (nv + 15) // 16
    m = torch.zeros(V, dtype=torch.bool)
    for w in range(16):
        m[4 * w * seg: 4 * min(nv, w * seg + 3 * 256)] = True
    return m


@pytest.mark.parametrize("mode", ["top_k", "top_k_top_p", "min_p"])
@pytest.mark.parametrize("case", ["plain", "zero", "tiny", "large", "clustered"])
def test_sample_one_read_and_fallbacks(dev, mode, case):
    """top_k with small k and min_p over a long row take their floor from a sample of the row
    (the start of every wave segment): an ordinary sample (one read), a sample of zeros (no
    floor: the two-pass path), a sample of tiny positives (the floor admits almost the whole row:
    the candidate lists overflow and the two-pass path runs), a sample holding the row's largest
    entries, and the largest entries clustered in one segment outside the sample (that wave's
    list fills and raises its own floor)."""
    print(f"sample {mode} case={case}", flush=True)
    B, V = 12, 128256
    g = torch.Generator().manual_seed(91)
    w = torch.randint(1, 4097, (B, V), generator=g).double() ** 2
    sm = _sample_positions(V)
    if case == "zero":
        w[:, sm] = 0
    elif case == "tiny":
        w[:, sm] = 1e3
    elif case == "large":
        w[:, sm] *= 64
    elif case == "clustered":
        seg = 4 * ((V // 4 + 15) // 16)
        w[:, 5 * seg + 4 * 3 * 256: 6 * seg] *= 64  # segment 5 past its sampled batches
    p = (torch.floor(w / w.sum(-1, keepdim=True) * 2**30) / 2**30).float()
    prm = _params(B, V, 92)
    prm["top_k"] = torch.randint(1, 257, (B,), generator=g).to(torch.int32)
    prm["top_k"][1] = 256
    prm["min_p"][0] = 1.0
    prm["min_p"][1] = 1e-4
    dp = {k: v.to(dev) for k, v in prm.items()}
    got = _call(mode, p.to(dev), dp, uniforms=dp["u"]).cpu().numpy()
    want, kept = oracle.sample(p.numpy(), mode, prm["u"].numpy(), top_k=prm["top_k"].numpy(),
                               top_p=prm["top_p"].numpy(), min_p=prm["min_p"].numpy())
    assert kept[np.arange(B), got].all()
    assert (got == want).all(), f"{got} vs {want}"
