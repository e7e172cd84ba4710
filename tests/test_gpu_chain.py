"""GPU: the Qwen3-8B decode-step op chain (configuration 5) eagerly vs the oracle, fused and
grouped (one launch) vs unfused bit for bit, and HIP-graph replays vs the eager result (every
replay checked, with eager work and synchronisation between replays). The configured
151936-row table runs once, grouped, against the oracle."""
from __future__ import annotations

import pytest
import torch

import oracle
from pie_amd import workloads as wl
from pie_amd.chain import DecodeChain
from tests._util import assert_bf16_close, assert_bits_equal

pytestmark = pytest.mark.gpu
N = oracle.to_np


@pytest.fixture(scope="module")
def cfg():
    return wl.cfg5(V=4096)  # full decode shape; a smaller vocabulary keeps the table small


def _snap(ch):
    torch.cuda.synchronize()
    return {k: N(v) for k, v in ch.outputs().items()}


def _check_vs_oracle(got, cfg):
    hid, _ = oracle.embedding(N(cfg["ids"]), N(cfg["W"]))
    assert_bits_equal(got["hidden"], hid, "embedding")
    y, s = oracle.add_rmsnorm(hid, N(cfg["residual"]), N(cfg["w_norm"]), cfg["eps"])
    assert_bits_equal(got["residual"], s, "residual")
    assert_bf16_close(got["normed"], y, what="add_rmsnorm")
    q, k, v = wl.split_qkv(cfg["qkv"], 32, 8, 128)
    qn = oracle.rmsnorm(N(q), N(cfg["q_norm"]), cfg["eps"])
    kn = oracle.rmsnorm(N(k), N(cfg["k_norm"]), cfg["eps"])
    pos = N(cfg["batch"].positions)
    f = oracle.inv_freq_std(128, 1.0, cfg["theta"])
    wq, wk = oracle.rope(qn, kn, pos, f)
    assert_bf16_close(got["q"], wq, what="q norm+rope")
    assert_bf16_close(got["k"], wk, what="k norm+rope")
    pb = cfg["batch"]
    want = N(wl.sentinel_cache(cfg["cache_shape"]))
    oracle.append(got["k"], N(v), N(pb.batch_indices), N(pb.positions), want, N(pb.kv_indices),
                  N(pb.kv_indptr))
    assert_bits_equal(got["cache"], want, "cache")
    assert_bf16_close(got["act"], oracle.silu_and_mul(N(cfg["gate_up"])), what="silu")


@pytest.mark.parametrize("grouped", [False, True])
def test_chain_vs_oracle(dev, cfg, grouped):
    print(f"chain vs oracle grouped={grouped}", flush=True)
    ch = DecodeChain(cfg, dev, fused=True, grouped=grouped)
    ch.run()
    _check_vs_oracle(_snap(ch), cfg)


def test_chain_full_vocabulary_grouped(dev):
    """Configuration 5 exactly as configured: the [151936, 4096] embedding table."""
    print("chain V=151936 grouped", flush=True)
    full = wl.cfg5()
    ch = DecodeChain(full, dev, grouped=True)
    ch.run()
    _check_vs_oracle(_snap(ch), full)


@pytest.mark.parametrize("mode", ["fused", "grouped"])
def test_chain_fused_equals_unfused(dev, cfg, mode):
    print(f"chain {mode} vs unfused", flush=True)
    a = DecodeChain(cfg, dev, fused=True, grouped=mode == "grouped")
    b = DecodeChain(cfg, dev, fused=False)
    a.run()
    b.run()
    ga, gb = _snap(a), _snap(b)
    for key in ga:
        assert_bits_equal(ga[key], gb[key], key)


@pytest.mark.parametrize("grouped", [False, True])
def test_chain_graph_replays(dev, cfg, grouped):
    print(f"chain graph replays grouped={grouped}", flush=True)
    ch = DecodeChain(cfg, dev, fused=True, grouped=grouped)
    ch.reset()
    ch.run()
    eager = _snap(ch)
    g = ch.capture()
    for i in range(4):
        ch.reset()
        junk = torch.randn(1 << 20, device=dev).sum()  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        got = _snap(ch)
        for key in eager:
            assert_bits_equal(got[key], eager[key], f"replay {i} {key}")
        del junk


def test_chain_saved_group_relaunches(dev, cfg):
    """The chain recorded once (ops.saved_group) and relaunched: every relaunch equals the
    one-off grouped launch bit for bit, the inputs reset in place between relaunches (the saved
    launch reads the recorded buffers when it runs)."""
    print("chain saved group relaunches", flush=True)
    a = DecodeChain(cfg, dev, grouped=True)
    a.reset()
    a.run()
    want = _snap(a)
    s = DecodeChain(cfg, dev, saved=True)
    for i in range(3):
        s.reset()  # restores the residual stream and the cache in place
        if i == 1:
            s.residual.add_(1.0)  # a changed input: the relaunch must see it
        s.run()
        got = _snap(s)
        if i == 1:
            assert not (got["residual"] == want["residual"]).all(), "relaunch ignored new inputs"
            continue
        for key in want:
            assert_bits_equal(got[key], want[key], f"relaunch {i} {key}")
