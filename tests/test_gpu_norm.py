"""GPU parity: RMSNorm, residual-add + RMSNorm, per-head q/k RMSNorm vs the CPU oracle.

Tolerance (floating outputs): 1e-2 relative / 2e-2 absolute of the fp32-accumulated oracle.
The residual sum s is bit-exact (one fp32 add + RNE, as torch's bf16 `residual + x`).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from pie_amd import ops
from pie_amd import workloads as wl
from tests._util import assert_bf16_close, assert_bf16_close_rows, assert_bits_equal, ulp_diff

pytestmark = pytest.mark.gpu
N = oracle.to_np


def _sync():
    torch.cuda.synchronize()


@pytest.mark.parametrize("T,H", [(1, 512), (7, 2048), (2048, 2048), (33, 4096), (5, 8192),
                                 (3, 5120), (4, 896), (3, 100), (9, 128), (2, 64), (0, 4096)])
def test_rmsnorm(dev, T, H):
    print(f"rmsnorm T={T} H={H}", flush=True)
    x, w = wl.normal((T, H), 1), wl.normal((H,), 2, 1.0, 0.1)
    y = ops.rmsnorm(x.to(dev), w.to(dev), 1e-5)
    _sync()
    want = oracle.rmsnorm(N(x), N(w), 1e-5)
    assert_bf16_close(N(y), want, what=f"rmsnorm {T}x{H}")
    if T:
        assert ulp_diff(N(y), want).max() <= 2


@pytest.mark.parametrize("T,H", [(8192, 4096), (16384, 2048), (8200, 3584)])
def test_rmsnorm_large_row_lists(dev, T, H):
    """Plain norms of row lists past 64 MB (the non-temporal, row-prefetching paths)."""
    print(f"rmsnorm large T={T} H={H}", flush=True)
    x, w = wl.normal((T, H), 5), wl.normal((H,), 6, 1.0, 0.1)
    y = ops.rmsnorm(x.to(dev), w.to(dev), 1e-5)
    _sync()
    want = oracle.rmsnorm(N(x), N(w), 1e-5)
    assert_bf16_close(N(y), want, what=f"rmsnorm {T}x{H}")
    assert ulp_diff(N(y), want).max() <= 2


def test_rmsnorm_strided_and_misaligned(dev):
    H = 2048
    big = wl.normal((16, H + 8), 3).to(dev)
    x = big[:, :H]                      # row stride H+8, 16-byte aligned rows
    w = wl.normal((H,), 4, 1.0, 0.1).to(dev)
    y = ops.rmsnorm(x, w, 1e-6)
    assert_bf16_close(N(y), oracle.rmsnorm(N(x), N(w), 1e-6), what="strided")
    xm = big[:, 1:H + 1]                # misaligned base: scalar path
    ym = ops.rmsnorm(xm, w, 1e-6)
    assert_bf16_close(N(ym), oracle.rmsnorm(N(xm), N(w), 1e-6), what="misaligned")


def test_rmsnorm_special_rows(dev):
    H = 4096
    x = torch.zeros((3, H), dtype=torch.bfloat16)
    x[1] = 2.5
    x[2] = wl.normal((H,), 5)
    w = wl.normal((H,), 6, 1.0, 0.1)
    y = oracle.bf16_to_f32(N(ops.rmsnorm(x.to(dev), w.to(dev), 1e-6)))
    assert (y[0] == 0).all()
    np.testing.assert_allclose(y[1], oracle.bf16_to_f32(N(w)), rtol=1e-2)


def test_rms_norm_torch_signature(dev):
    x = wl.normal((6, 1024), 7)
    w = wl.normal((1024,), 8, 1.0, 0.1)
    y = ops.rms_norm(x.to(dev), [1024], w.to(dev), 1e-5)
    want = torch.nn.functional.rms_norm(x, [1024], w, 1e-5)
    assert ulp_diff(N(y), N(want)).max() <= 2


@pytest.mark.parametrize("T,H", [(1, 512), (17, 4096), (64, 2048), (5, 8192), (4, 896), (3, 100)])
def test_add_rmsnorm(dev, T, H):
    print(f"add_rmsnorm T={T} H={H}", flush=True)
    c = wl.cfg2(T=T, H=H, I=8)
    y, s = ops.add_rms_norm(c["x"].to(dev), c["r"].to(dev), c["w"].to(dev), 1e-5)
    _sync()
    wy, ws = oracle.add_rmsnorm(N(c["x"]), N(c["r"]), N(c["w"]), 1e-5)
    assert_bits_equal(N(s), ws, "residual sum")
    assert_bf16_close(N(y), wy, what="add_rmsnorm y")


def test_fused_add_rmsnorm_inplace(dev):
    c = wl.cfg2(T=32, H=4096, I=8)
    x, r = c["x"].to(dev), c["r"].to(dev)
    ops.fused_add_rmsnorm(x, r, c["w"].to(dev), 1e-5)
    wy, ws = oracle.add_rmsnorm(N(c["x"]), N(c["r"]), N(c["w"]), 1e-5)
    assert_bits_equal(N(r), ws, "residual updated in place")
    assert_bf16_close(N(x), wy, what="input overwritten by the norm")


def test_add_rmsnorm_full_config2(dev):
    """Llama-3-8B prefill shape: s bit-exact everywhere (against the IEEE add and the oracle),
    every row of y against the oracle."""
    c = wl.cfg2(I=8)
    x, r, w = c["x"].to(dev), c["r"].to(dev), c["w"].to(dev)
    y, s = ops.add_rms_norm(x, r, w, 1e-5)
    assert torch.equal(s.view(torch.int16), (r + x).view(torch.int16))  # IEEE add + RNE
    wy, ws = oracle.add_rmsnorm(N(c["x"]), N(c["r"]), N(c["w"]), 1e-5)
    assert_bits_equal(N(s), ws, "cfg2 s")
    gy = N(y)
    assert_bf16_close_rows(gy, wy, what="cfg2 y")
    assert ulp_diff(gy, wy).max() <= 2


@pytest.mark.parametrize("D", [128, 64, 256, 96])
def test_qk_rmsnorm(dev, D):
    print(f"qk_rmsnorm D={D}", flush=True)
    T, Hq, Hkv = 37, 8, 2
    qkv = wl.normal((T, (Hq + 2 * Hkv) * D), 9).to(dev)
    q, k, _ = wl.split_qkv(qkv, Hq, Hkv, D)
    qw, kw = wl.normal((D,), 10, 1.0, 0.1), wl.normal((D,), 11, 1.0, 0.1)
    qo, ko = ops.qk_rms_norm(q, k, qw.to(dev), kw.to(dev), 1e-6)
    _sync()
    assert qo.is_contiguous() and ko.is_contiguous()
    assert_bf16_close(N(qo), oracle.rmsnorm(N(q), N(qw), 1e-6), what="q norm")
    assert_bf16_close(N(ko), oracle.rmsnorm(N(k), N(kw), 1e-6), what="k norm")


def test_qk_rmsnorm_inplace_decode_shape(dev):
    c = wl.cfg5(B=256, V=16)
    qkv = c["qkv"].to(dev)
    q, k, _ = wl.split_qkv(qkv, 32, 8, 128)
    wq = oracle.rmsnorm(N(q), N(c["q_norm"]), 1e-6)
    wk = oracle.rmsnorm(N(k), N(c["k_norm"]), 1e-6)
    ops.qk_rms_norm(q, k, c["q_norm"].to(dev), c["k_norm"].to(dev), 1e-6, q_out=q, k_out=k)
    assert_bf16_close(N(q), wq, what="q in place")
    assert_bf16_close(N(k), wk, what="k in place")


def test_rmsnorm_per_head_3d(dev):
    x = wl.normal((5, 6, 128), 12).to(dev)
    w = wl.normal((128,), 13, 1.0, 0.1).to(dev)
    y = ops.rmsnorm(x, w, 1e-6)
    assert_bf16_close(N(y), oracle.rmsnorm(N(x), N(w), 1e-6), what="3d per-head")
