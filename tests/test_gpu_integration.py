"""GPU: the routes that put this package's kernels under Pie's model files without editing them:
``install_functional`` (the model modules' ``fun`` = torch.nn.functional binding, llama3.py:7)
for rms_norm and embedding, and ``patch_mlp`` for a Llama-style ForwardPass.mlp
(llama3.py:543-586). The routed calls must equal the direct pie_amd ops bit for bit (so the HIP
kernels ran) and the oracle / a float32 torch restatement within tolerance."""
from __future__ import annotations

import types

import pytest
import torch
import torch.nn.functional as F

import oracle
from pie_amd import integration, ops
from pie_amd import workloads as wl
from tests._util import assert_bf16_close, assert_bits_equal

pytestmark = pytest.mark.gpu
N = oracle.to_np


def _model_module():
    m = types.ModuleType("fake_model")
    m.fun = F
    return m


def test_functional_rms_norm_and_embedding(dev):
    m = _model_module()
    integration.install_functional(m)
    try:
        assert m.fun.linear is F.linear  # GEMMs stay torch's
        x, w = wl.normal((64, 4096), 1).to(dev), wl.normal((4096,), 2, 1.0, 0.1).to(dev)
        y = m.fun.rms_norm(x, normalized_shape=[4096], weight=w, eps=1e-5)
        assert_bits_equal(N(y), N(ops.rms_norm(x, [4096], w, 1e-5)), "routed rms_norm")
        assert_bf16_close(N(y), oracle.rmsnorm(N(x.cpu()), N(w.cpu()), 1e-5), what="rms_norm")
        # per-head form of qwen3.py:651-662: q [T, Hq, D] view of the qkv projection
        qkv = wl.normal((16, 48 * 128), 3).to(dev)
        q = qkv[:, : 32 * 128].view(16, 32, 128)
        qw = wl.normal((128,), 4, 1.0, 0.1).to(dev)
        qn = m.fun.rms_norm(q, normalized_shape=[128], weight=qw, eps=1e-6)
        assert_bf16_close(N(qn), oracle.rmsnorm(N(q.cpu()), N(qw.cpu()), 1e-6), what="q norm")
        W = wl.normal((1000, 4096), 5).to(dev)
        ids = torch.randint(0, 1000, (33,), generator=torch.Generator().manual_seed(6))
        for dt in (torch.int32, torch.int64):
            e = m.fun.embedding(ids.to(dt).to(dev), W)
            assert_bits_equal(N(e), N(W[ids.long().to(dev)]), f"embedding {dt}")
        with pytest.raises(NotImplementedError):
            m.fun.embedding(ids.to(dev), W, padding_idx=0)
        with pytest.raises(ValueError):  # a GPU dtype the kernels do not serve is not rerouted
            m.fun.rms_norm(x.float(), [4096], w.float(), 1e-5)
    finally:
        integration.uninstall_functional(m)
    assert m.fun is F


class _Cfg:
    dim_hidden, dim_mlp, rms_norm_eps = 1024, 2816, 1e-5


class _ForwardPass:
    """The attributes a Llama-style ForwardPass.mlp reads (llama3.py:543-586)."""

    def __init__(self, weights):
        self.model_config = _Cfg()
        self.weights = weights
        self.tp_size = 1

    def mlp(self, hidden_states, layer_idx):
        raise AssertionError("unpatched mlp called")


def test_patch_mlp_matches_fp32_restatement(dev):
    H, I = _Cfg.dim_hidden, _Cfg.dim_mlp
    w = {"layers.0.norm_mlp": wl.normal((H,), 7, 1.0, 0.1).to(dev),
         "layers.0.proj_gate_up": (wl.normal((2 * I, H), 8).float() * 0.05).bfloat16().to(dev),
         "layers.0.proj_down": (wl.normal((H, I), 9).float() * 0.05).bfloat16().to(dev)}
    fp = _ForwardPass(w)
    integration.patch_mlp(_ForwardPass)
    try:
        h = wl.normal((40, H), 10).to(dev)
        got = fp.mlp(h, 0).float()
        f = {k: v.float() for k, v in w.items()}
        x = h.float()
        n = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + _Cfg.rms_norm_eps) * f["layers.0.norm_mlp"]
        gate, up = (n @ f["layers.0.proj_gate_up"].T).split([I, I], -1)
        want = x + (F.silu(gate) * up) @ f["layers.0.proj_down"].T
        err = (got - want).abs().max().item()
        assert err <= 0.03 * want.abs().max().item(), err
    finally:
        integration.unpatch_mlp(_ForwardPass)
    with pytest.raises(AssertionError, match="unpatched"):
        fp.mlp(h, 0)
