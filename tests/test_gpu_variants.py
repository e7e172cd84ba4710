"""GPU parity for the model-family variants of the fused ops: Gemma RMSNorm (plain, residual-add,
per-head q/k), GELU-tanh-and-mul, the scaled embedding gather, and RoPE from a precomputed
cos/sin table (flashinfer.apply_rope_with_cos_sin_cache_inplace).

Tolerances: the residual sum and the embedding gather are bit-exact. GELU and the cos/sin-table
RoPE are within 1e-2 rel / 2e-2 abs of the oracle. Gemma RMSNorm is bit-exact: the kernel sums the
bf16 squares in fp64 (exact in any order, as the oracle's sum is), rounds the mean straight to
bf16, and takes the rsqrt in fp64, so every bf16 step rounds the same exact value as the
oracle's."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from pie_amd import ops
from pie_amd import workloads as wl
from tests._util import assert_bf16_close, assert_bits_equal

pytestmark = pytest.mark.gpu
N = oracle.to_np


@pytest.mark.parametrize("T,H", [(1, 2304), (33, 3584), (7, 256), (5, 100), (0, 2304), (64, 5376), (2048, 3584)])
def test_gemma_rms_norm(dev, T, H):
    print(f"gemma_rms_norm T={T} H={H}", flush=True)
    x, w = wl.normal((T, H), 41), wl.normal((H,), 42, 0.0, 0.5)
    out = ops.gemma_rms_norm(x.to(dev), w.to(dev), 1e-6)
    torch.cuda.synchronize()
    assert_bits_equal(N(out), oracle.gemma_rmsnorm(N(x), N(w), 1e-6), f"gemma {T}x{H}")


@pytest.mark.parametrize("T,H", [(8192, 4096), (16384, 2304)])
def test_gemma_rms_norm_large_row_lists(dev, T, H):
    """Row lists past 64 MB take the row-prefetching kernel (rows_pf): bit-exact on the full
    output."""
    print(f"gemma_rms_norm large T={T} H={H}", flush=True)
    x, w = wl.normal((T, H), 43), wl.normal((H,), 44, 0.0, 0.5)
    out = ops.gemma_rms_norm(x.to(dev), w.to(dev), 1e-6)
    torch.cuda.synchronize()
    assert_bits_equal(N(out), oracle.gemma_rmsnorm(N(x), N(w), 1e-6), f"gemma {T}x{H}")


def test_gemma_rms_norm_mean_near_midpoint(dev):
    """The correctly rounded mean of the squares at and just above a bf16 rounding midpoint, on
    the row-prefetching kernel (64 MiB of rows): rows whose exact mean is a midpoint (a quarter
    1.0078125, the rest 1.0: squares 1.015625 and 1.0, mean 1.00390625, a tie that rounds to
    1.0) or sits 2^-18 above it (one more 1.0078125: rounds to 1.0078125) among ordinary rows;
    bit-exact on the full output, and the two kinds of rows differ."""
    T, H = 8192, 4096  # 64 MiB of rows: the row-prefetching kernel
    x = wl.normal((T, H), 45)
    special = (0, 1, 4095, 8191)
    for r in special:
        x[r] = 1.0
        x[r, : H // 4 + (r % 2)] = 1.0078125  # odd rows: the mean 2^-18 above the midpoint
        x[r, 1::2] = -x[r, 1::2]
    w = wl.normal((H,), 46, 0.0, 0.5)
    out = ops.gemma_rms_norm(x.to(dev), w.to(dev), 0.0)
    torch.cuda.synchronize()
    want = oracle.gemma_rmsnorm(N(x), N(w), 0.0)
    assert_bits_equal(N(out), want, "gemma near-midpoint means")
    wf = oracle.bf16_to_f32(want)
    assert not np.array_equal(wf[0, H - 2:], wf[1, H - 2:]), "the tie and the row above it round apart"


def test_gemma_rms_norm_every_scale(dev):
    """Rows of one repeated value a, eps = 0: the variance is bf16(a^2) and the kernel's rsqrt
    meets t = bf16(a^2) for every bf16 a in [2^-40, 2^40) (10240 rows), so every correction step
    of its correctly rounded rsqrt and mean is exercised; bit-exact against the oracle."""
    bits = np.arange(0x3F80 - 40 * 128, 0x3F80 + 40 * 128, dtype=np.uint16)
    a = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
    x = a[:, None].expand(-1, 512).contiguous()
    x[:, 1::2] = -x[:, 1::2]
    w = wl.normal((512,), 55, 0.0, 0.5)
    out = ops.gemma_rms_norm(x.to(dev), w.to(dev), 0.0)
    torch.cuda.synchronize()
    assert_bits_equal(N(out), oracle.gemma_rmsnorm(N(x), N(w), 0.0), "gemma every scale")


@pytest.mark.parametrize("T,H", [(3, 2304), (40, 3584), (2, 100)])
def test_gemma_add_rms_norm(dev, T, H):
    print(f"gemma_add_rms_norm T={T} H={H}", flush=True)
    x, r = wl.normal((T, H), 43), wl.normal((T, H), 44, 0.0, 4.0)
    w = wl.normal((H,), 45, 0.0, 0.5)
    y, s = ops.gemma_add_rms_norm(x.to(dev), r.to(dev), w.to(dev), 1e-6)
    torch.cuda.synchronize()
    wy, ws = oracle.gemma_add_rmsnorm(N(x), N(r), N(w), 1e-6)
    assert_bits_equal(N(s), ws, "gemma residual sum")
    assert_bits_equal(N(y), wy, f"gemma add {T}x{H}")


@pytest.mark.parametrize("T,Hq,Hkv,D", [(9, 8, 4, 256), (4, 16, 8, 128), (3, 2, 1, 64)])
def test_gemma_qk_rms_norm(dev, T, Hq, Hkv, D):
    print(f"gemma_qk_rms_norm T={T} Hq={Hq} Hkv={Hkv} D={D}", flush=True)
    qkv = wl.normal((T, (Hq + 2 * Hkv) * D), 46)
    q, k, _ = wl.split_qkv(qkv, Hq, Hkv, D)
    qw, kw = wl.normal((D,), 47, 0.0, 0.5), wl.normal((D,), 48, 0.0, 0.5)
    qo, ko = ops.gemma_qk_rms_norm(q.to(dev), k.to(dev), qw.to(dev), kw.to(dev), 1e-6)
    torch.cuda.synchronize()
    assert_bits_equal(N(qo), oracle.gemma_rmsnorm(N(q), N(qw), 1e-6), "gemma q")
    assert_bits_equal(N(ko), oracle.gemma_rmsnorm(N(k), N(kw), 1e-6), "gemma k")


@pytest.mark.parametrize("T,I", [(1, 8), (17, 9216), (64, 14336), (5, 13), (0, 64)])
def test_gelu_tanh_and_mul(dev, T, I):
    print(f"gelu_tanh_and_mul T={T} I={I}", flush=True)
    gu = wl.normal((T, 2 * I), 49, 0.0, 2 ** 0.5)
    out = ops.gelu_tanh_and_mul(gu.to(dev))
    torch.cuda.synchronize()
    assert_bf16_close(N(out), oracle.gelu_tanh_and_mul(N(gu)), what=f"gelu {T}x{I}")


@pytest.mark.parametrize("V,H,T", [(1000, 2304, 50), (300, 100, 40), (10, 3584, 0)])
def test_embedding_scaled(dev, V, H, T):
    print(f"embedding scaled V={V} H={H} T={T}", flush=True)
    c = wl.cfg4(V=V, H=H, T=T)
    ids = c["ids"].clone()
    if T > 2:
        ids[1], ids[2] = V, -1          # out of range: zero rows
    scale = float(torch.tensor(math.sqrt(H), dtype=torch.float32))
    out = ops.embedding(ids.to(dev), c["W"].to(dev), scale=scale)
    want, _ = oracle.embedding_scaled(N(ids), N(c["W"]), scale)
    assert_bits_equal(N(out).reshape(T, H), want, "scaled embedding")


def _yarn_like_table(rows, rd, seed):
    """A [rows, rd] fp32 cos/sin table (cos in the first half) with irregular frequencies, like the
    YaRN tables gpt_oss.py:520-547 builds; any table is valid input."""
    g = torch.Generator().manual_seed(seed)
    inv = (1e4 ** (-torch.arange(0, rd, 2, dtype=torch.float64) / rd)) * (0.5 + torch.rand(rd // 2, generator=g, dtype=torch.float64))
    ang = torch.arange(rows, dtype=torch.float64)[:, None] * inv[None, :]
    return torch.cat([ang.cos(), ang.sin()], -1).float()


@pytest.mark.parametrize("T,Hq,Hkv,D,rd,neox", [(37, 64, 8, 64, 64, True), (20, 4, 2, 128, 64, True),
                                                (11, 4, 2, 128, 128, False), (5, 3, 1, 32, 24, True)])
def test_rope_cos_sin_cache(dev, T, Hq, Hkv, D, rd, neox):
    print(f"rope cos_sin_cache T={T} Hq={Hq} Hkv={Hkv} D={D} rd={rd} neox={neox}", flush=True)
    rows = 4096
    cs = _yarn_like_table(rows, rd, 50)
    qkv = wl.normal((T, (Hq + 2 * Hkv) * D), 51)
    pos = torch.randint(0, rows, (T,), generator=torch.Generator().manual_seed(52), dtype=torch.int32)
    pos[0] = rows                        # outside the table: left unrotated
    q, k, _ = wl.split_qkv(qkv, Hq, Hkv, D)
    wq, wk = oracle.rope_cos_sin(N(q), N(k), N(pos), N(cs), interleave=not neox)
    qd, kd = q.contiguous().to(dev), k.contiguous().to(dev)
    ops.apply_rope_with_cos_sin_cache_inplace(pos.to(dev), qd.view(T, -1), kd.view(T, -1), D,
                                              cs.to(dev), is_neox=neox)
    torch.cuda.synchronize()
    assert_bf16_close(N(qd), wq, what="q")
    assert_bf16_close(N(kd), wk, what="k")
    assert_bits_equal(N(qd)[0], N(q)[0], "token outside the table")


def test_rope_cos_sin_cache_equals_frequency_rope(dev):
    """A table built from the standard inv_freq rotates like apply_rope_pos_ids_inplace."""
    T, Hq, Hkv, D = 30, 8, 2, 128
    inv = torch.from_numpy(np.asarray(oracle.inv_freq_std(D, 1.0, 1e4), dtype=np.float64))
    ang = torch.arange(2048, dtype=torch.float64)[:, None] * inv[None, :].float().double()
    cs = torch.cat([ang.cos(), ang.sin()], -1).float()
    qkv = wl.normal((T, (Hq + 2 * Hkv) * D), 53)
    q, k, _ = wl.split_qkv(qkv, Hq, Hkv, D)
    pos = torch.randint(0, 2048, (T,), generator=torch.Generator().manual_seed(54), dtype=torch.int32)
    qa, ka = q.contiguous().to(dev), k.contiguous().to(dev)
    qb, kb = qa.clone(), ka.clone()
    ops.apply_rope_with_cos_sin_cache_inplace(pos.to(dev), qa, ka, D, cs.to(dev))
    ops.apply_rope_pos_ids_inplace(qb, kb, pos.to(dev), rope_theta=1e4)
    torch.cuda.synchronize()
    assert_bf16_close(N(qa), N(qb), what="q table vs frequencies")
    assert_bf16_close(N(ka), N(kb), what="k table vs frequencies")
