"""Seeded synthetic inputs for the benchmark configurations of the per-layer hot path.

Each builder returns CPU tensors (bf16 activations, int32 indices) generated in fp32 with
``torch.Generator().manual_seed(seed)`` and cast, so the CPU checker, the CPU timing and
the GPU kernels all see identical bytes. Sizes default to the full configurations; keyword
arguments shrink them for parity tests.

  cfg1  RMSNorm [2048, 2048], eps 1e-5                                (Llama-3.2-1B layer)
  cfg2  residual-add + RMSNorm [8192, 4096] eps 1e-5, SiLU-and-mul [8192, 2x14336] (Llama-3-8B)
  cfg3  Llama-3.1 RoPE + paged append: 64 ragged requests, Hq 32 / Hkv 8 / D 128, page 16,
        pool 8192 pages, q/k/v as views of one [T, 6144] qkv projection
  cfg4  embedding gather [128256, 4096] with 16384 ids (10% repeats)
  cfg5  Qwen3-8B decode chain, 256 sequences x 1 token, contexts U[128, 4096]
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

BF16 = torch.bfloat16
SENTINEL_BITS = 0x7FA5  # a NaN pattern no kernel produces: marks untouched cache bytes


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def normal(shape, seed: int, mean: float = 0.0, std: float = 1.0) -> torch.Tensor:
    return (torch.randn(shape, generator=_gen(seed)) * std + mean).to(BF16)


def sentinel_cache(shape) -> torch.Tensor:
    return torch.full(shape, SENTINEL_BITS, dtype=torch.int16).view(BF16)


# ----------------------------------------------------------------------------- configs 1, 2
def cfg1(T: int = 2048, H: int = 2048) -> dict:
    return {"x": normal((T, H), 1), "w": normal((H,), 2, 1.0, 0.1), "eps": 1e-5}


def cfg2(T: int = 8192, H: int = 4096, I: int = 14336) -> dict:
    return {
        "r": normal((T, H), 3), "x": normal((T, H), 4), "w": normal((H,), 5, 1.0, 0.1),
        "eps": 1e-5,
        # N(0, 2) read as variance 2: std sqrt(2)
        "gate_up": normal((T, 2 * I), 6, 0.0, math.sqrt(2.0)),
    }


def cfg2_bytes(T: int = 8192, H: int = 4096, I: int = 14336) -> tuple[int, int]:
    """Algorithmic HBM bytes: (add+RMSNorm, SiLU-and-mul)."""
    return 4 * T * H * 2 + H * 2, T * 2 * I * 2 + T * I * 2


# ----------------------------------------------------------------------------- config 3
@dataclass
class PagedBatch:
    lens: torch.Tensor          # [B] tokens appended per request
    qo_indptr: torch.Tensor     # [B+1]
    kv_indptr: torch.Tensor     # [B+1] pages per request
    kv_indices: torch.Tensor    # [sum pages] physical page ids
    kv_last_page_len: torch.Tensor  # [B]
    positions: torch.Tensor     # [T] position of each appended token
    batch_indices: torch.Tensor  # [T]
    seq_lens: torch.Tensor      # [B] total length after the append
    num_pages: int
    page_size: int
    extra: dict = field(default_factory=dict)


def paged_batch(ctx_before: torch.Tensor, new_tokens: torch.Tensor, page_size: int,
                pool_pages: int, perm_seed: int) -> PagedBatch:
    """Page tables for requests holding ctx_before[b] cached tokens and appending
    new_tokens[b]; pages are a random permutation of the pool."""
    B = ctx_before.numel()
    total = ctx_before + new_tokens
    npages = (total + page_size - 1) // page_size
    need = int(npages.sum())
    if need > pool_pages:
        raise ValueError(f"pool of {pool_pages} pages cannot hold {need}")
    perm = torch.randperm(pool_pages, generator=_gen(perm_seed)).to(torch.int32)
    kv_indptr = torch.zeros(B + 1, dtype=torch.int32)
    kv_indptr[1:] = torch.cumsum(npages, 0).to(torch.int32)
    kv_indices = perm[:need].clone()
    last = (total - page_size * (npages - 1)).to(torch.int32)
    last[npages == 0] = 0
    qo = torch.zeros(B + 1, dtype=torch.int32)
    qo[1:] = torch.cumsum(new_tokens, 0).to(torch.int32)
    T = int(qo[-1])
    bidx = torch.repeat_interleave(torch.arange(B, dtype=torch.int32), new_tokens.to(torch.int64))
    starts = qo[:-1].to(torch.int64)[bidx.to(torch.int64)]
    pos = (ctx_before.to(torch.int64)[bidx.to(torch.int64)] + torch.arange(T) - starts).to(torch.int32)
    return PagedBatch(new_tokens.to(torch.int32), qo, kv_indptr, kv_indices, last, pos, bidx,
                      total.to(torch.int32), pool_pages, page_size)


def cfg3(B: int = 64, max_len: int = 2048, Hq: int = 32, Hkv: int = 8, D: int = 128,
         page_size: int = 16, pool_pages: int = 8192) -> dict:
    lens = torch.randint(1, max_len + 1, (B,), generator=_gen(7)).to(torch.int32)
    pb = paged_batch(torch.zeros(B, dtype=torch.int32), lens, page_size, pool_pages, 11)
    T = int(lens.sum())
    qkv = torch.empty((T, (Hq + 2 * Hkv) * D), dtype=BF16)
    qkv[:, : Hq * D] = normal((T, Hq * D), 8)
    qkv[:, Hq * D:(Hq + Hkv) * D] = normal((T, Hkv * D), 9)
    qkv[:, (Hq + Hkv) * D:] = normal((T, Hkv * D), 10)
    return {
        "qkv": qkv, "Hq": Hq, "Hkv": Hkv, "D": D, "batch": pb,
        "cache_shape": (pool_pages, 2, page_size, Hkv, D),
        "rope": dict(rope_scale=8.0, rope_theta=5e5, low_freq_factor=1.0, high_freq_factor=4.0,
                     old_context_len=8192),
    }


def split_qkv(qkv: torch.Tensor, Hq: int, Hkv: int, D: int):
    """q, k, v as strided views of the fused projection (llama3.py:633-657)."""
    T = qkv.shape[0]
    q, k, v = torch.split(qkv, [Hq * D, Hkv * D, Hkv * D], dim=-1)
    return q.view(T, Hq, D), k.view(T, Hkv, D), v.view(T, Hkv, D)


def cfg3_bytes(T: int, Hq: int = 32, Hkv: int = 8, D: int = 128) -> dict:
    """Algorithmic bytes of rope (q, k read+write + pos), append (k, v read + write, bidx/pos),
    and the fused pass (rotated k goes to the cache from registers)."""
    rope = T * (2 * 2 * (Hq + Hkv) * D + 4)
    append = T * (2 * 2 * 2 * Hkv * D + 8)
    fused = T * (2 * 2 * Hq * D + 3 * 2 * Hkv * D + 2 * 2 * Hkv * D + 12)
    return {"rope": rope, "append": append, "fused": fused}


# ----------------------------------------------------------------------------- config 4
def cfg4(V: int = 128256, H: int = 4096, T: int = 16384, repeat_frac: float = 0.1) -> dict:
    n_rep = int(round(T * repeat_frac))
    n_uni = T - n_rep
    g = _gen(13)
    uni = torch.randint(0, V, (n_uni,), generator=g)
    rep = uni[torch.randint(0, max(n_uni, 1), (n_rep,), generator=g)] if n_uni else uni
    ids = torch.cat([uni, rep])[torch.randperm(T, generator=g)].to(torch.int32)
    return {"W": normal((V, H), 12, 0.0, 0.02), "ids": ids}


def cfg4_bytes(T: int = 16384, H: int = 4096) -> int:
    return 2 * T * H * 2 + T * 4


# ----------------------------------------------------------------------------- config 5
def cfg5(B: int = 256, V: int = 151936, H: int = 4096, Hq: int = 32, Hkv: int = 8, D: int = 128,
         I: int = 12288, page_size: int = 16, ctx_lo: int = 128, ctx_hi: int = 4096) -> dict:
    ctx = torch.randint(ctx_lo, ctx_hi + 1, (B,), generator=_gen(14)).to(torch.int32)
    pool = int(((ctx + 1 + page_size - 1) // page_size).sum())
    pb = paged_batch(ctx, torch.ones(B, dtype=torch.int32), page_size, pool, 15)
    return {
        "W": normal((V, H), 16), "ids": torch.randint(0, V, (B,), generator=_gen(17)).to(torch.int32),
        "residual": normal((B, H), 18), "w_norm": normal((H,), 19),
        "qkv": normal((B, (Hq + 2 * Hkv) * D), 20), "q_norm": normal((D,), 21),
        "k_norm": normal((D,), 22), "gate_up": normal((B, 2 * I), 23),
        "batch": pb, "cache_shape": (pool, 2, page_size, Hkv, D), "eps": 1e-6, "theta": 1e6,
        "Hq": Hq, "Hkv": Hkv, "D": D, "I": I, "H": H,
    }


def cfg5_bytes(B: int = 256, H: int = 4096, Hq: int = 32, Hkv: int = 8, D: int = 128,
               I: int = 12288) -> dict:
    return {
        "embedding": 2 * B * H * 2 + B * 4,
        "add_rmsnorm": 4 * B * H * 2 + H * 2,
        "qk_rmsnorm": 2 * B * (Hq + Hkv) * D * 2 + 2 * D * 2,
        "rope": B * (2 * 2 * (Hq + Hkv) * D + 4),
        "append": B * (2 * 2 * 2 * Hkv * D + 8),
        "silu_and_mul": B * 2 * I * 2 + B * I * 2,
    }


# ----------------------------------------------------------------------------- paged attention
def attn_batch(ctx_before, new_tokens, Hq: int = 32, Hkv: int = 8, D: int = 128,
               page_size: int = 16, pool_pages: int | None = None, seed: int = 30,
               layout: str = "NHD") -> dict:
    """Paged attention inputs: requests holding ctx_before[b] cached tokens and ending with
    new_tokens[b] query tokens (whose k/v are already in the cache, as after the append of
    llama3.py:675-685). The cache is filled with N(0,1) everywhere, q [T, Hq, D] ~ N(0,1)."""
    ctx_before = torch.as_tensor(ctx_before, dtype=torch.int32)
    new_tokens = torch.as_tensor(new_tokens, dtype=torch.int32)
    total = ctx_before + new_tokens
    need = int(((total + page_size - 1) // page_size).sum())
    pool = need if pool_pages is None else pool_pages
    pb = paged_batch(ctx_before, new_tokens, page_size, pool, seed + 1)
    T = int(new_tokens.sum())
    shape = (pool, 2, page_size, Hkv, D) if layout == "NHD" else (pool, 2, Hkv, page_size, D)
    return {"q": normal((T, Hq, D), seed + 2), "cache": normal(shape, seed + 3), "batch": pb,
            "Hq": Hq, "Hkv": Hkv, "D": D, "layout": layout}


def attn_decode_cfg(B: int = 256, ctx_lo: int = 128, ctx_hi: int = 4096, **kw) -> dict:
    """Decode attention at the Qwen3-8B decode-chain shape: B sequences x 1 query token over
    contexts U[ctx_lo, ctx_hi] (the same draw as cfg5), Hq 32 / Hkv 8 / D 128, page 16."""
    ctx = torch.randint(ctx_lo, ctx_hi + 1, (B,), generator=_gen(14)).to(torch.int32)
    return attn_batch(ctx, torch.ones(B, dtype=torch.int32), seed=40, **kw)


def attn_prefill_cfg(B: int = 64, max_len: int = 2048, **kw) -> dict:
    """Causal prefill attention over cfg3's ragged batch (64 requests, lengths U[1, 2048], the
    same draw), Llama-3-8B heads (Hq 32 / Hkv 8 / D 128), page 16."""
    lens = torch.randint(1, max_len + 1, (B,), generator=_gen(7)).to(torch.int32)
    return attn_batch(torch.zeros(B, dtype=torch.int32), lens, seed=50, **kw)


def attn_bytes(pb: PagedBatch, Hq: int, Hkv: int, D: int) -> int:
    """Algorithmic HBM bytes of one attention call: q read + out written once, every cached
    k/v row of every request read once, plus the page table and indptr arrays."""
    T = int(pb.qo_indptr[-1])
    kv_tokens = int(pb.seq_lens.sum())
    B = pb.seq_lens.numel()
    return (2 * T * Hq * D * 2 + kv_tokens * Hkv * D * 2 * 2 + pb.kv_indices.numel() * 4
            + (3 * B + 2) * 4)


def attn_flops(pb: PagedBatch, Hq: int, D: int, causal: bool = True) -> int:
    """Useful flops (QK^T and PV, 2 per multiply-add) over the causal window."""
    qo = (pb.qo_indptr[1:] - pb.qo_indptr[:-1]).to(torch.int64)
    kv = pb.seq_lens.to(torch.int64)
    if causal:  # query i sees kv - qo + i + 1 positions
        pairs = (qo * (kv - qo) + qo * (qo + 1) // 2).sum()
    else:
        pairs = (qo * kv).sum()
    return int(pairs) * Hq * D * 4
