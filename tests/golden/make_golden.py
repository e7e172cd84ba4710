"""Writes the golden fixtures tests/golden/*.npz (run: python tests/golden/make_golden.py).

Each fixture holds seeded inputs and expected outputs computed WITHOUT the oracle:
  rmsnorm, add_rmsnorm, qk_norm, silu_mul, embed: torch-CPU running the reference's own
    expressions (F.rms_norm, `r + x`, F.silu(g) * u, F.embedding; llama3.py:555, :586,
    :569-572, :471; qwen3.py:651-662) — the reference implementation of these ops;
  rope_llama31, rope_std: HF rotate-half applied in float64 with transformers' Llama-3
    frequency rule (flashinfer, the reference's RoPE, is not installable here);
  append, index: brute-force Python loops restating
    pie/src/flashinfer_metal/kernels/metal_append_paged_kv_cache.metal:51-103 and
    pie/src/flashinfer_metal/ops.py:392-436.
bf16 tensors are stored as uint16 bit patterns. Seeds and shapes are in each file.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from pie_amd import workloads as wl  # noqa: E402

def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def save(name: str, **arrs):
    np.savez_compressed(HERE / f"{name}.npz", **arrs)


def hf_inv_freq_llama3(D, theta, factor, lo, hi, L):
    from transformers import LlamaConfig
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    cfg = LlamaConfig(hidden_size=D * 4, num_attention_heads=4, head_dim=D,
                      rope_parameters=dict(rope_type="llama3", rope_theta=theta, factor=factor,
                                           low_freq_factor=lo, high_freq_factor=hi,
                                           original_max_position_embeddings=L))
    return ROPE_INIT_FUNCTIONS["llama3"](cfg, "cpu")[0].double()


def hf_rope(x: torch.Tensor, pos: torch.Tensor, inv_freq: torch.Tensor) -> torch.Tensor:
    x = x.double()
    ang = pos.double()[:, None] * inv_freq[None, :]
    cos = torch.cat([torch.cos(ang)] * 2, -1)[:, None, :]
    sin = torch.cat([torch.sin(ang)] * 2, -1)[:, None, :]
    h = x.shape[-1] // 2
    return (x * cos + torch.cat([-x[..., h:], x[..., :h]], -1) * sin).float().to(torch.bfloat16)


def main():
    # a1 RMSNorm (configuration 1 shape family, fewer rows)
    x, w = wl.normal((64, 2048), 101), wl.normal((2048,), 102, 1.0, 0.1)
    save("rmsnorm", x=bits(x), w=bits(w), eps=1e-5, y=bits(F.rms_norm(x, [2048], w, 1e-5)),
         seeds=[101, 102])
    # a2 residual add + RMSNorm
    x, r, w = wl.normal((24, 4096), 103), wl.normal((24, 4096), 104), wl.normal((4096,), 105, 1.0, 0.1)
    s = r + x
    save("add_rmsnorm", x=bits(x), r=bits(r), w=bits(w), eps=1e-5, s=bits(s),
         y=bits(F.rms_norm(s, [4096], w, 1e-5)), seeds=[103, 104, 105])
    # a3 per-head q/k RMSNorm on views of a qkv projection (Qwen3-8B heads)
    qkv = wl.normal((8, 48 * 128), 106)
    q, k, _ = wl.split_qkv(qkv, 32, 8, 128)
    qw, kw = wl.normal((128,), 107, 1.0, 0.1), wl.normal((128,), 108, 1.0, 0.1)
    save("qk_norm", qkv=bits(qkv), qw=bits(qw), kw=bits(kw), eps=1e-6,
         q=bits(F.rms_norm(q, [128], qw, 1e-6)), k=bits(F.rms_norm(k, [128], kw, 1e-6)),
         seeds=[106, 107, 108])
    # a4 SiLU-and-mul
    gu = wl.normal((16, 2 * 1024), 109, 0.0, 2 ** 0.5)
    g, u = torch.split(gu, [1024, 1024], -1)
    save("silu_mul", gate_up=bits(gu), out=bits(F.silu(g) * u), seeds=[109])
    # a5 embedding with repeats
    c = wl.cfg4(V=512, H=256, T=200)
    save("embed", W=bits(c["W"]), ids=c["ids"].numpy(), out=bits(F.embedding(c["ids"], c["W"])))
    # a6 Llama-3.1 RoPE on a ragged batch
    lens = torch.tensor([5, 1, 9], dtype=torch.int32)
    pos = torch.cat([torch.arange(n) + 3000 * i for i, n in enumerate(lens.tolist())]).to(torch.int32)
    T = int(lens.sum())
    q, k = wl.normal((T, 4, 128), 110), wl.normal((T, 2, 128), 111)
    f = hf_inv_freq_llama3(128, 5e5, 8.0, 1.0, 4.0, 8192)
    save("rope_llama31", q=bits(q), k=bits(k), pos=pos.numpy(), params=[8.0, 5e5, 1.0, 4.0, 8192],
         q_out=bits(hf_rope(q, pos, f)), k_out=bits(hf_rope(k, pos, f)), seeds=[110, 111])
    # a7 standard RoPE (theta 1e6)
    f = 1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float64) / 128))
    save("rope_std", q=bits(q), k=bits(k), pos=pos.numpy(), theta=1e6,
         q_out=bits(hf_rope(q, pos, f)), k_out=bits(hf_rope(k, pos, f)))
    # a8 paged append (NHD), sentinel-filled cache, one skipped token
    pb = wl.paged_batch(torch.tensor([3, 17, 0], dtype=torch.int32),
                        torch.tensor([6, 2, 20], dtype=torch.int32), 16, 12, 112)
    T = int(pb.lens.sum())
    kk, vv = wl.normal((T, 2, 64), 113), wl.normal((T, 2, 64), 114)
    bidx = pb.batch_indices.clone()
    bidx[3] = 9  # out-of-range batch index: skipped
    cache = wl.sentinel_cache((12, 2, 16, 2, 64))
    want = cache.clone()
    for t in range(T):
        b, p = int(bidx[t]), int(pb.positions[t])
        if not 0 <= b < 3:
            continue
        lg = int(pb.kv_indptr[b]) + p // 16
        if lg >= int(pb.kv_indptr[b + 1]):
            continue
        page = int(pb.kv_indices[lg])
        want[page, 0, p % 16] = kk[t]
        want[page, 1, p % 16] = vv[t]
    save("append", k=bits(kk), v=bits(vv), batch_indices=bidx.numpy(), positions=pb.positions.numpy(),
         kv_indices=pb.kv_indices.numpy(), kv_indptr=pb.kv_indptr.numpy(),
         kv_last_page_len=pb.kv_last_page_len.numpy(), cache_in=bits(cache), cache_out=bits(want))
    # a9 index helpers (one empty request)
    indptr = np.array([0, 2, 2, 7, 8], np.int32)
    last = np.array([5, 16, 1, 16], np.int32)
    sl = np.array([(indptr[i + 1] - indptr[i] - 1) * 16 + last[i] if indptr[i + 1] > indptr[i] else 0
                   for i in range(4)], np.int32)
    qo = np.array([0, 3, 3, 4, 20], np.int32)
    bi = np.zeros(20, np.int32)
    po = np.zeros(20, np.int32)
    for b in range(4):
        for j, t in enumerate(range(qo[b], qo[b + 1])):
            bi[t] = b
            po[t] = sl[b] - (qo[b + 1] - qo[b]) + j
    save("index", kv_indptr=indptr, last_page_len=last, page_size=16, seq_lens=sl, qo_indptr=qo,
         batch_indices=bi, positions=po)
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
