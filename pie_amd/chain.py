"""The decode-step op chain of one Qwen3 layer (benchmark configuration 5).

Runs the hot-path ops of a decode step in model order, with the GEMMs and attention left
out (they are not part of this path):
  (1) embedding gather            qwen3.py:468-472
  (2) residual add + RMSNorm      qwen3.py:571 -> :538
  (3) per-head q/k RMSNorm        qwen3.py:651-662
  (4) RoPE at each sequence's position and (5) paged-KV append   qwen3.py:665-684
      (fused=True runs (3)-(5) as one kernel, fused=False as three launches)
  (6) SiLU-and-mul                qwen3.py:553-556
grouped=True (implies the fused prologue) records the ops in ops.op_group(), so the whole chain
is ONE kernel launch: the embedding gather runs fused into the residual add + RMSNorm, and the
q/k prologue and SiLU-and-mul, which do not depend on them here, run in their own block ranges.
saved=True (implies grouped) records the group once (ops.saved_group()) and relaunches it on
every later ``run()`` with one library call, as a decode loop without graphs would.
All buffers are preallocated, so ``run()`` launches kernels only and can be captured into a
HIP graph (``capture()``), as the reference captures its decode layers (llama3.py:315-414).
"""
from __future__ import annotations

import torch

from . import ops
from . import workloads as wl


class DecodeChain:
    def __init__(self, cfg: dict, device, fused: bool = True, grouped: bool = False,
                 share: "DecodeChain | None" = None, saved: bool = False):
        """share: take the embedding table and the paged cache of another chain (several chains
        over their own activations, as the layers of one decode step share a cache pool)."""
        d = device
        self.cfg = cfg
        self.fused = fused or grouped or saved
        self.grouped = grouped or saved
        self.saved = saved
        self._saved = None
        self.Hq, self.Hkv, self.D = cfg["Hq"], cfg["Hkv"], cfg["D"]
        self.eps, self.theta = cfg["eps"], cfg["theta"]
        pb = cfg["batch"]
        self.W = share.W if share is not None else cfg["W"].to(d)
        self.ids = cfg["ids"].to(d)
        self.residual0 = cfg["residual"].to(d)
        self.residual = self.residual0.clone()
        self.w_norm = cfg["w_norm"].to(d)
        self.qkv0 = cfg["qkv"].to(d)
        self.qkv = self.qkv0.clone()
        self.q_norm, self.k_norm = cfg["q_norm"].to(d), cfg["k_norm"].to(d)
        self.gate_up = cfg["gate_up"].to(d)
        self.batch = {n: getattr(pb, n).to(d) for n in (
            "batch_indices", "positions", "kv_indices", "kv_indptr", "kv_last_page_len")}
        self.cache = share.cache if share is not None else wl.sentinel_cache(cfg["cache_shape"]).to(d)
        B = self.ids.numel()
        self.hidden = torch.empty((B, cfg["H"]), dtype=torch.bfloat16, device=d)
        self.normed = torch.empty_like(self.hidden)
        self.q_out = torch.empty((B, self.Hq, self.D), dtype=torch.bfloat16, device=d)
        self.k_out = torch.empty((B, self.Hkv, self.D), dtype=torch.bfloat16, device=d)
        self.act = torch.empty((B, cfg["I"]), dtype=torch.bfloat16, device=d)
        self.graph = None

    def reset(self):
        """Restore the inputs the chain mutates (residual stream, cache)."""
        self.residual.copy_(self.residual0)
        self.cache.view(torch.int16).fill_(wl.SENTINEL_BITS)

    def run(self):
        if self.saved:
            if self._saved is None:
                with ops.saved_group(self.hidden.device) as g:
                    self._ops()
                self._saved = g[0]
            self._saved.launch()
        elif self.grouped:
            with ops.op_group(self.hidden.device):
                self._ops()
        else:
            self._ops()

    def _ops(self):
        b = self.batch
        ops.embedding(self.ids, self.W, out=self.hidden)
        ops.add_rms_norm(self.hidden, self.residual, self.w_norm, self.eps, out=self.normed,
                         residual_out=self.residual)
        q, k, v = wl.split_qkv(self.qkv0, self.Hq, self.Hkv, self.D)
        if self.fused:
            ops.qk_rms_norm_rope_append(
                q, k, v, self.q_norm, self.k_norm, self.eps, b["positions"], b["batch_indices"],
                b["positions"], self.cache, b["kv_indices"], b["kv_indptr"],
                b["kv_last_page_len"], rope_theta=self.theta, q_out=self.q_out, k_out=self.k_out)
        else:
            ops.qk_rms_norm(q, k, self.q_norm, self.k_norm, self.eps, q_out=self.q_out, k_out=self.k_out)
            ops.apply_rope_pos_ids_inplace(self.q_out, self.k_out, b["positions"],
                                           rope_theta=self.theta)
            ops.append_paged_kv_cache(self.k_out, v, b["batch_indices"], b["positions"],
                                      self.cache, b["kv_indices"], b["kv_indptr"],
                                      b["kv_last_page_len"])
        ops.silu_and_mul(self.gate_up, out=self.act)

    def capture(self):
        """Record run() into a HIP graph (warm-up launch first, on a side stream)."""
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.run()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.run()
        torch.cuda.synchronize()
        return self.graph

    def outputs(self) -> dict:
        return {"hidden": self.hidden, "normed": self.normed, "residual": self.residual,
                "q": self.q_out, "k": self.k_out, "cache": self.cache, "act": self.act}
