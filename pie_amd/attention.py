"""flashinfer's paged-attention wrappers, on this package's gfx950 kernels.

Pie builds these objects once per forward-pass owner and calls ``plan`` then ``run`` per batch
(pie/src/pie_worker/model/llama3.py:293-313 construction, :765-790 plan, :689 run; graph
capture plans once per batch-size bin and replays with new page tables, :340-414, :905-950).
The API is flashinfer 0.6.1's, restated in pie/src/flashinfer_metal/ops.py:163-282.

    BatchDecodeWithPagedKVCacheWrapper   one query token per request  -> pie_hip_attention_decode

``plan`` runs on the host and allocates nothing on the device; ``run`` launches kernels on the
current stream and allocates only its output (unless ``out=`` is given), so it can be captured.
Split requests keep their partial results in the caller's workspace buffer, as flashinfer does.
Unsupported options (positional encodings inside attention, sliding windows, soft caps, lse
output) raise instead of being ignored.
"""
from __future__ import annotations

import ctypes as C
import math
from typing import Optional, Tuple, Union

import torch

from . import _lib
from .ops import _cache_desc, _check, _stream

__all__ = ["BatchDecodeWithPagedKVCacheWrapper"]

_BF16 = torch.bfloat16
_CUS: dict = {}


def _num_cus(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _CUS:
        _CUS[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _CUS[idx]


def _unsupported(name: str, pos_encoding_mode="NONE", window_left=-1, logits_soft_cap=None,
                 rope_scale=None, rope_theta=None):
    if pos_encoding_mode not in ("NONE", None):
        raise NotImplementedError(f"{name}: pos_encoding_mode={pos_encoding_mode!r} (RoPE is "
                                  "applied before the append, as Pie does)")
    if window_left not in (-1, None):
        raise NotImplementedError(f"{name}: sliding windows (window_left={window_left})")
    if logits_soft_cap not in (None, 0, 0.0):
        raise NotImplementedError(f"{name}: logits_soft_cap={logits_soft_cap}")


class BatchDecodeWithPagedKVCacheWrapper:
    """flashinfer.BatchDecodeWithPagedKVCacheWrapper: attention of one query token per request
    over that request's pages (llama3.py:293-301, :311-313, :765-777, :689)."""

    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD",
                 use_cuda_graph: bool = False, use_tensor_cores: bool = False,
                 paged_kv_indptr_buffer: Optional[torch.Tensor] = None,
                 paged_kv_indices_buffer: Optional[torch.Tensor] = None,
                 paged_kv_last_page_len_buffer: Optional[torch.Tensor] = None,
                 backend: str = "auto", **_ignored) -> None:
        if kv_layout not in ("NHD", "HND"):
            raise ValueError(f"kv_layout must be 'NHD' or 'HND', got {kv_layout!r}")
        self._workspace = float_workspace_buffer
        self._kv_layout = kv_layout
        self._use_cuda_graph = use_cuda_graph
        self._fixed = (paged_kv_indptr_buffer, paged_kv_indices_buffer,
                       paged_kv_last_page_len_buffer)
        if use_cuda_graph and any(b is None for b in self._fixed):
            raise ValueError("use_cuda_graph=True needs the paged_kv_*_buffer tensors")
        self._plan = None

    @property
    def is_cuda_graph_enabled(self) -> bool:
        return self._use_cuda_graph

    def plan(self, indptr: torch.Tensor, indices: torch.Tensor, last_page_len: torch.Tensor,
             num_qo_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
             pos_encoding_mode: str = "NONE", window_left: int = -1,
             logits_soft_cap: Optional[float] = None, q_data_type=torch.float16,
             kv_data_type=None, data_type=None, sm_scale: Optional[float] = None,
             rope_scale: Optional[float] = None, rope_theta: Optional[float] = None,
             non_blocking: bool = True, **_ignored) -> None:
        name = "BatchDecodeWithPagedKVCacheWrapper.plan"
        _unsupported(name, pos_encoding_mode, window_left, logits_soft_cap)
        if num_kv_heads <= 0 or num_qo_heads % num_kv_heads:
            raise ValueError(f"{name}: num_qo_heads {num_qo_heads} is not a multiple of "
                             f"num_kv_heads {num_kv_heads}")
        batch = indptr.numel() - 1
        if self._use_cuda_graph:
            # the fixed buffers are what the captured launches read; copy new tables into them
            ib, xb, lb = self._fixed
            if indptr.data_ptr() != ib.data_ptr():
                ib[: batch + 1].copy_(indptr, non_blocking=non_blocking)
            if indices.data_ptr() != xb.data_ptr():
                xb[: indices.numel()].copy_(indices, non_blocking=non_blocking)
            if last_page_len.data_ptr() != lb.data_ptr():
                lb[:batch].copy_(last_page_len, non_blocking=non_blocking)
            indptr, indices, last_page_len = ib[: batch + 1], xb, lb[:batch]
        # the longest context is known without a device sync only for host tables
        max_kv = -1
        if indptr.device.type == "cpu" and not self._use_cuda_graph:
            np_ = (indptr[1:] - indptr[:-1]).to(torch.int64)
            if batch:
                max_kv = int(((np_ - 1).clamp(min=0) * page_size + last_page_len.to(torch.int64)).max())
        splits = C.c_int64(0)
        dev = self._workspace.device
        _lib.call("pie_hip_attention_decode_plan", batch, num_kv_heads, max_kv,
                  _num_cus(dev) if dev.type == "cuda" else 0, C.byref(splits))
        s = splits.value
        need = batch * s * num_qo_heads * (head_dim + 1) * 4 if s > 1 else 0
        ws_bytes = self._workspace.numel() * self._workspace.element_size()
        if need > ws_bytes:
            s = 1  # fall back to one work group per (request, kv head): no partials needed
            need = 0
        if any(t.device.type != "cuda" for t in (indptr, indices, last_page_len)):
            indptr, indices, last_page_len = (t.to(dev, non_blocking=non_blocking)
                                              for t in (indptr, indices, last_page_len))
        self._plan = dict(indptr=indptr, indices=indices, last_page_len=last_page_len,
                          batch=batch, Hq=num_qo_heads, Hkv=num_kv_heads, D=head_dim,
                          P=page_size, splits=s,
                          sm_scale=(1.0 / math.sqrt(head_dim)) if sm_scale is None else sm_scale)

    begin_forward = plan

    def run(self, q: torch.Tensor,
            paged_kv_cache: Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]], *args,
            q_scale=None, k_scale=None, v_scale=None, out: Optional[torch.Tensor] = None,
            lse: Optional[torch.Tensor] = None, return_lse: bool = False, **_ignored):
        name = "BatchDecodeWithPagedKVCacheWrapper.run"
        p = self._plan
        if p is None:
            raise RuntimeError(f"{name}: plan() must be called before run()")
        if return_lse or lse is not None:
            raise NotImplementedError(f"{name}: lse output")
        if q_scale not in (None, 1.0) or k_scale not in (None, 1.0) or v_scale not in (None, 1.0):
            raise NotImplementedError(f"{name}: quantisation scales")
        _check(name, _BF16, q=q)
        _check(name, torch.int32, indptr=p["indptr"], indices=p["indices"],
               last_page_len=p["last_page_len"])
        B, Hq, Hkv, D = p["batch"], p["Hq"], p["Hkv"], p["D"]
        if q.dim() != 3 or tuple(q.shape) != (B, Hq, D) or q.stride(2) != 1:
            raise ValueError(f"{name}: q must be [{B}, {Hq}, {D}] with unit inner stride, got "
                             f"{tuple(q.shape)}")
        kp, vp, npages, ps, ss, hs, P = _cache_desc(paged_kv_cache, self._kv_layout, Hkv, D, name)
        if P != p["P"]:
            raise ValueError(f"{name}: cache page size {P} != planned {p['P']}")
        if out is None:
            out = torch.empty((B, Hq, D), dtype=_BF16, device=q.device)
        else:
            _check(name, _BF16, out=out)
            if tuple(out.shape) != (B, Hq, D) or out.stride(2) != 1:
                raise ValueError(f"{name}: out must be [{B}, {Hq}, {D}]")
        ws = self._workspace
        _lib.call("pie_hip_attention_decode", q.data_ptr(), q.stride(0), q.stride(1), kp, vp, ps,
                  ss, hs, npages, p["indptr"].data_ptr(), p["indices"].data_ptr(),
                  p["last_page_len"].data_ptr(), B, Hq, Hkv, D, P, float(p["sm_scale"]),
                  p["splits"], ws.data_ptr(), ws.numel() * ws.element_size(), out.data_ptr(),
                  out.stride(0), out.stride(1), _stream(q))
        return out

    forward = run

    def end_forward(self) -> None:
        pass
