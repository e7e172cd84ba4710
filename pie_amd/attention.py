"""flashinfer's paged-attention wrappers, on this package's gfx950 kernels.

Pie builds these objects once per forward-pass owner and calls ``plan`` then ``run`` per batch
(pie/src/pie_worker/model/llama3.py:293-313 construction, :765-790 plan, :689 run; graph
capture plans once per batch-size bin and replays with new page tables, :340-414, :905-950).
The API is flashinfer 0.6.1's, restated in pie/src/flashinfer_metal/ops.py:163-282.

    BatchDecodeWithPagedKVCacheWrapper   one query token per request  -> pie_hip_attention_decode
    BatchPrefillWithPagedKVCacheWrapper  ragged query tokens, causal /
                                         custom-mask / full visibility -> pie_hip_attention_prefill
    BatchAttentionWithAttentionSinkWrapper  gpt-oss: causal (optionally windowed) attention
                                         whose softmax denominators hold a per-head sink logit
                                         -> pie_hip_attention_decode (one query token per
                                         request) or pie_hip_attention_prefill

``plan`` runs on the host and allocates nothing on the device; ``run`` launches kernels on the
current stream and allocates only its output (unless ``out=`` is given), so it can be captured.
Split requests keep their partial results in the caller's workspace buffer, as flashinfer does.
``window_left`` (flashinfer's sliding window, which OLMo-3 plans per layer) is supported; the
options Pie's models do not use (positional encodings inside attention, logit soft caps, lse
output, fp8 scales) raise instead of being ignored.
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
from typing import Optional, Tuple, Union

import torch

from . import _lib
from .ops import _cache_desc, _check, _stream

__all__ = ["BatchDecodeWithPagedKVCacheWrapper", "BatchPrefillWithPagedKVCacheWrapper",
           "BatchAttentionWithAttentionSinkWrapper"]

_BF16 = torch.bfloat16
_CUS: dict = {}


def _num_cus(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _CUS:
        _CUS[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _CUS[idx]


def _unsupported(name: str, pos_encoding_mode="NONE", logits_soft_cap=None):
    if pos_encoding_mode not in ("NONE", None):
        raise NotImplementedError(f"{name}: pos_encoding_mode={pos_encoding_mode!r} (RoPE is "
                                  "applied before the append, as Pie does)")
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
        _unsupported(name, pos_encoding_mode, logits_soft_cap)
        window_left = -1 if window_left is None or window_left < 0 else int(window_left)
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
                          P=page_size, splits=s, window_left=window_left,
                          sm_scale=(1.0 / math.sqrt(head_dim)) if sm_scale is None else sm_scale)

    begin_forward = plan

    def run(self, q: torch.Tensor,
            paged_kv_cache: Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]], *args,
            q_scale=None, k_scale=None, v_scale=None, out: Optional[torch.Tensor] = None,
            lse: Optional[torch.Tensor] = None, return_lse: bool = False,
            _sinks: Optional[torch.Tensor] = None, **_ignored):
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
                  p["window_left"], None if _sinks is None else _sinks.data_ptr(), p["splits"],
                  ws.data_ptr(), ws.numel() * ws.element_size(),
                  out.data_ptr(),
                  out.stride(0), out.stride(1), _stream(q))
        return out

    forward = run

    def end_forward(self) -> None:
        pass


class BatchPrefillWithPagedKVCacheWrapper:
    """flashinfer.BatchPrefillWithPagedKVCacheWrapper: attention of ragged query tokens (the last
    qo_len positions of each request) over the request's pages (llama3.py:307-309, :779-790,
    :689). Visibility: the custom mask when given (Pie always passes one, batching.py:226-228),
    else causal=True's window, else every cached position (flashinfer's default)."""

    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD",
                 use_cuda_graph: bool = False, **_ignored) -> None:
        if kv_layout not in ("NHD", "HND"):
            raise ValueError(f"kv_layout must be 'NHD' or 'HND', got {kv_layout!r}")
        if use_cuda_graph:
            raise NotImplementedError("BatchPrefillWithPagedKVCacheWrapper: use_cuda_graph "
                                      "(Pie captures only decode)")
        self._workspace = float_workspace_buffer
        self._kv_layout = kv_layout
        self._plan = None

    def plan(self, qo_indptr: torch.Tensor, paged_kv_indptr: torch.Tensor,
             paged_kv_indices: torch.Tensor, paged_kv_last_page_len: torch.Tensor,
             num_qo_heads: int, num_kv_heads: int, head_dim_qk: int, page_size: int,
             head_dim_vo: Optional[int] = None, custom_mask: Optional[torch.Tensor] = None,
             packed_custom_mask: Optional[torch.Tensor] = None, causal: bool = False,
             pos_encoding_mode: str = "NONE", use_fp16_qk_reduction: bool = False,
             sm_scale: Optional[float] = None, window_left: int = -1,
             logits_soft_cap: Optional[float] = None, rope_scale: Optional[float] = None,
             rope_theta: Optional[float] = None, q_data_type=torch.float16, kv_data_type=None,
             non_blocking: bool = True, **_ignored) -> None:
        name = "BatchPrefillWithPagedKVCacheWrapper.plan"
        _unsupported(name, pos_encoding_mode, logits_soft_cap)
        window_left = -1 if window_left is None or window_left < 0 else int(window_left)
        if head_dim_vo not in (None, head_dim_qk):
            raise NotImplementedError(f"{name}: head_dim_vo {head_dim_vo} != head_dim_qk")
        if num_kv_heads <= 0 or num_qo_heads % num_kv_heads:
            raise ValueError(f"{name}: num_qo_heads {num_qo_heads} is not a multiple of "
                             f"num_kv_heads {num_kv_heads}")
        dev = self._workspace.device
        batch = qo_indptr.numel() - 1
        if paged_kv_indptr.numel() != batch + 1 or paged_kv_last_page_len.numel() != batch:
            raise ValueError(f"{name}: qo_indptr, paged_kv_indptr and paged_kv_last_page_len "
                             "disagree on the batch size")
        # host copies of the small index arrays (flashinfer's plan reads them on the host too)
        qo_h = qo_indptr.to("cpu", torch.int32).contiguous()
        kv_h = paged_kv_indptr.to("cpu", torch.int32).contiguous()
        ll_h = paged_kv_last_page_len.to("cpu", torch.int32).contiguous()
        mask = custom_mask
        if mask is None and packed_custom_mask is not None:
            bits = (packed_custom_mask.to(torch.uint8).unsqueeze(-1)
                    >> torch.arange(8, dtype=torch.uint8, device=packed_custom_mask.device)) & 1
            mask = bits.flatten().bool()
        mode = 2 if mask is not None else (1 if causal else 0)
        G = num_qo_heads // num_kv_heads
        T = int(qo_h[-1]) if batch else 0
        n_items = T * G // 64 + batch + 1
        # header, 8-word items, the persistent schedule (slot offsets, one word per (kv head,
        # item) unit), mask offsets
        cap = 16 + 8 * n_items + (4096 + n_items * num_kv_heads) + 4 * batch + 8
        plan = np.zeros(cap, dtype=np.int32)
        words, items, mbytes, mwords = C.c_int64(0), C.c_int64(0), C.c_int64(0), C.c_int64(0)
        _lib.call("pie_hip_attention_prefill_plan", qo_h.data_ptr(), kv_h.data_ptr(), ll_h.data_ptr(),
                  batch, page_size, num_qo_heads, num_kv_heads, head_dim_qk, mode, plan.ctypes.data, cap,
                  C.byref(words), C.byref(items), C.byref(mbytes), C.byref(mwords))
        if mode == 2:
            if mask.dtype not in (torch.bool, torch.uint8):
                raise ValueError(f"{name}: custom_mask must be bool, got {mask.dtype}")
            mask = mask.reshape(-1)
            if mask.numel() < mbytes.value:
                raise ValueError(f"{name}: custom_mask has {mask.numel()} entries, the batch needs "
                                 f"{mbytes.value} (sum of qo_len * kv_len)")
            mask = mask.to(dev).contiguous()
        # workspace layout: [plan words | packed mask words | per-token extents] (mode 2), each
        # 16-byte aligned
        nbytes = (words.value * 4 + 15) // 16 * 16
        mask_off = nbytes
        ext_off = mask_off + (mwords.value * 4 + 15) // 16 * 16
        need = ext_off + T * 4 if mode == 2 else nbytes
        ws_bytes = self._workspace.numel() * self._workspace.element_size()
        if need > ws_bytes:
            raise ValueError(f"{name}: the plan needs {need} bytes of workspace, have {ws_bytes}")
        ws8 = self._workspace.view(torch.uint8)
        plan_d = ws8[: words.value * 4].view(torch.int32)
        plan_d.copy_(torch.from_numpy(plan[: words.value]), non_blocking=False)
        tables = [t if t.device == dev else t.to(dev) for t in
                  (qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len)]
        packed = extent = None
        if mode == 2 and mwords.value:
            packed = ws8[mask_off: mask_off + mwords.value * 4].view(torch.int32)
            extent = ws8[ext_off: ext_off + T * 4].view(torch.int32)
            _lib.call("pie_hip_attention_pack_mask", mask.data_ptr(), plan_d.data_ptr(),
                      tables[0].data_ptr(), tables[1].data_ptr(), tables[3].data_ptr(), batch,
                      page_size, mwords.value, T, packed.data_ptr(), extent.data_ptr(),
                      _stream(plan_d))
        self._plan = dict(qo_indptr=tables[0], indptr=tables[1], indices=tables[2],
                          last_page_len=tables[3], batch=batch, T=T, Hq=num_qo_heads,
                          Hkv=num_kv_heads, D=head_dim_qk, P=page_size, mode=mode, packed=packed, extent=extent,
                          window_left=window_left,
                          plan=plan_d, items=items.value, woff_word=int(plan[4]),
                          sm_scale=(1.0 / math.sqrt(head_dim_qk)) if sm_scale is None else sm_scale)

    begin_forward = plan

    def run(self, q: torch.Tensor,
            paged_kv_cache: Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]], *args,
            q_scale=None, k_scale=None, v_scale=None, out: Optional[torch.Tensor] = None,
            lse: Optional[torch.Tensor] = None, return_lse: bool = False,
            _sinks: Optional[torch.Tensor] = None, **_ignored):
        name = "BatchPrefillWithPagedKVCacheWrapper.run"
        p = self._plan
        if p is None:
            raise RuntimeError(f"{name}: plan() must be called before run()")
        if return_lse or lse is not None:
            raise NotImplementedError(f"{name}: lse output")
        if q_scale not in (None, 1.0) or k_scale not in (None, 1.0) or v_scale not in (None, 1.0):
            raise NotImplementedError(f"{name}: quantisation scales")
        _check(name, _BF16, q=q)
        _check(name, torch.int32, qo_indptr=p["qo_indptr"], indptr=p["indptr"],
               indices=p["indices"], last_page_len=p["last_page_len"])
        T, Hq, Hkv, D = p["T"], p["Hq"], p["Hkv"], p["D"]
        if q.dim() != 3 or tuple(q.shape) != (T, Hq, D) or q.stride(2) != 1:
            raise ValueError(f"{name}: q must be [{T}, {Hq}, {D}] with unit inner stride, got "
                             f"{tuple(q.shape)}")
        kp, vp, npages, ps, ss, hs, P = _cache_desc(paged_kv_cache, self._kv_layout, Hkv, D, name)
        if P != p["P"]:
            raise ValueError(f"{name}: cache page size {P} != planned {p['P']}")
        if out is None:
            out = torch.empty((T, Hq, D), dtype=_BF16, device=q.device)
        else:
            _check(name, _BF16, out=out)
            if tuple(out.shape) != (T, Hq, D) or out.stride(2) != 1:
                raise ValueError(f"{name}: out must be [{T}, {Hq}, {D}]")
        packed = p["packed"]
        if p["mode"] == 2 and packed is None:  # a mask over zero positions: nothing is visible
            return out.zero_()
        _lib.call("pie_hip_attention_prefill", q.data_ptr(), q.stride(0), q.stride(1), kp, vp, ps,
                  ss, hs, npages, p["qo_indptr"].data_ptr(), p["indptr"].data_ptr(),
                  p["indices"].data_ptr(), p["last_page_len"].data_ptr(), Hq, Hkv, D, P,
                  float(p["sm_scale"]), p["mode"], p["window_left"],
                  None if _sinks is None else _sinks.data_ptr(),
                  packed.data_ptr() if packed is not None else None,
                  p["extent"].data_ptr() if p["extent"] is not None else None,
                  p["plan"].data_ptr(), p["items"], p["woff_word"], out.data_ptr(), out.stride(0),
                  out.stride(1), _stream(q))
        return out

    forward = run

    def end_forward(self) -> None:
        pass


class BatchAttentionWithAttentionSinkWrapper:
    """flashinfer's BatchAttentionWithAttentionSinkWrapper as gpt-oss uses it
    (pie/src/pie_worker/model/gpt_oss.py:420-438 construction, :839-870 plan, :693-697 run):
    causal attention over the paged cache, optionally in a sliding window (``window_left``),
    where each query head's softmax denominator also holds that head's sink logit ``sinks[h]``
    (fp32, in the units of the scaled scores) and the sink contributes no value:
        out = sum_t e^{s_t} v_t / (sum_t e^{s_t} + e^{sinks[h]}),  s_t = q . k_t * sm_scale.
    A batch of one query token per request runs the decode kernel (split over the context),
    any other batch the prefill kernel in causal mode; the sink enters both kernels' final
    normalisation."""

    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD",
                 window_left: int = -1, q_data_type=torch.bfloat16, kv_data_type=None,
                 head_dim_qk: Optional[int] = None, head_dim_vo: Optional[int] = None,
                 **_ignored) -> None:
        if head_dim_vo not in (None, head_dim_qk):
            raise NotImplementedError("BatchAttentionWithAttentionSinkWrapper: head_dim_vo != head_dim_qk")
        self._window_left = -1 if window_left is None or window_left < 0 else int(window_left)
        self._decode = BatchDecodeWithPagedKVCacheWrapper(float_workspace_buffer, kv_layout)
        self._prefill = BatchPrefillWithPagedKVCacheWrapper(float_workspace_buffer, kv_layout)
        self._use = None
        self._Hq = 0

    def plan(self, qo_indptr: torch.Tensor, paged_kv_indptr: torch.Tensor,
             paged_kv_indices: torch.Tensor, paged_kv_last_page_len: torch.Tensor,
             num_qo_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
             causal: bool = True, window_left: Optional[int] = None, sm_scale: Optional[float] = None,
             q_data_type=torch.bfloat16, kv_data_type=None, non_blocking: bool = True,
             **_ignored) -> None:
        name = "BatchAttentionWithAttentionSinkWrapper.plan"
        if not causal:
            raise NotImplementedError(f"{name}: causal=False")
        wl = self._window_left if window_left is None else window_left
        qo_h = qo_indptr.to("cpu", torch.int64)
        single = qo_h.numel() > 1 and bool(((qo_h[1:] - qo_h[:-1]) == 1).all())
        self._Hq = num_qo_heads
        if single:
            self._decode.plan(paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len,
                              num_qo_heads, num_kv_heads, head_dim, page_size, window_left=wl,
                              sm_scale=sm_scale, non_blocking=non_blocking)
            self._use = self._decode
        else:
            self._prefill.plan(qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len,
                               num_qo_heads, num_kv_heads, head_dim, page_size, causal=True,
                               window_left=wl, sm_scale=sm_scale, non_blocking=non_blocking)
            self._use = self._prefill

    begin_forward = plan

    def run(self, q: torch.Tensor,
            paged_kv_cache: Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]],
            sinks: torch.Tensor, sm_scale: Optional[float] = None,
            out: Optional[torch.Tensor] = None, **_ignored) -> torch.Tensor:
        name = "BatchAttentionWithAttentionSinkWrapper.run"
        if self._use is None:
            raise RuntimeError(f"{name}: plan() must be called before run()")
        if not isinstance(sinks, torch.Tensor) or tuple(sinks.shape) != (self._Hq,):
            raise ValueError(f"{name}: sinks must be a [{self._Hq}] tensor (one logit per query head)")
        if not sinks.is_cuda or sinks.device != q.device:
            raise RuntimeError(f"{name}: sinks must be on {q.device}")
        s = sinks if sinks.dtype == torch.float32 and sinks.is_contiguous() else sinks.float().contiguous()
        p = self._use._plan
        if sm_scale is not None:
            p = dict(p, sm_scale=float(sm_scale))
        saved, self._use._plan = self._use._plan, p
        try:
            return self._use.run(q, paged_kv_cache, out=out, _sinks=s)
        finally:
            self._use._plan = saved

    forward = run

    def end_forward(self) -> None:
        pass
