"""flashinfer.sampling's samplers and Pie's safe_scaled_softmax on this package's gfx950 kernels.

Pie imports the five samplers from ``flashinfer.sampling`` (pie/src/pie_worker/model/common.py:13-28)
and calls them per sampler group (:316-344) on the probabilities its safe_scaled_softmax produced
(:68-188). The signatures are flashinfer 0.6.1's; the semantics are restated in
pie/src/flashinfer_metal/sampling.py:19-79 (whose top-k keeps the batch's largest k for every
row and whose top-p drops the token that crosses p; these follow flashinfer: per-row k, and the
crossing token stays).

Each call is one kernel launch (``pie_hip_sample``): one work group per row, exact thresholds by
radix select, an inverse-CDF draw in index order. Randomness: Philox4x32-10 keyed by ``seed`` and
counted by ``offset``; when neither is given, a per-process seed (from torch's default generator)
and an offset that advances by one per call, so successive calls draw independent numbers and a
fixed (seed, offset) reproduces a draw exactly. ``generator=`` (a torch.Generator) supplies the
numbers: a CPU generator draws each call's seed from its own stream, a GPU generator gives its
seed and its Philox offset, which each call advances. ``uniforms=`` (float64 [batch], this
package's extension) fixes the uniform of every row, which tests use for exact comparisons.
"""
from __future__ import annotations

import ctypes as C
import threading
from typing import Optional, Union

import torch

from . import _lib
from .ops import _check, _stream

__all__ = ["sampling_from_probs", "top_p_sampling_from_probs", "top_k_sampling_from_probs",
           "min_p_sampling_from_probs", "top_k_top_p_sampling_from_probs", "safe_scaled_softmax"]

_MODES = {"plain": 0, "top_p": 1, "top_k": 2, "min_p": 3, "top_k_top_p": 4}
_lock = threading.Lock()
_state = {"seed": None, "offset": 0}


def _seed_offset(generator, seed, offset):
    if seed is not None:
        return int(seed) & (2**64 - 1), int(offset or 0) & (2**64 - 1)
    if generator is not None:
        if generator.device.type == "cpu":
            # a fresh 62-bit seed from the generator's own stream (advances it; no device sync)
            return int(torch.randint(0, 2**62, (1,), generator=generator)), 0
        # a GPU (Philox) generator: its seed, and its offset, which each call advances
        off = generator.get_offset()
        generator.set_offset(off + 4)
        return generator.initial_seed() & (2**64 - 1), off
    with _lock:
        if _state["seed"] is None:
            _state["seed"] = int(torch.randint(0, 2**62, (1,)).item())
        off = _state["offset"]
        _state["offset"] = off + 1
        return _state["seed"], off


def _param(name, v, B, dtype, dev):
    """(device pointer or None, scalar) for a per-row parameter given as a number or tensor."""
    if isinstance(v, torch.Tensor):
        if v.numel() == 1 and v.dim() == 0:
            return None, v.item()
        if v.shape != (B,):
            raise ValueError(f"{name} must be a scalar or a [{B}] tensor, got {tuple(v.shape)}")
        t = v.to(device=dev, dtype=dtype).contiguous()
        return t, 0
    return None, v


def _sample(name, mode, probs, indices, top_k=0, top_p=1.0, min_p=0.0, generator=None,
            seed=None, offset=None, uniforms=None, check_nan=False):
    _check(name, torch.float32, probs=probs)
    if probs.dim() != 2 or probs.stride(1) != 1:
        raise ValueError(f"{name}: probs must be [batch, vocab] with unit inner stride")
    dev = probs.device
    rows = None
    B = probs.shape[0]
    if indices is not None:
        if indices.dtype not in (torch.int32, torch.int64):
            raise ValueError(f"{name}: indices must be int32 or int64, got {indices.dtype}")
        rows = indices.to(device=dev, dtype=torch.int32).contiguous()
        if rows.dim() != 1:
            raise ValueError(f"{name}: indices must be 1-D")
        B = rows.numel()
    if check_nan and torch.isnan(probs).any():
        raise ValueError(f"{name}: probs contain NaN")
    tk, tks = _param("top_k", top_k, B, torch.int32, dev)
    tp, tps = _param("top_p", top_p, B, torch.float32, dev)
    mp, mps = _param("min_p", min_p, B, torch.float32, dev)
    u = None
    if uniforms is not None:
        u = torch.as_tensor(uniforms, dtype=torch.float64, device=dev).reshape(B).contiguous()
    s, o = _seed_offset(generator, seed, offset)
    out = torch.empty(B, dtype=torch.int32, device=dev)
    ptr = lambda t: t.data_ptr() if t is not None else None
    _lib.call("pie_hip_sample", probs.data_ptr(), probs.stride(0), probs.shape[0], probs.shape[1], B,
              ptr(rows),
              _MODES[mode], ptr(tk), int(tks), ptr(tp), float(tps), ptr(mp), float(mps), ptr(u),
              C.c_uint64(s), C.c_uint64(o), out.data_ptr(), _stream(probs))
    return out


def sampling_from_probs(probs: torch.Tensor, indices: Optional[torch.Tensor] = None,
                        deterministic: bool = True, generator=None, check_nan: bool = False,
                        seed: Optional[int] = None, offset: Optional[int] = None,
                        uniforms=None) -> torch.Tensor:
    """Draw one token per row from probs [batch, vocab] (fp32). Returns int32 [batch]."""
    return _sample("sampling_from_probs", "plain", probs, indices, generator=generator, seed=seed,
                   offset=offset, uniforms=uniforms, check_nan=check_nan)


def top_p_sampling_from_probs(probs: torch.Tensor, top_p: Union[torch.Tensor, float],
                              indices: Optional[torch.Tensor] = None, deterministic: bool = True,
                              generator=None, check_nan: bool = False, seed: Optional[int] = None,
                              offset: Optional[int] = None, uniforms=None) -> torch.Tensor:
    """Nucleus sampling: token i stays iff the mass of more probable tokens is below top_p."""
    return _sample("top_p_sampling_from_probs", "top_p", probs, indices, top_p=top_p,
                   generator=generator, seed=seed, offset=offset, uniforms=uniforms,
                   check_nan=check_nan)


def top_k_sampling_from_probs(probs: torch.Tensor, top_k: Union[torch.Tensor, int],
                              indices: Optional[torch.Tensor] = None, deterministic: bool = True,
                              generator=None, check_nan: bool = False, seed: Optional[int] = None,
                              offset: Optional[int] = None, uniforms=None) -> torch.Tensor:
    """Top-k sampling: token i stays iff fewer than k tokens are more probable."""
    return _sample("top_k_sampling_from_probs", "top_k", probs, indices, top_k=top_k,
                   generator=generator, seed=seed, offset=offset, uniforms=uniforms,
                   check_nan=check_nan)


def min_p_sampling_from_probs(probs: torch.Tensor, min_p: Union[torch.Tensor, float],
                              indices: Optional[torch.Tensor] = None, deterministic: bool = True,
                              generator=None, check_nan: bool = False, seed: Optional[int] = None,
                              offset: Optional[int] = None, uniforms=None) -> torch.Tensor:
    """Min-p sampling: token i stays iff p_i >= min_p * max p."""
    return _sample("min_p_sampling_from_probs", "min_p", probs, indices, min_p=min_p,
                   generator=generator, seed=seed, offset=offset, uniforms=uniforms,
                   check_nan=check_nan)


def top_k_top_p_sampling_from_probs(probs: torch.Tensor, top_k: Union[torch.Tensor, int],
                                    top_p: Union[torch.Tensor, float],
                                    indices: Optional[torch.Tensor] = None,
                                    filter_apply_order: str = "top_k_first",
                                    deterministic: bool = True, generator=None,
                                    check_nan: bool = False, seed: Optional[int] = None,
                                    offset: Optional[int] = None, uniforms=None) -> torch.Tensor:
    """Top-k, then top-p inside the top-k set (filter_apply_order="top_k_first")."""
    if filter_apply_order != "top_k_first":
        raise NotImplementedError(f"filter_apply_order={filter_apply_order!r}")
    return _sample("top_k_top_p_sampling_from_probs", "top_k_top_p", probs, indices, top_k=top_k,
                   top_p=top_p, generator=generator, seed=seed, offset=offset, uniforms=uniforms,
                   check_nan=check_nan)


def safe_scaled_softmax(logits: torch.Tensor, temperatures: torch.Tensor,
                        greedy_threshold: float = 1e-5, out: Optional[torch.Tensor] = None):
    """Pie's safe_scaled_softmax (common.py:38-59, :68-188): softmax(logits / T) per row, the
    one-hot of the first maximum where T < greedy_threshold; output in the logits' dtype."""
    name = "safe_scaled_softmax"
    if logits.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"{name}: logits must be float32 or bfloat16, got {logits.dtype}")
    _check(name, logits.dtype, logits=logits)
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError(f"{name}: logits must be [batch, vocab] with unit inner stride")
    B, V = logits.shape
    t = temperatures.reshape(-1).to(device=logits.device, dtype=torch.float32).contiguous()
    if t.numel() != B:
        raise ValueError(f"{name}: {t.numel()} temperatures for {B} rows")
    if out is None:
        out = torch.empty_like(logits)
    elif out.shape != logits.shape or out.dtype != logits.dtype or out.stride(1) != 1:
        raise ValueError(f"{name}: out must match logits")
    _lib.call("pie_hip_scaled_softmax", logits.data_ptr(), 1 if logits.dtype == torch.bfloat16 else 0,
              logits.stride(0), B, V, t.data_ptr(), float(greedy_threshold), out.data_ptr(),
              out.stride(0), _stream(logits))
    return out
