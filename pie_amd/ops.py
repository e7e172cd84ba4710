"""Drop-in op namespace for Pie's per-layer hot path on MI355X.

The model files bind their kernel namespace at import time
(``import flashinfer as ops`` at pie/src/pie_worker/model/llama3.py:18-21 and qwen3.py:18-21)
and call ``torch.nn.functional`` inline for the rest. This module provides both:

flashinfer names (same arguments, same in-place / return behaviour; the API restated in
pie/src/flashinfer_metal/ops.py:285-436):
    apply_rope_pos_ids_inplace, apply_llama31_rope_pos_ids_inplace, append_paged_kv_cache,
    get_seq_lens, get_batch_indices_positions, rmsnorm, fused_add_rmsnorm, silu_and_mul

replacements for the inline torch expressions:
    rms_norm(x, normalized_shape, weight, eps)   fun.rms_norm      (llama3.py:555, qwen3.py:651)
    add_rms_norm(x, residual, weight, eps)       residual + x, then the next fun.rms_norm
    qk_rms_norm(q, k, q_weight, k_weight, eps)   the two per-head fun.rms_norm of qwen3.py:651-662
    silu_and_mul(gate_up)                        fun.silu(gate) * up (llama3.py:569-572)
    embedding(ids, weight)                       fun.embedding      (llama3.py:471)

plus fused entries with no single reference counterpart:
    apply_{llama31_,}rope_pos_ids_and_append_paged_kv_cache   RoPE + append in one HBM pass
    qk_rms_norm_rope_append                      q/k norm + RoPE + append (qwen3.py:651-684)
    op_group()                                   context: the independent ops of a decode step
                                                 (embedding -> add_rms_norm, q/k prologue,
                                                 silu_and_mul) in ONE kernel launch

variant ops of the other model families (gemma2/3, gpt-oss, olmo3):
    gemma_rms_norm, gemma_add_rms_norm, gemma_qk_rms_norm, gelu_tanh_and_mul,
    embedding(..., scale=), apply_rope_with_cos_sin_cache_inplace

Every op runs a hand-written gfx950 kernel from libpie_hip.so on the current torch stream.
Nothing here allocates except the outputs of out-of-place ops (as the reference's torch calls
do), nothing synchronises the host, and so every op can be captured into a HIP graph. There is
no fallback: a missing library, a non-GPU tensor or an unsupported dtype raises.
"""
from __future__ import annotations

import contextlib
import ctypes as C
from typing import Optional, Sequence, Tuple, Union

import torch

from . import _lib

__all__ = [
    "rmsnorm", "rms_norm", "fused_add_rmsnorm", "add_rms_norm", "qk_rms_norm", "silu_and_mul",
    "embedding", "apply_rope_pos_ids_inplace", "apply_llama31_rope_pos_ids_inplace",
    "append_paged_kv_cache", "apply_rope_pos_ids_and_append_paged_kv_cache",
    "apply_llama31_rope_pos_ids_and_append_paged_kv_cache", "get_seq_lens",
    "get_batch_indices_positions", "rope_inv_freq", "llama31_inv_freq",
    "qk_rms_norm_rope_append", "gemma_rms_norm", "gemma_add_rms_norm", "gemma_qk_rms_norm",
    "gelu_tanh_and_mul", "apply_rope_with_cos_sin_cache_inplace", "op_group",
]

_BF16 = torch.bfloat16


# ----------------------------------------------------------------------------- helpers
# Tensors handed to recorded calls while an op_group() is open: held until the group's kernel
# is enqueued, so a temporary (a contiguous copy, a fresh output) cannot be freed and reused
# before the kernel that reads or writes it is on the stream.
_group_keep: Optional[list] = None


def _keep(*tensors) -> None:
    if _group_keep is not None:
        _group_keep.extend(tensors)


@contextlib.contextmanager
def op_group(device: Optional[torch.device] = None):
    """Record the groupable ops called inside the block and launch them as ONE kernel at its end
    (pie_hip_group_begin / pie_hip_group_end) on the current stream. Groupable: ``embedding``
    (no scale), ``add_rms_norm`` / ``fused_add_rmsnorm``, ``silu_and_mul``,
    ``gelu_tanh_and_mul``, ``qk_rms_norm_rope_append``. The ops must be independent, except
    that an embedding may produce the ``input`` of an ``add_rms_norm`` in the same group (it then
    runs fused into the norm). Results equal the separate calls bit for bit. Other ops called
    inside launch at once. Outputs hold their values only after the block exits."""
    global _group_keep
    if _group_keep is not None:
        raise RuntimeError("op_group: groups do not nest")
    _lib.call("pie_hip_group_begin")
    _group_keep = []
    ok = False
    try:
        yield
        ok = True
    finally:
        keep, _group_keep = _group_keep, None
        idx = torch.cuda.current_device() if device is None else torch.device(device).index
        st = _raw_stream(idx) if _raw_stream is not None else torch.cuda.current_stream(idx).cuda_stream
        if ok:
            _lib.call("pie_hip_group_end", st)
        else:  # close the group; the block's own exception is the one to report
            _lib.load().pie_hip_group_end(st)
        del keep
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


class SavedGroup:
    """A recorded op group kept for relaunching (pie_hip_group_save / pie_hip_group_launch):
    ``launch()`` enqueues what the group's block would have launched, on the current stream, in
    one library call, reading and writing the recorded tensors as they are at launch time. It
    holds those tensors (so they stay allocated and in place); write new inputs into them in place
    between launches."""

    def __init__(self, handle: int, keep: list, device_index: int):
        self._h, self._keep, self._dev = handle, keep, device_index
        self._free = _lib.load().pie_hip_group_free
        self._launch = _lib.load().pie_hip_group_launch

    def launch(self) -> None:
        st = _raw_stream(self._dev) if _raw_stream is not None else \
            torch.cuda.current_stream(self._dev).cuda_stream
        if self._launch(self._h, st) != 0:
            _lib.call("pie_hip_group_launch", self._h, st)  # raises with the library's message

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._free(h)


@contextlib.contextmanager
def saved_group(device: Optional[torch.device] = None):
    """Like op_group(), but the block's ops are not launched: the yielded list receives ONE
    SavedGroup whose ``launch()`` runs them (same kernels, same results) as often as needed."""
    global _group_keep
    if _group_keep is not None:
        raise RuntimeError("saved_group: groups do not nest")
    _lib.call("pie_hip_group_begin")
    _group_keep = []
    out: list = []
    ok = False
    try:
        yield out
        ok = True
    finally:
        keep, _group_keep = _group_keep, None
        idx = torch.cuda.current_device() if device is None else torch.device(device).index
        st = _raw_stream(idx) if _raw_stream is not None else torch.cuda.current_stream(idx).cuda_stream
        h = C.c_void_p(0)
        if ok:
            _lib.call("pie_hip_group_save", st, C.byref(h))
            out.append(SavedGroup(h.value, keep, idx))
        else:  # close the group; the block's own exception is the one to report
            _lib.load().pie_hip_group_save(st, C.byref(h))
            if h.value:
                _lib.load().pie_hip_group_free(h.value)


def _stream(t: torch.Tensor) -> int:
    """The current torch stream of t's device as a raw handle (the raw accessor skips building a
    Stream object: ~0.2 µs against ~2 µs per call)."""
    if _raw_stream is not None:
        idx = t.device.index
        return _raw_stream(torch.cuda.current_device() if idx is None else idx)
    return torch.cuda.current_stream(t.device).cuda_stream


def _check(name: str, dtype: torch.dtype, **tensors: torch.Tensor) -> None:
    dev = None
    for arg, t in tensors.items():
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name}: {arg} must be a torch.Tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise RuntimeError(f"{name}: {arg} must be on a ROCm GPU device, got {t.device}")
        if t.dtype != dtype:
            raise ValueError(f"{name}: {arg} must be {dtype}, got {t.dtype}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{name}: {arg} is on {t.device}, expected {dev}")


def _rows(name: str, x: torch.Tensor, cols: int) -> torch.Tensor:
    """View x as [rows, cols] with unit inner stride (copies only if no such view exists)."""
    if x.shape[-1] != cols:
        raise ValueError(f"{name}: last dim {x.shape[-1]} != {cols}")
    if x.dim() == 2 and x.stride(1) == 1:
        return x
    try:
        v = x.view(-1, cols)
        if v.stride(1) == 1:
            return v
    except RuntimeError:
        pass
    return x.reshape(-1, cols).contiguous()


def _eps(eps: Optional[float]) -> float:
    return float(torch.finfo(torch.float32).eps if eps is None else eps)


# ----------------------------------------------------------------------------- RMSNorm
def rmsnorm(input: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
            out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """flashinfer.norm.rmsnorm: RMSNorm over the last dim, bf16 in/out, fp32 accumulation.

    Numerics follow torch's rms_norm (torch/_decomp/decompositions.py:1760-1810), the op the
    reference calls at pie/src/pie_worker/model/llama3.py:555-560.
    """
    return _rmsnorm("rmsnorm", input, weight, eps, out, False)


def gemma_rms_norm(input: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Gemma RMSNorm, ``x * rsqrt(x.pow(2).mean(-1) + eps) * (1.0 + weight)`` evaluated as bf16
    torch ops (every step rounded to bf16): pie/src/pie_worker/model/gemma2.py:514-526,
    gemma3.py:491-510 (a [T, H, D] input is normalised per head, as gemma3's _qk_norm)."""
    return _rmsnorm("gemma_rms_norm", input, weight, eps, out, True)


def _rmsnorm(name, input, weight, eps, out, gemma):
    _check(name, _BF16, input=input, weight=weight)
    H = input.shape[-1]
    if weight.shape != (H,):
        raise ValueError(f"rmsnorm: weight shape {tuple(weight.shape)} != ({H},)")
    weight = weight.contiguous()
    if input.dim() == 3 and H in (64, 128, 256) and input.stride(-1) == 1:
        return _per_head_norm(input, weight, eps, out, gemma)
    x2 = _rows(name, input, H)
    if out is None:
        out = torch.empty(input.shape, dtype=_BF16, device=input.device)
    y2 = _rows(name, out, H)
    if y2.data_ptr() != out.data_ptr():
        raise ValueError(f"{name}: out must be viewable as [rows, H] with unit inner stride")
    _lib.call("pie_hip_gemma_rmsnorm" if gemma else "pie_hip_rmsnorm", x2.data_ptr(),
              x2.stride(0), weight.data_ptr(), y2.data_ptr(), y2.stride(0), x2.shape[0], H,
              C.c_float(float(eps)), _stream(input))
    return out


def rms_norm(input: torch.Tensor, normalized_shape: Union[int, Sequence[int]],
             weight: Optional[torch.Tensor] = None, eps: Optional[float] = None) -> torch.Tensor:
    """torch.nn.functional.rms_norm signature (normalized over the last dim only)."""
    ns = (normalized_shape,) if isinstance(normalized_shape, int) else tuple(normalized_shape)
    if len(ns) != 1 or input.shape[-1] != ns[0]:
        raise ValueError(f"rms_norm: normalized_shape {ns} must be the last dim of {tuple(input.shape)}")
    if weight is None:
        weight = torch.ones(ns[0], dtype=input.dtype, device=input.device)
    return rmsnorm(input, weight, _eps(eps))


def _per_head_norm(x: torch.Tensor, w: torch.Tensor, eps: float,
                   out: Optional[torch.Tensor], gemma: bool = False) -> torch.Tensor:
    T, H, D = x.shape
    if out is None:
        out = torch.empty((T, H, D), dtype=_BF16, device=x.device)
    if out.shape != x.shape or out.stride(-1) != 1:
        raise ValueError("rmsnorm: out must match input shape with unit inner stride")
    _lib.call("pie_hip_gemma_qk_rmsnorm" if gemma else "pie_hip_qk_rmsnorm", x.data_ptr(),
              x.stride(0), x.stride(1), out.data_ptr(), out.stride(0), out.stride(1), None, 0, 0,
              None, 0, 0, w.data_ptr(), None, T, H, 0, D, C.c_float(float(eps)), _stream(x))
    return out


def gemma_qk_rms_norm(q, k, q_weight, k_weight, eps=None, q_out=None, k_out=None):
    """Gemma3's per-head q/k norm with (1 + weight) and bf16 step rounding (gemma3.py:499-510,
    :653-654), q and k in one launch."""
    return qk_rms_norm(q, k, q_weight, k_weight, eps, q_out, k_out, _gemma=True)


def qk_rms_norm(q: torch.Tensor, k: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor,
                eps: Optional[float] = None, q_out: Optional[torch.Tensor] = None,
                k_out: Optional[torch.Tensor] = None,
                _gemma: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-head RMSNorm of q [T,Hq,D] and k [T,Hkv,D] in one launch.

    Replaces ``q = fun.rms_norm(q, [D], q_norm, eps); k = fun.rms_norm(k, [D], k_norm, eps)``
    (pie/src/pie_worker/model/qwen3.py:651-662). q and k may be strided views of the fused
    qkv projection; the outputs are new contiguous tensors unless q_out/k_out are given
    (which may be q/k themselves for an in-place update).
    """
    _check("qk_rms_norm", _BF16, q=q, k=k, q_weight=q_weight, k_weight=k_weight)
    if q.dim() != 3 or k.dim() != 3 or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError(f"qk_rms_norm: q {tuple(q.shape)} / k {tuple(k.shape)} must be [T,H,D]")
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    if q.stride(2) != 1 or k.stride(2) != 1:
        raise ValueError("qk_rms_norm: head dim must have unit stride")
    if q_weight.shape != (D,) or k_weight.shape != (D,):
        raise ValueError("qk_rms_norm: weights must be [D]")
    q_out = torch.empty((T, Hq, D), dtype=_BF16, device=q.device) if q_out is None else q_out
    k_out = torch.empty((T, Hkv, D), dtype=_BF16, device=k.device) if k_out is None else k_out
    if q_out.shape != q.shape or k_out.shape != k.shape or q_out.stride(2) != 1 or k_out.stride(2) != 1:
        raise ValueError("qk_rms_norm: outputs must match inputs with unit inner stride")
    q_weight, k_weight = q_weight.contiguous(), k_weight.contiguous()
    _lib.call("pie_hip_gemma_qk_rmsnorm" if _gemma else "pie_hip_qk_rmsnorm", q.data_ptr(),
              q.stride(0), q.stride(1), q_out.data_ptr(),
              q_out.stride(0), q_out.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
              k_out.data_ptr(), k_out.stride(0), k_out.stride(1), q_weight.data_ptr(),
              k_weight.data_ptr(), T, Hq, Hkv, D, C.c_float(_eps(eps)), _stream(q))
    return q_out, k_out


def gemma_add_rms_norm(input, residual, weight, eps=None, out=None, residual_out=None):
    """``residual + input`` then Gemma RMSNorm of the sum (gemma3.py:585 / :705 feeding the next
    layer's _gemma_rms_norm); returns (normed, new_residual)."""
    return add_rms_norm(input, residual, weight, eps, out, residual_out, _gemma=True)


def add_rms_norm(input: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                 eps: Optional[float] = None, out: Optional[torch.Tensor] = None,
                 residual_out: Optional[torch.Tensor] = None,
                 _gemma: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Residual add + RMSNorm of the sum; returns (normed, new_residual).

    new_residual = bf16(residual + input)  -- `residual + down` at llama3.py:586 / :710
    normed       = rms_norm(new_residual)  -- the next layer's fun.rms_norm (llama3.py:555/:618)
    Pass residual_out=residual to update the residual stream in place.
    """
    _check("add_rms_norm", _BF16, input=input, residual=residual, weight=weight)
    if input.shape != residual.shape:
        raise ValueError(f"add_rms_norm: input {tuple(input.shape)} != residual {tuple(residual.shape)}")
    H = input.shape[-1]
    if weight.shape != (H,):
        raise ValueError(f"add_rms_norm: weight shape {tuple(weight.shape)} != ({H},)")
    x2, r2 = _rows("add_rms_norm", input, H), _rows("add_rms_norm", residual, H)
    out = torch.empty(input.shape, dtype=_BF16, device=input.device) if out is None else out
    residual_out = (torch.empty(input.shape, dtype=_BF16, device=input.device)
                    if residual_out is None else residual_out)
    y2, s2 = _rows("add_rms_norm", out, H), _rows("add_rms_norm", residual_out, H)
    if y2.data_ptr() != out.data_ptr() or s2.data_ptr() != residual_out.data_ptr():
        raise ValueError("add_rms_norm: outputs must be viewable as [rows, H]")
    weight = weight.contiguous()
    _keep(x2, r2, y2, s2, weight)
    _lib.call("pie_hip_gemma_fused_add_rmsnorm" if _gemma else "pie_hip_fused_add_rmsnorm",
              x2.data_ptr(), x2.stride(0), r2.data_ptr(), r2.stride(0),
              s2.data_ptr(), s2.stride(0), y2.data_ptr(), y2.stride(0), weight.data_ptr(),
              x2.shape[0], H, C.c_float(_eps(eps)), _stream(input))
    return out, residual_out


def fused_add_rmsnorm(input: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                      eps: float = 1e-6) -> None:
    """flashinfer.norm.fused_add_rmsnorm (in place): residual <- residual + input,
    input <- rmsnorm(residual). The sum is rounded to bf16 before the norm, as torch's
    `residual + x` followed by fun.rms_norm rounds it."""
    add_rms_norm(input, residual, weight, eps, out=input, residual_out=residual)


# ----------------------------------------------------------------------------- SiLU-and-mul
def silu_and_mul(input: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """flashinfer.activation.silu_and_mul: input [..., 2I] = [gate | up] -> silu(gate) * up.

    Same values as ``gate, up = torch.split(gate_up, [I, I], -1); fun.silu(gate) * up``
    (pie/src/pie_worker/model/llama3.py:569-572), including torch's rounding of silu to bf16
    before the multiply.
    """
    return _act_and_mul("silu_and_mul", "pie_hip_silu_and_mul", input, out)


def gelu_tanh_and_mul(input: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """flashinfer.activation.gelu_tanh_and_mul: ``fun.gelu(gate, approximate="tanh") * up``
    (gemma2.py:224-226, :608; gemma3.py:246-248, :566), gelu rounded to bf16 before the
    multiply as torch does."""
    return _act_and_mul("gelu_tanh_and_mul", "pie_hip_gelu_tanh_and_mul", input, out)


def _act_and_mul(name, sym, input, out):
    _check(name, _BF16, input=input)
    if input.shape[-1] % 2:
        raise ValueError(f"{name}: last dim {input.shape[-1]} must be even")
    I = input.shape[-1] // 2
    x2 = _rows(name, input, 2 * I)
    if out is None:
        out = torch.empty((*input.shape[:-1], I), dtype=_BF16, device=input.device)
    y2 = _rows(name, out, I)
    if y2.data_ptr() != out.data_ptr():
        raise ValueError(f"{name}: out must be viewable as [rows, I]")
    _keep(x2, y2)
    _lib.call(sym, x2.data_ptr(), x2.stride(0), y2.data_ptr(), y2.stride(0), x2.shape[0], I,
              _stream(input))
    return out


# ----------------------------------------------------------------------------- embedding
def embedding(input: torch.Tensor, weight: torch.Tensor, out: Optional[torch.Tensor] = None,
              check_ids: bool = False, scale: Optional[float] = None) -> torch.Tensor:
    """fun.embedding(ids, W) for int32 ids and a bf16 table (llama3.py:471): a bit copy.
    With ``scale``: ``fun.embedding(ids, W) * scale`` rounded once to bf16, as gemma's
    ``embeddings * self.embed_normalizer`` (gemma3.py:476-489; torch multiplies in fp32).

    The kernel writes a zero row for an id outside [0, V) (it cannot raise without a host
    sync); check_ids=True validates on the host first and raises IndexError as torch does.
    """
    _check("embedding", _BF16, weight=weight)
    _check("embedding", torch.int32, input=input)
    if weight.dim() != 2 or weight.stride(1) != 1:
        raise ValueError("embedding: weight must be [V, H] with unit inner stride")
    V, H = weight.shape
    if check_ids and input.numel() and (int(input.min()) < 0 or int(input.max()) >= V):
        raise IndexError("index out of range in self")
    ids = input.reshape(-1).contiguous()
    T = ids.numel()
    if out is None:
        out = torch.empty((*input.shape, H), dtype=_BF16, device=weight.device)
    y2 = _rows("embedding", out, H)
    if y2.data_ptr() != out.data_ptr() or y2.shape[0] != T:
        raise ValueError("embedding: out must be viewable as [T, H]")
    _keep(ids, weight, y2)
    if scale is None:
        _lib.call("pie_hip_embedding", ids.data_ptr(), T, weight.data_ptr(), V, H,
                  weight.stride(0), y2.data_ptr(), y2.stride(0), _stream(weight))
    else:
        _lib.call("pie_hip_embedding_scaled", ids.data_ptr(), T, weight.data_ptr(), V, H,
                  weight.stride(0), y2.data_ptr(), y2.stride(0), C.c_float(float(scale)),
                  _stream(weight))
    return out


# ----------------------------------------------------------------------------- RoPE
_freq_cache: dict = {}


def rope_inv_freq(rotary_dim: int, rope_scale: float = 1.0, rope_theta: float = 1e4):
    """Host fp32 table of standard RoPE inverse frequencies (computed in float64)."""
    key = ("std", rotary_dim, float(rope_scale), float(rope_theta))
    arr = _freq_cache.get(key)
    if arr is None:
        arr = (C.c_float * (rotary_dim // 2))()
        _lib.call("pie_hip_rope_inv_freq", arr, rotary_dim, C.c_float(rope_scale), C.c_float(rope_theta))
        _freq_cache[key] = arr
    return arr


def llama31_inv_freq(rotary_dim: int, rope_scale: float = 8.0, rope_theta: float = 5e5,
                     low_freq_factor: float = 1.0, high_freq_factor: float = 4.0,
                     old_context_len: float = 8192):
    """Host fp32 table of Llama-3.1 scaled inverse frequencies (metal_rope.metal:63-89)."""
    key = ("l31", rotary_dim, float(rope_scale), float(rope_theta), float(low_freq_factor),
           float(high_freq_factor), float(old_context_len))
    arr = _freq_cache.get(key)
    if arr is None:
        arr = (C.c_float * (rotary_dim // 2))()
        _lib.call("pie_hip_llama31_inv_freq", arr, rotary_dim, C.c_float(rope_scale),
                  C.c_float(rope_theta), C.c_float(low_freq_factor), C.c_float(high_freq_factor),
                  C.c_float(old_context_len))
        _freq_cache[key] = arr
    return arr


def _rope_shapes(name: str, q: torch.Tensor, k: torch.Tensor, pos_ids: torch.Tensor,
                 rotary_dim: Optional[int]) -> Tuple[int, int, int, int, int]:
    _check(name, _BF16, q=q, k=k)
    _check(name, torch.int32, pos_ids=pos_ids)
    if q.dim() != 3 or k.dim() != 3:
        raise ValueError(f"{name}: q and k must be [nnz, heads, head_dim]")
    T, Hq, D = q.shape
    if k.shape[0] != T or k.shape[2] != D:
        raise ValueError(f"{name}: q {tuple(q.shape)} and k {tuple(k.shape)} disagree")
    if pos_ids.shape != (T,) or not pos_ids.is_contiguous():
        raise ValueError(f"{name}: pos_ids must be a contiguous [{T}] tensor")
    if q.stride(2) != 1 or k.stride(2) != 1:
        raise ValueError(f"{name}: head dim must have unit stride")
    rd = D if rotary_dim is None else int(rotary_dim)
    if rd <= 0 or rd > D or rd % 2 or rd // 2 > 256:
        raise ValueError(f"{name}: rotary_dim {rd} must be even, in (0, head_dim={D}] and <= 512")
    return T, Hq, k.shape[1], D, rd


def _rope(name, q, k, pos_ids, rd, interleave, freqs):
    T, Hq, Hkv, D, rd = _rope_shapes(name, q, k, pos_ids, rd)
    _lib.call("pie_hip_rope_inplace", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
              k.stride(0), k.stride(1), pos_ids.data_ptr(), T, Hq, Hkv, D, rd,
              1 if interleave else 0, freqs(rd), _stream(q))


def apply_rope_pos_ids_inplace(q: torch.Tensor, k: torch.Tensor, pos_ids: torch.Tensor,
                               rotary_dim: Optional[int] = None, interleave: bool = False,
                               rope_scale: float = 1, rope_theta: float = 1e4) -> None:
    """flashinfer.apply_rope_pos_ids_inplace (qwen3.py:665-670; spec
    pie/src/flashinfer_metal/ops.py:285-303): rotates q and k in place at pos_ids."""
    _rope("apply_rope_pos_ids_inplace", q, k, pos_ids, rotary_dim, interleave,
          lambda rd: rope_inv_freq(rd, rope_scale, rope_theta))


def apply_llama31_rope_pos_ids_inplace(q: torch.Tensor, k: torch.Tensor, pos_ids: torch.Tensor,
                                       rotary_dim: Optional[int] = None, interleave: bool = False,
                                       rope_scale: float = 8, rope_theta: float = 5e5,
                                       low_freq_factor: float = 1, high_freq_factor: float = 4,
                                       old_context_len: int = 8192) -> None:
    """flashinfer.apply_llama31_rope_pos_ids_inplace (llama3.py:660-669; spec
    pie/src/flashinfer_metal/ops.py:306-346 + kernels/metal_rope.metal:26-107)."""
    _rope("apply_llama31_rope_pos_ids_inplace", q, k, pos_ids, rotary_dim, interleave,
          lambda rd: llama31_inv_freq(rd, rope_scale, rope_theta, low_freq_factor,
                                      high_freq_factor, old_context_len))


def apply_rope_with_cos_sin_cache_inplace(positions: torch.Tensor, query: torch.Tensor,
                                          key: torch.Tensor, head_size: int,
                                          cos_sin_cache: torch.Tensor, is_neox: bool = True) -> None:
    """flashinfer.apply_rope_with_cos_sin_cache_inplace (gpt_oss.py:671-678, olmo3.py:797-804):
    query [nnz, Hq*head_size] (or [nnz, Hq, head_size]) and key likewise, rotated in place with
    cos/sin read from ``cos_sin_cache`` [max_pos, rotary_dim] fp32 (cos in the first half, sin in
    the second). is_neox=True pairs (i, i + rotary_dim/2), else (2i, 2i+1). Positions outside
    the table leave their token unchanged."""
    _check("apply_rope_with_cos_sin_cache_inplace", _BF16, query=query, key=key)
    _check("apply_rope_with_cos_sin_cache_inplace", torch.int32, positions=positions)
    _check("apply_rope_with_cos_sin_cache_inplace", torch.float32, cos_sin_cache=cos_sin_cache)
    D = int(head_size)
    q = query.view(query.shape[0], -1, D) if query.dim() == 2 else query
    k = key.view(key.shape[0], -1, D) if key.dim() == 2 else key
    if cos_sin_cache.dim() != 2 or cos_sin_cache.stride(1) != 1:
        raise ValueError("apply_rope_with_cos_sin_cache_inplace: cos_sin_cache must be [max_pos, rotary_dim]")
    rd = cos_sin_cache.shape[1]
    T, Hq, Hkv, D, rd = _rope_shapes("apply_rope_with_cos_sin_cache_inplace", q, k, positions, rd)
    _lib.call("pie_hip_rope_cos_sin_cache_inplace", q.data_ptr(), q.stride(0), q.stride(1),
              k.data_ptr(), k.stride(0), k.stride(1), positions.data_ptr(), T, Hq, Hkv, D,
              0 if is_neox else 1, cos_sin_cache.data_ptr(), cos_sin_cache.shape[0], rd,
              cos_sin_cache.stride(0), _stream(q))


# ----------------------------------------------------------------------------- paged KV append
def _cache_desc(paged_kv_cache, kv_layout: str, Hkv: int, D: int,
                name: str = "append_paged_kv_cache"):
    """(k_cache, v_cache, num_pages, page_stride, slot_stride, head_stride, page_size)."""
    if kv_layout not in ("NHD", "HND"):
        raise ValueError(f"{name}: kv_layout must be 'NHD' or 'HND', got {kv_layout!r}")
    if isinstance(paged_kv_cache, (tuple, list)):
        kc, vc = paged_kv_cache
        _check(name, _BF16, k_cache=kc, v_cache=vc)
        if kc.dim() != 4 or kc.shape != vc.shape or kc.stride() != vc.stride():
            raise ValueError(f"{name}: k/v caches must be matching 4-D tensors")
        sl, hd = (1, 2) if kv_layout == "NHD" else (2, 1)
        shape, st = kc.shape, kc.stride()
        k_ptr, v_ptr = kc.data_ptr(), vc.data_ptr()
        page_stride = st[0]
    else:
        c = paged_kv_cache
        _check(name, _BF16, paged_kv_cache=c)
        if c.dim() != 5 or c.shape[1] != 2:
            raise ValueError(f"{name}: cache must be [pages, 2, ...] (5-D)")
        sl, hd = (2, 3) if kv_layout == "NHD" else (3, 2)
        shape, st = c.shape, c.stride()
        k_ptr = c.data_ptr()
        v_ptr = k_ptr + st[1] * c.element_size()
        page_stride = st[0]
    if shape[hd] != Hkv or shape[-1] != D or st[-1] != 1:
        raise ValueError(f"{name}: cache shape {tuple(shape)} does not hold "
                         f"{Hkv} kv heads of dim {D} ({kv_layout})")
    return k_ptr, v_ptr, shape[0], page_stride, st[sl], st[hd], shape[sl]


def _append_checks(append_key, append_value, batch_indices, positions, kv_indices, kv_indptr,
                   kv_last_page_len):
    _check("append_paged_kv_cache", _BF16, append_key=append_key, append_value=append_value)
    _check("append_paged_kv_cache", torch.int32, batch_indices=batch_indices, positions=positions,
           kv_indices=kv_indices, kv_indptr=kv_indptr, kv_last_page_len=kv_last_page_len)
    if append_key.dim() != 3 or append_key.shape != append_value.shape:
        raise ValueError("append_paged_kv_cache: key/value must be matching [nnz, Hkv, D]")
    if append_key.stride(2) != 1 or append_value.stride(2) != 1:
        raise ValueError("append_paged_kv_cache: head dim must have unit stride")
    T = append_key.shape[0]
    for name, t in (("batch_indices", batch_indices), ("positions", positions)):
        if t.shape != (T,) or not t.is_contiguous():
            raise ValueError(f"append_paged_kv_cache: {name} must be a contiguous [{T}] tensor")
    if kv_indptr.dim() != 1 or kv_indptr.numel() < 1 or not kv_indptr.is_contiguous():
        raise ValueError("append_paged_kv_cache: kv_indptr must be a contiguous [B+1] tensor")
    if not kv_indices.is_contiguous():
        raise ValueError("append_paged_kv_cache: kv_indices must be contiguous")


def append_paged_kv_cache(append_key: torch.Tensor, append_value: torch.Tensor,
                          batch_indices: torch.Tensor, positions: torch.Tensor,
                          paged_kv_cache: Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]],
                          kv_indices: torch.Tensor, kv_indptr: torch.Tensor,
                          kv_last_page_len: torch.Tensor, kv_layout: str = "NHD") -> None:
    """flashinfer.append_paged_kv_cache (llama3.py:675-685; spec
    pie/src/flashinfer_metal/ops.py:349-389 + kernels/metal_append_paged_kv_cache.metal).

    Writes token t's k/v rows to slot positions[t] % P of page
    kv_indices[kv_indptr[batch_indices[t]] + positions[t] // P]. kv_last_page_len is accepted
    for API compatibility and, as in the reference restatement, not read.
    """
    _append_checks(append_key, append_value, batch_indices, positions, kv_indices, kv_indptr,
                   kv_last_page_len)
    T, Hkv, D = append_key.shape
    kp, vp, npages, ps, ss, hs, P = _cache_desc(paged_kv_cache, kv_layout, Hkv, D)
    _lib.call("pie_hip_paged_kv_append", append_key.data_ptr(), append_key.stride(0),
              append_key.stride(1), append_value.data_ptr(), append_value.stride(0),
              append_value.stride(1), batch_indices.data_ptr(), positions.data_ptr(),
              kv_indices.data_ptr(), kv_indptr.data_ptr(), kv_indptr.numel() - 1, kp, vp, npages,
              ps, ss, hs, P, T, Hkv, D, _stream(append_key))


def _rope_append(name, q, k, v, pos_ids, batch_indices, positions, paged_kv_cache, kv_indices,
                 kv_indptr, kv_last_page_len, kv_layout, rotary_dim, interleave, freqs):
    T, Hq, Hkv, D, rd = _rope_shapes(name, q, k, pos_ids, rotary_dim)
    _append_checks(k, v, batch_indices, positions, kv_indices, kv_indptr, kv_last_page_len)
    kp, vp, npages, ps, ss, hs, P = _cache_desc(paged_kv_cache, kv_layout, Hkv, D)
    _lib.call("pie_hip_rope_append", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
              k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), pos_ids.data_ptr(),
              T, Hq, Hkv, D, rd, 1 if interleave else 0, freqs(rd), batch_indices.data_ptr(),
              positions.data_ptr(), kv_indices.data_ptr(), kv_indptr.data_ptr(),
              kv_indptr.numel() - 1, kp, vp, npages, ps, ss, hs, P, _stream(q))


def apply_rope_pos_ids_and_append_paged_kv_cache(
        q, k, v, pos_ids, batch_indices, positions, paged_kv_cache, kv_indices, kv_indptr,
        kv_last_page_len, kv_layout="NHD", rotary_dim=None, interleave=False, rope_scale=1,
        rope_theta=1e4) -> None:
    """Fused apply_rope_pos_ids_inplace(q, k, pos_ids) + append_paged_kv_cache(k, v, ...):
    identical results (q, k rotated in place; rotated k and raw v in the cache) in one pass."""
    _rope_append("apply_rope_pos_ids_and_append_paged_kv_cache", q, k, v, pos_ids, batch_indices,
                 positions, paged_kv_cache, kv_indices, kv_indptr, kv_last_page_len, kv_layout,
                 rotary_dim, interleave, lambda rd: rope_inv_freq(rd, rope_scale, rope_theta))


def apply_llama31_rope_pos_ids_and_append_paged_kv_cache(
        q, k, v, pos_ids, batch_indices, positions, paged_kv_cache, kv_indices, kv_indptr,
        kv_last_page_len, kv_layout="NHD", rotary_dim=None, interleave=False, rope_scale=8,
        rope_theta=5e5, low_freq_factor=1, high_freq_factor=4, old_context_len=8192) -> None:
    """Fused apply_llama31_rope_pos_ids_inplace + append_paged_kv_cache (llama3.py:660-685)."""
    _rope_append("apply_llama31_rope_pos_ids_and_append_paged_kv_cache", q, k, v, pos_ids,
                 batch_indices, positions, paged_kv_cache, kv_indices, kv_indptr,
                 kv_last_page_len, kv_layout, rotary_dim, interleave,
                 lambda rd: llama31_inv_freq(rd, rope_scale, rope_theta, low_freq_factor,
                                             high_freq_factor, old_context_len))


def qk_rms_norm_rope_append(q, k, v, q_weight, k_weight, eps, pos_ids, batch_indices, positions,
                            paged_kv_cache, kv_indices, kv_indptr, kv_last_page_len,
                            kv_layout="NHD", rope_scale=1, rope_theta=1e4, q_out=None,
                            k_out=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Qwen3's attention prologue in one pass (qwen3.py:651-684):
    q, k = qk_rms_norm(q, k, q_weight, k_weight, eps);
    apply_rope_pos_ids_inplace(q, k, pos_ids, rope_scale=rope_scale, rope_theta=rope_theta);
    append_paged_kv_cache(k, v, batch_indices, positions, paged_kv_cache, ...).
    Returns the normalised, rotated (q, k) (new contiguous tensors unless q_out/k_out given);
    bit-identical to the three calls."""
    T, Hq, Hkv, D, rd = _rope_shapes("qk_rms_norm_rope_append", q, k, pos_ids, None)
    _check("qk_rms_norm_rope_append", _BF16, q_weight=q_weight, k_weight=k_weight)
    if q_weight.shape != (D,) or k_weight.shape != (D,):
        raise ValueError("qk_rms_norm_rope_append: weights must be [D]")
    _append_checks(k, v, batch_indices, positions, kv_indices, kv_indptr, kv_last_page_len)
    q_out = torch.empty((T, Hq, D), dtype=_BF16, device=q.device) if q_out is None else q_out
    k_out = torch.empty((T, Hkv, D), dtype=_BF16, device=k.device) if k_out is None else k_out
    if q_out.shape != q.shape or k_out.shape != k.shape or q_out.stride(2) != 1 or k_out.stride(2) != 1:
        raise ValueError("qk_rms_norm_rope_append: outputs must match inputs with unit inner stride")
    kp, vp, npages, ps, ss, hs, P = _cache_desc(paged_kv_cache, kv_layout, Hkv, D)
    q_weight, k_weight = q_weight.contiguous(), k_weight.contiguous()
    _keep(q, k, v, q_out, k_out, q_weight, k_weight, pos_ids, batch_indices, positions,
          paged_kv_cache, kv_indices, kv_indptr)
    _lib.call("pie_hip_qk_rmsnorm_rope_append", q.data_ptr(), q.stride(0), q.stride(1),
              k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1),
              q_out.data_ptr(), q_out.stride(0), q_out.stride(1), k_out.data_ptr(),
              k_out.stride(0), k_out.stride(1), q_weight.data_ptr(), k_weight.data_ptr(),
              C.c_float(_eps(eps)), pos_ids.data_ptr(), T, Hq, Hkv, D,
              rope_inv_freq(D, rope_scale, rope_theta), batch_indices.data_ptr(),
              positions.data_ptr(), kv_indices.data_ptr(), kv_indptr.data_ptr(),
              kv_indptr.numel() - 1, kp, vp, npages, ps, ss, hs, P, _stream(q))
    return q_out, k_out


# ----------------------------------------------------------------------------- index helpers
def get_seq_lens(kv_indptr: torch.Tensor, kv_last_page_len: torch.Tensor,
                 page_size: int) -> torch.Tensor:
    """flashinfer.get_seq_lens (llama3.py:745-749; spec flashinfer_metal/ops.py:392-407)."""
    _check("get_seq_lens", torch.int32, kv_indptr=kv_indptr, kv_last_page_len=kv_last_page_len)
    B = kv_indptr.numel() - 1
    if B < 0 or kv_last_page_len.numel() < B:
        raise ValueError("get_seq_lens: kv_indptr must be [B+1] and kv_last_page_len [B]")
    kv_indptr, kv_last_page_len = kv_indptr.contiguous(), kv_last_page_len.contiguous()
    out = torch.empty(B, dtype=torch.int32, device=kv_indptr.device)
    _lib.call("pie_hip_get_seq_lens", kv_indptr.data_ptr(), kv_last_page_len.data_ptr(), B,
              int(page_size), out.data_ptr(), _stream(kv_indptr))
    return out


def get_batch_indices_positions(append_indptr: torch.Tensor, seq_lens: torch.Tensor,
                                nnz: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """flashinfer.get_batch_indices_positions (llama3.py:751-755; spec
    flashinfer_metal/ops.py:410-436). Entries of tokens outside every request are
    uninitialised, as with the reference's torch.empty."""
    _check("get_batch_indices_positions", torch.int32, append_indptr=append_indptr,
           seq_lens=seq_lens)
    B = append_indptr.numel() - 1
    if B < 0 or seq_lens.numel() < B:
        raise ValueError("get_batch_indices_positions: append_indptr must be [B+1], seq_lens [B]")
    append_indptr, seq_lens = append_indptr.contiguous(), seq_lens.contiguous()
    nnz = int(nnz)
    bidx = torch.empty(nnz, dtype=torch.int32, device=append_indptr.device)
    pos = torch.empty(nnz, dtype=torch.int32, device=append_indptr.device)
    _lib.call("pie_hip_get_batch_indices_positions", append_indptr.data_ptr(), seq_lens.data_ptr(),
              B, nnz, bidx.data_ptr(), pos.data_ptr(), _stream(append_indptr))
    return bidx, pos
