"""Install pie_amd.ops under the module names Pie's model files import.

The model files choose their kernel namespace at import time
(pie/src/pie_worker/model/llama3.py:18-21, qwen3.py:18-21; the same in every model file):

    if is_apple_silicon(): import flashinfer_metal as ops
    else:                  import flashinfer as ops

``install()`` registers a module named ``flashinfer`` whose hot-path functions are this
package's gfx950 kernels, as are the paged-attention wrappers and the ``flashinfer.sampling``
submodule (Pie's samplers, pie/src/pie_worker/model/common.py:13-28). Any other attribute raises
AttributeError naming the op, so one model run never mixes two kernel backends silently; pass
``forward_unserved=True`` to look unserved names up in a real flashinfer package instead. Call it
before the model modules are imported; it is idempotent.

The model files also call ``torch.nn.functional`` inline, bound as ``fun`` at import
(llama3.py:7, qwen3.py:9): ``install_functional(module)`` rebinds that name to a namespace whose
``rms_norm`` and ``embedding`` run this package's kernels (llama3.py:471, :555, :618; qwen3.py:651-662),
and ``patch_mlp(cls)`` replaces a Llama-style ``ForwardPass.mlp`` (llama3.py:543-586,
qwen3.py:526-571) with one that runs ``fun.silu(gate) * up`` as one SiLU-and-mul kernel. Neither
edits the model files.

``PIE_HIP_OPS=0`` in the environment turns all three into no-ops, so the same launch script runs
the reference path (the real flashinfer and torch) for A/B comparisons; the kernels themselves
never fall back to anything.
"""
from __future__ import annotations

import importlib
import os
import sys
import types

import torch
import torch.nn.functional as _F

from . import _lib, attention, ops, sampling

# flashinfer names this package serves (the calls at llama3.py:660-755, qwen3.py:665-684,
# gemma2.py:608, gpt_oss.py:671-678).
HOT_PATH = (
    "apply_rope_pos_ids_inplace",
    "apply_llama31_rope_pos_ids_inplace",
    "append_paged_kv_cache",
    "get_seq_lens",
    "get_batch_indices_positions",
    "rmsnorm",
    "fused_add_rmsnorm",
    "silu_and_mul",
    "gelu_tanh_and_mul",
    "apply_rope_with_cos_sin_cache_inplace",
)
# flashinfer's attention wrapper classes (llama3.py:293-313)
ATTENTION = ("BatchDecodeWithPagedKVCacheWrapper", "BatchPrefillWithPagedKVCacheWrapper",
             "BatchAttentionWithAttentionSinkWrapper")  # the last: gpt_oss.py:420-438


def enabled() -> bool:
    """False when PIE_HIP_OPS=0: install(), install_functional() and patch_mlp() leave the
    reference path in place."""
    return os.environ.get("PIE_HIP_OPS", "1").strip() != "0"


class _Namespace(types.ModuleType):
    def __init__(self, name: str, fallback):
        super().__init__(name, "pie_amd kernels for the per-layer hot path; other names from "
                               + (fallback.__name__ if fallback else "nowhere"))
        self._fallback = fallback
        for n in HOT_PATH:
            setattr(self, n, getattr(ops, n))
        for n in ATTENTION:
            setattr(self, n, getattr(attention, n))
        self.sampling = sampling  # `from flashinfer.sampling import ...` (common.py:13-28)

    def __getattr__(self, item):
        if item.startswith("__"):
            raise AttributeError(item)
        fb = self.__dict__.get("_fallback")
        if not self.__dict__.get("_forward", False) or fb is None:
            raise AttributeError(
                f"flashinfer.{item} is not provided by pie_amd (its gfx950 kernels serve "
                f"{', '.join(HOT_PATH + ATTENTION)} and flashinfer.sampling); "
                + ("no flashinfer package is installed" if fb is None else
                   "install(forward_unserved=True) would take it from the installed flashinfer"))
        return getattr(fb, item)


def install(name: str = "flashinfer", forward_unserved: bool = False) -> types.ModuleType:
    """Make ``import <name>`` return the pie_amd namespace; returns that module. With
    forward_unserved=True, names this package does not serve come from the real package. With
    PIE_HIP_OPS=0 nothing is installed and the real package (None if absent) is returned."""
    cur = sys.modules.get(name)
    if not enabled():
        if isinstance(cur, _Namespace):
            return cur
        try:
            return cur if cur is not None else importlib.import_module(name)
        except ImportError:
            return None
    if isinstance(cur, _Namespace):
        cur._forward = forward_unserved
        return cur
    fallback = cur
    if fallback is None and forward_unserved:
        try:
            fallback = importlib.import_module(name)
        except ImportError:
            fallback = None
    mod = _Namespace(name, fallback)
    mod._forward = forward_unserved
    sys.modules[name] = mod
    mod._saved_sampling = sys.modules.get(name + ".sampling")
    sys.modules[name + ".sampling"] = sampling
    return mod


def uninstall(name: str = "flashinfer") -> None:
    """Undo install(): restore the real module (if any)."""
    cur = sys.modules.get(name)
    if isinstance(cur, _Namespace):
        if cur._saved_sampling is not None:
            sys.modules[name + ".sampling"] = cur._saved_sampling
        else:
            sys.modules.pop(name + ".sampling", None)
        if cur._fallback is not None:
            sys.modules[name] = cur._fallback
        else:
            del sys.modules[name]


# ----------------------------------------------------------------------------- torch.nn.functional
class _Functional(types.ModuleType):
    """``torch.nn.functional`` with the per-layer hot-path ops on this package's kernels.

    rms_norm over the last dimension of a GPU tensor (llama3.py:555-560, :618-623; qwen3.py:651-662
    on [T, H, D] views) runs pie_hip_rmsnorm / pie_hip_qk_rmsnorm; embedding from a GPU table with
    int32 (or int64, narrowed on the device) ids (llama3.py:471, qwen3.py:468-472) runs
    pie_hip_embedding. GPU calls these kernels cannot serve (non-bf16 tensors, a multi-dimension
    normalized_shape, padding_idx / max_norm) raise instead of running another implementation.
    CPU tensors, and every other name (linear, ...), are torch's.
    """

    def __init__(self):
        super().__init__("pie_amd.functional", "torch.nn.functional with pie_amd hot-path kernels")

    def __getattr__(self, item):
        return getattr(_F, item)

    @staticmethod
    def rms_norm(input, normalized_shape, weight=None, eps=None):
        if not input.is_cuda:
            return _F.rms_norm(input, normalized_shape, weight, eps)
        shape = (normalized_shape,) if isinstance(normalized_shape, int) else tuple(normalized_shape)
        if weight is None or len(shape) != 1:
            raise NotImplementedError("pie_amd rms_norm: one normalised dimension and a weight")
        return ops.rms_norm(input, shape, weight, eps)

    @staticmethod
    def embedding(input, weight, padding_idx=None, max_norm=None, norm_type=2.0,
                  scale_grad_by_freq=False, sparse=False):
        if not weight.is_cuda:
            return _F.embedding(input, weight, padding_idx, max_norm, norm_type,
                                scale_grad_by_freq, sparse)
        if padding_idx is not None or max_norm is not None:
            raise NotImplementedError("pie_amd embedding: padding_idx / max_norm")
        ids = input.to(torch.int32) if input.dtype == torch.int64 else input
        return ops.embedding(ids, weight)


functional = _Functional()


def install_functional(*modules) -> None:
    """Rebind ``fun`` (torch.nn.functional) in the given model modules to ``functional``; loads
    the kernel library first, so a missing library fails here, not on the first call. With
    PIE_HIP_OPS=0 the modules keep torch.nn.functional."""
    if not enabled():
        return
    _lib.load()
    for m in modules:
        if getattr(m, "fun", None) is not _F and getattr(m, "fun", None) is not functional:
            raise ValueError(f"{m.__name__}: `fun` is not torch.nn.functional")
        m.fun = functional


def uninstall_functional(*modules) -> None:
    for m in modules:
        if getattr(m, "fun", None) is functional:
            m.fun = _F


def _mlp(self, hidden_states: torch.Tensor, layer_idx: int) -> torch.Tensor:
    """A Llama-style ForwardPass.mlp (llama3.py:543-586, qwen3.py:526-571): pre-norm, the fused
    gate/up projection ([gate; up] rows, llama3.py:68-80), SiLU(gate) * up, the down projection,
    the TP all-reduce, the residual add. The norm and SiLU-and-mul run this package's kernels
    (the activation in one pass instead of silu, mul and a temporary); the GEMMs and the
    all-reduce are torch's, as in the reference."""
    cfg = self.model_config
    w = self.weights.get
    normed = functional.rms_norm(hidden_states, [cfg.dim_hidden], w(f"layers.{layer_idx}.norm_mlp"),
                                 cfg.rms_norm_eps)
    gate_up = _F.linear(normed, w(f"layers.{layer_idx}.proj_gate_up"))
    act = ops.silu_and_mul(gate_up)
    down = _F.linear(act, w(f"layers.{layer_idx}.proj_down"))
    if getattr(self, "tp_size", 1) > 1:
        torch.distributed.all_reduce(down, group=self.compute_process_group)
    return hidden_states + down


def patch_mlp(cls) -> None:
    """Replace ``cls.mlp`` (a Llama-style ForwardPass: llama3, qwen2, qwen3, mistral3) with _mlp;
    ``unpatch_mlp`` restores it. With PIE_HIP_OPS=0 the class keeps its own mlp."""
    if not enabled():
        return
    _lib.load()
    if getattr(cls, "_pie_amd_mlp", None) is None:
        cls._pie_amd_mlp = cls.mlp
        cls.mlp = _mlp


def unpatch_mlp(cls) -> None:
    orig = getattr(cls, "_pie_amd_mlp", None)
    if orig is not None:
        cls.mlp = orig
        cls._pie_amd_mlp = None
