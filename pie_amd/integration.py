"""Install pie_amd.ops under the module names Pie's model files import.

The model files choose their kernel namespace at import time
(pie/src/pie_worker/model/llama3.py:18-21, qwen3.py:18-21; the same in every model file):

    if is_apple_silicon(): import flashinfer_metal as ops
    else:                  import flashinfer as ops

``install()`` registers a module named ``flashinfer`` whose hot-path functions are this
package's gfx950 kernels, as are the paged-attention wrappers and the ``flashinfer.sampling``
submodule (Pie's samplers, pie/src/pie_worker/model/common.py:13-28). Every other attribute is
looked up in the real flashinfer package when one is importable, and raises AttributeError
otherwise. Call it before the model modules are imported; it is idempotent.
"""
from __future__ import annotations

import importlib
import sys
import types

from . import attention, ops, sampling

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
ATTENTION = ("BatchDecodeWithPagedKVCacheWrapper", "BatchPrefillWithPagedKVCacheWrapper")


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
        fb = self.__dict__.get("_fallback")
        if fb is None:
            raise AttributeError(f"flashinfer.{item} is not provided by pie_amd and no flashinfer "
                                 "package is installed")
        return getattr(fb, item)


def install(name: str = "flashinfer") -> types.ModuleType:
    """Make ``import <name>`` return the pie_amd namespace; returns that module."""
    cur = sys.modules.get(name)
    if isinstance(cur, _Namespace):
        return cur
    fallback = cur
    if fallback is None:
        try:
            fallback = importlib.import_module(name)
        except ImportError:
            fallback = None
    mod = _Namespace(name, fallback)
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
