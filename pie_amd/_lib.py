"""ctypes binding of libpie_hip.so (declared in include/pie_hip.h).

The library is the only compute path: if it is missing or fails to load, every op raises.
There is no CPU or torch fallback.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("PIE_HIP_LIB", _PKG / "libpie_hip.so"))
HEADER = _PKG.parent / "include" / "pie_hip.h"

i64, i32, f32, vp = C.c_int64, C.c_int, C.c_float, C.c_void_p
u64 = C.c_uint64

# name -> argtypes (restype is int for all but pie_hip_last_error)
SIGNATURES: dict[str, list] = {
    "pie_hip_abi_version": [],
    "pie_hip_rmsnorm": [vp, i64, vp, vp, i64, i64, i64, f32, vp],
    "pie_hip_fused_add_rmsnorm": [vp, i64, vp, i64, vp, i64, vp, i64, vp, i64, i64, f32, vp],
    "pie_hip_gemma_rmsnorm": [vp, i64, vp, vp, i64, i64, i64, f32, vp],
    "pie_hip_gemma_fused_add_rmsnorm": [vp, i64, vp, i64, vp, i64, vp, i64, vp, i64, i64, f32, vp],
    "pie_hip_gemma_qk_rmsnorm": [vp, i64, i64, vp, i64, i64, vp, i64, i64, vp, i64, i64, vp, vp,
                                 i64, i64, i64, i64, f32, vp],
    "pie_hip_gelu_tanh_and_mul": [vp, i64, vp, i64, i64, i64, vp],
    "pie_hip_embedding_scaled": [vp, i64, vp, i64, i64, i64, vp, i64, f32, vp],
    "pie_hip_rope_cos_sin_cache_inplace": [vp, i64, i64, vp, i64, i64, vp, i64, i64, i64, i64, i32,
                                           vp, i64, i64, i64, vp],
    "pie_hip_qk_rmsnorm": [vp, i64, i64, vp, i64, i64, vp, i64, i64, vp, i64, i64, vp, vp,
                           i64, i64, i64, i64, f32, vp],
    "pie_hip_silu_and_mul": [vp, i64, vp, i64, i64, i64, vp],
    "pie_hip_embedding": [vp, i64, vp, i64, i64, i64, vp, i64, vp],
    "pie_hip_rope_inplace": [vp, i64, i64, vp, i64, i64, vp, i64, i64, i64, i64, i64, i32, vp, vp],
    "pie_hip_rope_inv_freq": [vp, i64, f32, f32],
    "pie_hip_llama31_inv_freq": [vp, i64, f32, f32, f32, f32, f32],
    "pie_hip_paged_kv_append": [vp, i64, i64, vp, i64, i64, vp, vp, vp, vp, i64, vp, vp, i64,
                                i64, i64, i64, i64, i64, i64, i64, vp],
    "pie_hip_rope_append": [vp, i64, i64, vp, i64, i64, vp, i64, i64, vp, i64, i64, i64, i64,
                            i64, i32, vp, vp, vp, vp, vp, i64, vp, vp, i64, i64, i64, i64, i64,
                            vp],
    "pie_hip_qk_rmsnorm_rope_append": [vp, i64, i64, vp, i64, i64, vp, i64, i64, vp, i64, i64, vp,
                                       i64, i64, vp, vp, f32, vp, i64, i64, i64, i64, vp, vp, vp,
                                       vp, vp, i64, vp, vp, i64, i64, i64, i64, i64, vp],
    "pie_hip_attention_decode_plan": [i64, i64, i64, i64, vp],
    "pie_hip_attention_decode": [vp, i64, i64, vp, vp, i64, i64, i64, i64, vp, vp, vp, i64, i64,
                                 i64, i64, i64, f32, i64, vp, i64, vp, i64, vp, i64, i64, vp],
    "pie_hip_attention_decode_noalloc": [vp, i64, i64, vp, vp, i64, i64, i64, i64, vp, vp, vp, i64,
                                         i64, i64, i64, i64, f32, i64, vp, i64, vp, i64, i64, vp],
    "pie_hip_attention_prefill_plan": [vp, vp, vp, i64, i64, i64, i64, i64, i32, vp, i64, vp, vp,
                                       vp, vp],
    "pie_hip_attention_pack_mask": [vp, vp, vp, vp, vp, i64, i64, i64, i64, vp, vp, vp],
    "pie_hip_attention_prefill": [vp, i64, i64, vp, vp, i64, i64, i64, i64, vp, vp, vp, vp, i64,
                                  i64, i64, i64, f32, i32, i64, vp, vp, vp, vp, i64, i64, vp, i64,
                                  i64, vp],
    "pie_hip_sample": [vp, i64, i64, i64, i64, vp, i32, vp, i32, vp, f32, vp, f32, vp, u64, u64, vp, vp],
    "pie_hip_scaled_softmax": [vp, i32, i64, i64, i64, vp, f32, vp, i64, vp],
    "pie_hip_group_begin": [],
    "pie_hip_group_end": [vp],
    "pie_hip_group_save": [vp, vp],
    "pie_hip_group_launch": [vp, vp],
    "pie_hip_get_seq_lens": [vp, vp, i64, i64, vp, vp],
    "pie_hip_get_batch_indices_positions": [vp, vp, i64, i64, vp, vp, vp],
}
ABI_VERSION = 3

_lib: C.CDLL | None = None


class PieHipError(RuntimeError):
    """A kernel entry point returned a nonzero status."""


def header_symbols() -> list[str]:
    """Every function name declared in include/pie_hip.h."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(pie_hip_[a-z0-9_]+)\s*\(", text)))


def load() -> C.CDLL:
    """Load (once) and return the kernel library; raises if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"pie_amd: kernel library {LIB_PATH} not built; run `python -m pie_amd.build` "
            "(there is no fallback path)")
    lib = C.CDLL(str(LIB_PATH))
    lib.pie_hip_last_error.restype = C.c_char_p
    lib.pie_hip_last_error.argtypes = []
    lib.pie_hip_group_free.restype = None
    lib.pie_hip_group_free.argtypes = [C.c_void_p]
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = C.c_int
        fn.argtypes = argtypes
    if lib.pie_hip_abi_version() != ABI_VERSION:
        raise ImportError(f"pie_amd: {LIB_PATH} has ABI {lib.pie_hip_abi_version()}, "
                          f"expected {ABI_VERSION}; rebuild it")
    _lib = lib
    return lib


_fns: dict = {}


def call(name: str, *args) -> None:
    """Invoke an entry point and raise PieHipError with the library's message on failure."""
    fn = _fns.get(name)
    if fn is None:
        fn = _fns[name] = getattr(load(), name)
    rc = fn(*args)
    if rc != 0:
        msg = load().pie_hip_last_error().decode(errors="replace")
        if rc == 1:
            raise ValueError(f"{name}: {msg}")
        raise PieHipError(f"{name} failed ({rc}): {msg}")
