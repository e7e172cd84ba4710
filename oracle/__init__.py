"""CPU oracle for Pie's per-layer hot path — TEST INFRASTRUCTURE ONLY.

This package is the checker the HIP kernels are compared against. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it; the
product (``pie_amd``) never does and has no CPU fallback.

The arithmetic lives in ``oracle.c`` (float64 math, explicit bf16 round-to-nearest-even);
this module wraps it for numpy arrays (bf16 as uint16 bit patterns) and torch tensors.
Each function cites the reference behaviour it restates (paths in the zyma98/pie repository):

  rmsnorm / add_rmsnorm   torch rms_norm (torch/_decomp/decompositions.py:1760-1810) as called
                          at pie/src/pie_worker/model/llama3.py:555-560, :586; qwen3.py:651-662
  silu_and_mul            llama3.py:569-572 (torch's double rounding, mode 0)
  embedding               llama3.py:471
  rope / inv_freq_*       pie/src/flashinfer_metal/kernels/metal_rope.metal:26-107
  append                  pie/src/flashinfer_metal/kernels/metal_append_paged_kv_cache.metal:23-107
  seq_lens, batch_indices_positions   pie/src/flashinfer_metal/ops.py:392-436
  scaled_softmax          pie/src/pie_worker/model/common.py:38-59, :68-188 (safe_scaled_softmax)
  sample                  flashinfer.sampling.*_sampling_from_probs as called at common.py:316-344
  attention               flashinfer Batch{Prefill,Decode}WithPagedKVCacheWrapper.run, restated in
                          pie/src/flashinfer_metal/ops.py:163-282 and
                          kernels/metal_attention_simdgroup_opt.metal:120-470; custom masks as
                          built at pie/src/pie_worker/batching.py:335-386

How each function is pinned (tests/test_oracle.py): against torch-CPU running the
reference's own expressions (rmsnorm, add, silu*mul, embedding), against transformers'
Llama-3 frequency rule and HF rotate-half RoPE (rope), against brute-force Python loops
(append, index helpers), against the committed golden fixtures, and against closed-form
invariants (pos=0 identity, pair-norm preservation, rotation composition, scale invariance).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "_build" / "liboracle.so"
_lib = None

_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
i64 = C.c_int64


def build() -> Path:
    """Compile oracle.c (make -C oracle)."""
    subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not _LIB_PATH.exists() or _LIB_PATH.stat().st_mtime < (_DIR / "oracle.c").stat().st_mtime:
        build()
    lib = C.CDLL(str(_LIB_PATH))
    sig = {
        "oracle_rmsnorm": (None, [_u16p, i64, i64, _u16p, _u16p, i64, i64, i64, i64, i64, C.c_double]),
        "oracle_add_rmsnorm": (None, [_u16p, _u16p, _u16p, _u16p, _u16p, i64, i64, C.c_double]),
        "oracle_silu_and_mul": (None, [_u16p, i64, _u16p, i64, i64, C.c_int]),
        "oracle_embedding": (i64, [_i32p, i64, _u16p, i64, i64, _u16p]),
        "oracle_inv_freq_std": (None, [_f64p, i64, C.c_double, C.c_double]),
        "oracle_inv_freq_llama31": (None, [_f64p, i64, C.c_double, C.c_double, C.c_double,
                                           C.c_double, C.c_double]),
        "oracle_rope": (None, [_u16p, i64, i64, _u16p, i64, i64, _i32p, i64, i64, i64, i64,
                               C.c_int, _f64p]),
        "oracle_append": (i64, [_u16p, i64, i64, _u16p, i64, i64, _i32p, _i32p, _i32p, _i32p, i64,
                                C.c_void_p, C.c_void_p, i64, i64, i64, i64, i64, i64, i64, i64]),
        "oracle_seq_lens": (None, [_i32p, _i32p, i64, i64, _i32p]),
        "oracle_batch_indices_positions": (None, [_i32p, _i32p, i64, i64, _i32p, _i32p]),
        "oracle_gemma_rmsnorm": (None, [_u16p, i64, i64, _u16p, _u16p, i64, i64, i64, i64, i64, C.c_double]),
        "oracle_gemma_add_rmsnorm": (None, [_u16p, _u16p, _u16p, _u16p, _u16p, i64, i64, C.c_double]),
        "oracle_gelu_tanh_and_mul": (None, [_u16p, i64, _u16p, i64, i64]),
        "oracle_embedding_scaled": (i64, [_i32p, i64, _u16p, i64, i64, C.c_float, _u16p]),
        "oracle_rope_cs": (None, [_u16p, i64, i64, _u16p, i64, i64, _i32p, i64, i64, i64, i64,
                                  C.c_int, _f32p, i64, i64]),
        "oracle_attention": (None, [_u16p, i64, i64, C.c_void_p, C.c_void_p, i64, i64, i64,
                                    _i32p, _i32p, _i32p, _i32p, C.c_void_p, C.c_void_p, C.c_int, i64, i64, i64,
                                    i64, i64, i64, C.c_double, _u16p, i64, i64, C.c_void_p,
                                    C.c_void_p]),
        "oracle_scaled_softmax": (None, [_f32p, i64, i64, _f32p, C.c_double, _f64p]),
        "oracle_sample": (None, [_f32p, i64, i64, i64, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                 _f64p, _i32p, C.c_void_p]),
        "oracle_f32_to_bf16": (C.c_uint16, [C.c_float]),
        "oracle_f64_to_bf16": (C.c_uint16, [C.c_double]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


# ----------------------------------------------------------------------------- bf16 helpers
def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 values (exact)."""
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (vectorised; matches oracle.c f2bf)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def to_np(t) -> np.ndarray:
    """torch bf16/int32 tensor (any device) -> numpy uint16/int32 copy, C-contiguous."""
    import torch
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().copy()


def to_torch(a: np.ndarray, device="cpu"):
    """numpy uint16 (bf16 bits) or int32 -> torch tensor."""
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(device)
    return torch.from_numpy(a.copy()).to(device)


# ----------------------------------------------------------------------------- ops
def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """x [..., H] bf16 bits -> y [..., H] (contiguous input)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    H = x.shape[-1]
    rows = x.size // H if H else 0
    y = np.empty_like(x)
    _load().oracle_rmsnorm(x, H, 0, np.ascontiguousarray(w, np.uint16), y, H, 0, rows, 1, H, eps)
    return y


def add_rmsnorm(x: np.ndarray, r: np.ndarray, w: np.ndarray, eps: float):
    """Returns (y, s): s = bf16(r + x) (the new residual), y = rmsnorm(s)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    r = np.ascontiguousarray(r, dtype=np.uint16)
    H = x.shape[-1]
    s, y = np.empty_like(x), np.empty_like(x)
    _load().oracle_add_rmsnorm(x, r, np.ascontiguousarray(w, np.uint16), s, y, x.size // H, H, eps)
    return y, s


def silu_and_mul(gu: np.ndarray, mode: int = 0) -> np.ndarray:
    """gu [..., 2I] -> [..., I]; mode 0 = torch rounding (silu rounded to bf16 first)."""
    gu = np.ascontiguousarray(gu, dtype=np.uint16)
    I = gu.shape[-1] // 2
    rows = gu.size // (2 * I) if I else 0
    out = np.empty((*gu.shape[:-1], I), dtype=np.uint16)
    _load().oracle_silu_and_mul(gu, 2 * I, out, rows, I, mode)
    return out


def gemma_rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """Gemma RMSNorm with bf16 rounding after every torch op (gemma2.py:514-526)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    H = x.shape[-1]
    y = np.empty_like(x)
    _load().oracle_gemma_rmsnorm(x, H, 0, np.ascontiguousarray(w, np.uint16), y, H, 0,
                                 x.size // H if H else 0, 1, H, eps)
    return y


def gemma_add_rmsnorm(x: np.ndarray, r: np.ndarray, w: np.ndarray, eps: float):
    """Returns (y, s): s = bf16(r + x), y = gemma_rmsnorm(s)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    r = np.ascontiguousarray(r, dtype=np.uint16)
    H = x.shape[-1]
    s, y = np.empty_like(x), np.empty_like(x)
    _load().oracle_gemma_add_rmsnorm(x, r, np.ascontiguousarray(w, np.uint16), s, y, x.size // H, H, eps)
    return y, s


def gelu_tanh_and_mul(gu: np.ndarray) -> np.ndarray:
    gu = np.ascontiguousarray(gu, dtype=np.uint16)
    I = gu.shape[-1] // 2
    out = np.empty((*gu.shape[:-1], I), dtype=np.uint16)
    _load().oracle_gelu_tanh_and_mul(gu, 2 * I, out, gu.size // (2 * I) if I else 0, I)
    return out


def embedding_scaled(ids: np.ndarray, W: np.ndarray, scale: float):
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    W = np.ascontiguousarray(W, dtype=np.uint16)
    V, H = W.shape
    out = np.empty((ids.size, H), dtype=np.uint16)
    bad = _load().oracle_embedding_scaled(ids, ids.size, W, V, H, float(np.float32(scale)), out)
    return out, int(bad)


def rope_cos_sin(q: np.ndarray, k: np.ndarray, pos, cos_sin: np.ndarray, interleave=False):
    """Rotated copies of q [T,Hq,D], k [T,Hkv,D] with cos/sin from a [rows, rd] fp32 table."""
    q = np.array(q, dtype=np.uint16, order="C", copy=True)
    k = np.array(k, dtype=np.uint16, order="C", copy=True)
    cs = np.ascontiguousarray(cos_sin, dtype=np.float32)
    T, Hq, D = q.shape
    _load().oracle_rope_cs(q, Hq * D, D, k, k.shape[1] * D, D, np.ascontiguousarray(pos, np.int32),
                           T, Hq, k.shape[1], cs.shape[1], 1 if interleave else 0, cs,
                           cs.shape[0], cs.shape[1])
    return q, k


def embedding(ids: np.ndarray, W: np.ndarray):
    """Returns (out [T,H], n_out_of_range)."""
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    W = np.ascontiguousarray(W, dtype=np.uint16)
    V, H = W.shape
    out = np.empty((ids.size, H), dtype=np.uint16)
    bad = _load().oracle_embedding(ids, ids.size, W, V, H, out)
    return out, int(bad)


def inv_freq_std(rd: int, rope_scale: float = 1.0, rope_theta: float = 1e4) -> np.ndarray:
    f = np.empty(rd // 2, dtype=np.float64)
    _load().oracle_inv_freq_std(f, rd, rope_scale, rope_theta)
    return f


def inv_freq_llama31(rd: int, rope_scale=8.0, rope_theta=5e5, low_freq_factor=1.0,
                     high_freq_factor=4.0, old_context_len=8192.0) -> np.ndarray:
    f = np.empty(rd // 2, dtype=np.float64)
    _load().oracle_inv_freq_llama31(f, rd, rope_scale, rope_theta, low_freq_factor,
                                    high_freq_factor, old_context_len)
    return f


def rope(q: np.ndarray, k: np.ndarray, pos: np.ndarray, inv_freq: np.ndarray,
         rotary_dim: int | None = None, interleave: bool = False):
    """Returns rotated copies of q [T,Hq,D] and k [T,Hkv,D]."""
    q = np.array(q, dtype=np.uint16, order="C", copy=True)
    k = np.array(k, dtype=np.uint16, order="C", copy=True)
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    rd = D if rotary_dim is None else rotary_dim
    _load().oracle_rope(q, Hq * D, D, k, Hkv * D, D, np.ascontiguousarray(pos, np.int32), T, Hq,
                        Hkv, rd, 1 if interleave else 0,
                        np.ascontiguousarray(inv_freq, np.float64))
    return q, k


def append(k: np.ndarray, v: np.ndarray, batch_indices, positions, cache: np.ndarray,
           kv_indices, kv_indptr, layout: str = "NHD") -> int:
    """Append k/v [T,Hkv,D] into cache [pages, 2, P, Hkv, D] (NHD) or [pages, 2, Hkv, P, D]
    (HND), in place. Returns the number of tokens written."""
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    assert cache.flags.c_contiguous and cache.dtype == np.uint16
    T, Hkv, D = k.shape
    npages = cache.shape[0]
    if layout == "NHD":
        P = cache.shape[2]
        ss, hs = Hkv * D, D
    else:
        P = cache.shape[3]
        ss, hs = D, P * D
    ps = 2 * P * Hkv * D
    base = cache.ctypes.data
    return int(_load().oracle_append(
        k, Hkv * D, D, v, Hkv * D, D, np.ascontiguousarray(batch_indices, np.int32),
        np.ascontiguousarray(positions, np.int32), np.ascontiguousarray(kv_indices, np.int32),
        np.ascontiguousarray(kv_indptr, np.int32), len(kv_indptr) - 1, base,
        base + P * Hkv * D * 2, npages, ps, ss, hs, P, T, Hkv, D))


def seq_lens(kv_indptr, last_page_len, page_size: int) -> np.ndarray:
    kv_indptr = np.ascontiguousarray(kv_indptr, np.int32)
    B = kv_indptr.size - 1
    out = np.empty(B, dtype=np.int32)
    _load().oracle_seq_lens(kv_indptr, np.ascontiguousarray(last_page_len, np.int32), B,
                            page_size, out)
    return out


def batch_indices_positions(append_indptr, seq_lens_, nnz: int, fill: int = -1):
    """Returns (batch_indices, positions) int32 [nnz]; tokens outside every request = fill."""
    append_indptr = np.ascontiguousarray(append_indptr, np.int32)
    B = append_indptr.size - 1
    bidx = np.full(nnz, fill, dtype=np.int32)
    pos = np.full(nnz, fill, dtype=np.int32)
    _load().oracle_batch_indices_positions(append_indptr, np.ascontiguousarray(seq_lens_, np.int32),
                                           B, nnz, bidx, pos)
    return bidx, pos


def attention(q: np.ndarray, cache: np.ndarray, qo_indptr, kv_indptr, kv_indices, last_page_len,
              custom_mask=None, sm_scale: float | None = None, layout: str = "NHD",
              return_lse: bool = False, causal: bool = True, window_left: int = -1, sinks=None):
    """Paged attention over cache [pages, 2, P, Hkv, D] (NHD) or [pages, 2, Hkv, P, D] (HND).
    q [T, Hq, D] bf16 bits -> out [T, Hq, D] bf16 bits (and lse [T, Hq] float64, natural log).
    custom_mask: flat bool/uint8, per request a row-major [qo_len, kv_len] block, concatenated
    in request order; None means the causal window t <= kv_len - qo_len + i (causal=True) or
    every cached position (causal=False); window_left >= 0 also hides positions before
    kv_len - qo_len + i - window_left (flashinfer's sliding window). sinks: optional float32 [Hq]
    attention-sink logits (gpt-oss): each head's denominator gains exp(sinks[h])."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    assert cache.flags.c_contiguous and cache.dtype == np.uint16
    T, Hq, D = q.shape
    qo_indptr = np.ascontiguousarray(qo_indptr, np.int32)
    kv_indptr = np.ascontiguousarray(kv_indptr, np.int32)
    last = np.ascontiguousarray(last_page_len, np.int32)
    B = qo_indptr.size - 1
    if layout == "NHD":
        P, Hkv = cache.shape[2], cache.shape[3]
        ss, hs = Hkv * D, D
    else:
        Hkv, P = cache.shape[2], cache.shape[3]
        ss, hs = D, P * D
    ps = 2 * P * Hkv * D
    scale = 1.0 / np.sqrt(D) if sm_scale is None else float(sm_scale)
    out = np.zeros((T, Hq, D), dtype=np.uint16)
    lse = np.zeros((T, Hq), dtype=np.float64)
    mask_arr = off = None
    if custom_mask is not None:
        mask_arr = np.ascontiguousarray(custom_mask, dtype=np.uint8)
        npg = np.diff(kv_indptr)
        kvl = np.where(npg > 0, (npg - 1) * P + last, 0).astype(np.int64)
        qol = np.diff(qo_indptr).astype(np.int64)
        off = np.zeros(B, dtype=np.int64)
        off[1:] = np.cumsum(qol * kvl)[:-1]
        assert mask_arr.size >= int((qol * kvl).sum()), "custom_mask too short"
    sk = None if sinks is None else np.ascontiguousarray(sinks, dtype=np.float32)
    assert sk is None or sk.shape == (Hq,), "sinks must be [Hq]"
    base = cache.ctypes.data
    _load().oracle_attention(
        q, Hq * D, D, base, base + P * Hkv * D * 2, ps, ss, hs, qo_indptr, kv_indptr,
        np.ascontiguousarray(kv_indices, np.int32), last,
        None if mask_arr is None else mask_arr.ctypes.data,
        None if off is None else off.ctypes.data, 1 if causal else 0, window_left, B, Hq, Hkv, D, P,
        scale, out, Hq * D, D,
        lse.ctypes.data, None if sinks is None else sk.ctypes.data)
    return (out, lse) if return_lse else out


def scaled_softmax(logits: np.ndarray, temperatures, greedy_threshold: float = 1e-5) -> np.ndarray:
    """logits [B, V] (float32 values) -> float64 probabilities (one-hot rows for T < threshold)."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    B, V = x.shape
    out = np.empty((B, V), dtype=np.float64)
    _load().oracle_scaled_softmax(x, B, V, np.ascontiguousarray(temperatures, np.float32),
                                  greedy_threshold, out)
    return out


SAMPLE_MODES = {"plain": 0, "top_p": 1, "top_k": 2, "min_p": 3, "top_k_top_p": 4}


def sample(probs: np.ndarray, mode: str, uniforms, top_k=None, top_p=None, min_p=None):
    """Inverse-CDF draw (index order) over each row's kept set; returns (samples int32 [B],
    kept bool [B, V])."""
    p = np.ascontiguousarray(probs, dtype=np.float32)
    B, V = p.shape
    arr = lambda a, dt: None if a is None else np.ascontiguousarray(np.broadcast_to(a, (B,)), dt)
    tk, tp, mp = arr(top_k, np.int32), arr(top_p, np.float32), arr(min_p, np.float32)
    out = np.empty(B, dtype=np.int32)
    kept = np.empty((B, V), dtype=np.uint8)
    ptr = lambda a: None if a is None else a.ctypes.data
    _load().oracle_sample(p, B, V, V, SAMPLE_MODES[mode], ptr(tk), ptr(tp), ptr(mp),
                          np.ascontiguousarray(uniforms, np.float64), out, kept.ctypes.data)
    return out, kept.astype(bool)
