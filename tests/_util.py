"""Comparison helpers shared by the tests (bf16 values travel as uint16 bit patterns)."""
from __future__ import annotations

import numpy as np

import oracle

# Tolerance for floating-point outputs (bf16 RMSNorm, SiLU-and-mul, RoPE) against the
# fp32-accumulated reference: |got - want| <= ATOL + RTOL * |want|.
RTOL = 1e-2
ATOL = 2e-2


def assert_bf16_close(got, want, rtol=RTOL, atol=ATOL, what=""):
    g = oracle.bf16_to_f32(np.asarray(got, dtype=np.uint16)).astype(np.float64)
    w = oracle.bf16_to_f32(np.asarray(want, dtype=np.uint16)).astype(np.float64)
    assert g.shape == w.shape, f"{what}: shape {g.shape} != {w.shape}"
    nan_g, nan_w = np.isnan(g), np.isnan(w)
    assert (nan_g == nan_w).all(), f"{what}: NaN pattern differs ({nan_g.sum()} vs {nan_w.sum()})"
    ok = nan_w | (np.abs(g - w) <= atol + rtol * np.abs(w))
    if not ok.all():
        idx = np.argwhere(~ok)[:5]
        detail = ", ".join(f"{tuple(i)}: got {g[tuple(i)]} want {w[tuple(i)]}" for i in idx)
        raise AssertionError(f"{what}: {int((~ok).sum())} of {ok.size} outside tolerance; {detail}")


def assert_bf16_close_rows(got, want, chunk=1024, what="", **kw):
    """assert_bf16_close over the leading dimension in chunks (bounded temporaries at full size)."""
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    for r0 in range(0, got.shape[0], chunk):
        assert_bf16_close(got[r0:r0 + chunk], want[r0:r0 + chunk], what=f"{what} rows {r0}+", **kw)


def assert_bits_equal(got, want, what=""):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    diff = got != want
    if diff.any():
        idx = np.argwhere(diff)[:5]
        raise AssertionError(f"{what}: {int(diff.sum())} of {diff.size} differ, first at "
                             f"{[tuple(i) for i in idx]}")


def ulp_diff(got, want) -> np.ndarray:
    """Distance in bf16 units in the last place (same-sign values)."""
    g = np.asarray(got, np.uint16).astype(np.int32)
    w = np.asarray(want, np.uint16).astype(np.int32)
    # map sign-magnitude to a monotone integer line
    g = np.where(g & 0x8000, 0x8000 - g, g)
    w = np.where(w & 0x8000, 0x8000 - w, w)
    return np.abs(g - w)
