"""CPU: the C-ABI library loads, exports exactly what include/pie_hip.h declares, rejects bad
arguments before touching a GPU, and the Python wrappers validate inputs and never fall back
to a CPU path."""
from __future__ import annotations

import ctypes as C
import re
import subprocess

import numpy as np
import pytest
import torch

from pie_amd import _lib, ops


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    declared = _lib.header_symbols()
    assert len(declared) >= 14
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in pie_hip.h but not exported"
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                        text=True, check=True).stdout
    exported = set(re.findall(r"\b(pie_hip_[a-z0-9_]+)\b", nm))
    assert exported == set(declared), f"exported but undeclared: {exported - set(declared)}"


def test_ctypes_signatures_match_header_arity():
    text = re.sub(r"/\*.*?\*/|//[^\n]*", "", _lib.HEADER.read_text(), flags=re.S)
    for name, argtypes in _lib.SIGNATURES.items():
        m = re.search(rf"\b{name}\s*\(([^;]*?)\)\s*;", text, re.S)
        assert m, name
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(argtypes), f"{name}: header {len(params)} vs ctypes {len(argtypes)}"


def test_abi_version():
    assert _lib.load().pie_hip_abi_version() == _lib.ABI_VERSION


def _rc(name, *args):
    lib = _lib.load()
    return getattr(lib, name)(*args), lib.pie_hip_last_error().decode()


def test_bad_arguments_return_einval_without_a_gpu():
    rc, msg = _rc("pie_hip_rmsnorm", None, 0, None, None, 0, -1, 16, C.c_float(1e-6), None)
    assert rc == 1 and "bad shape" in msg
    rc, msg = _rc("pie_hip_rmsnorm", 8, 4, 8, 8, 16, 2, 16, C.c_float(1e-6), None)
    assert rc == 1 and "stride" in msg
    rc, msg = _rc("pie_hip_silu_and_mul", 8, 3, 8, 2, 1, 2, None)
    assert rc == 1 and "stride" in msg
    rc, msg = _rc("pie_hip_rope_inplace", 16, 0, 0, 16, 0, 0, 16, 4, 1, 1, 128, 130, 0, 16, None)
    assert rc == 1 and "rotary_dim" in msg
    rc, msg = _rc("pie_hip_paged_kv_append", 16, 0, 0, 16, 0, 0, 16, 16, 16, 16, 1, 16, 16, 4,
                  0, 0, 0, 0, 1, 8, 128, None)
    assert rc == 1 and "page" in msg
    rc, msg = _rc("pie_hip_llama31_inv_freq", None, 128, C.c_float(8), C.c_float(5e5), C.c_float(4),
                  C.c_float(1), C.c_float(8192))
    assert rc == 1


def test_empty_inputs_are_noops_without_a_gpu():
    assert _rc("pie_hip_rmsnorm", None, 0, None, None, 0, 0, 16, C.c_float(1e-6), None)[0] == 0
    assert _rc("pie_hip_silu_and_mul", None, 0, None, 0, 0, 8, None)[0] == 0
    assert _rc("pie_hip_embedding", None, 0, None, 10, 8, 8, None, 8, None)[0] == 0


def test_inv_freq_tables_match_oracle():
    import oracle
    got = (C.c_float * 64)()
    assert _lib.load().pie_hip_llama31_inv_freq(got, 128, C.c_float(8), C.c_float(5e5),
                                                C.c_float(1), C.c_float(4), C.c_float(8192)) == 0
    np.testing.assert_allclose(np.array(got), oracle.inv_freq_llama31(128), rtol=1e-7)
    assert _lib.load().pie_hip_rope_inv_freq(got, 128, C.c_float(1), C.c_float(1e6)) == 0
    np.testing.assert_allclose(np.array(got), oracle.inv_freq_std(128, 1.0, 1e6), rtol=1e-7)


def test_call_raises_with_library_message():
    with pytest.raises(ValueError, match="bad shape"):
        _lib.call("pie_hip_rmsnorm", None, 0, None, None, 0, -1, 16, C.c_float(1e-6), None)


def test_wrappers_reject_cpu_tensors_and_wrong_dtypes():
    x = torch.zeros(4, 128, dtype=torch.bfloat16)
    w = torch.ones(128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.rmsnorm(x, w)                      # no silent CPU fallback
    with pytest.raises(RuntimeError, match="GPU"):
        ops.silu_and_mul(torch.zeros(2, 16, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="GPU"):
        ops.embedding(torch.zeros(3, dtype=torch.int32), x)
    with pytest.raises(TypeError):
        ops.rmsnorm(np.zeros((2, 2)), w)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(ImportError, match="not built"):
        _lib.load()


def test_integration_installs_flashinfer_namespace():
    import importlib
    import sys
    from pie_amd import integration
    mod = integration.install()
    try:
        fi = importlib.import_module("flashinfer")
        assert fi is mod
        for n in integration.HOT_PATH:
            assert getattr(fi, n) is getattr(ops, n)
        from pie_amd import attention
        for n in integration.ATTENTION:
            assert getattr(fi, n) is getattr(attention, n)
        from pie_amd import sampling
        assert fi.sampling is sampling
        from flashinfer.sampling import top_k_top_p_sampling_from_probs  # Pie's import form
        assert top_k_top_p_sampling_from_probs is sampling.top_k_top_p_sampling_from_probs
        with pytest.raises(AttributeError):
            fi.trtllm_fp8_block_scale_moe  # not served here, and no real flashinfer
        assert integration.install() is mod  # idempotent
    finally:
        integration.uninstall()
    assert "flashinfer" not in sys.modules and "flashinfer.sampling" not in sys.modules


def test_integration_does_not_forward_unserved_names_by_default(monkeypatch):
    import sys
    import types
    from pie_amd import integration
    real = types.ModuleType("flashinfer")
    real.mm_fp8 = lambda *a: "real"
    monkeypatch.setitem(sys.modules, "flashinfer", real)
    mod = integration.install()
    try:
        with pytest.raises(AttributeError, match="not provided by pie_amd"):
            mod.mm_fp8
        assert integration.install(forward_unserved=True).mm_fp8() == "real"
    finally:
        integration.uninstall()
    assert sys.modules["flashinfer"] is real


def test_pie_hip_ops_0_leaves_the_reference_path(monkeypatch):
    """PIE_HIP_OPS=0 (the A/B switch): install() keeps the real flashinfer (or none), the
    model modules keep torch.nn.functional and the Llama-style mlp stays the model's own."""
    import sys
    import types
    import torch.nn.functional as F
    from pie_amd import integration
    monkeypatch.setenv("PIE_HIP_OPS", "0")
    assert not integration.enabled()
    real = types.ModuleType("flashinfer")
    monkeypatch.setitem(sys.modules, "flashinfer", real)
    assert integration.install() is real and sys.modules["flashinfer"] is real
    monkeypatch.delitem(sys.modules, "flashinfer")
    assert integration.install() is None and "flashinfer" not in sys.modules  # no real package here
    model = types.ModuleType("fake_model")
    model.fun = F
    integration.install_functional(model)
    assert model.fun is F

    class FP:
        def mlp(self):
            return "own"
    integration.patch_mlp(FP)
    assert FP().mlp() == "own"
    monkeypatch.setenv("PIE_HIP_OPS", "1")
    assert integration.enabled()
    integration.install_functional(model)
    assert model.fun is integration.functional
    integration.uninstall_functional(model)


def test_prefill_plan_position_limits_without_a_gpu():
    """The prefill plan (host code) takes requests of up to 2^31 - 1 positions, and up to
    2^30 - 1 under a custom mask (the extent kernel marks exactly causal rows in bit 30)."""
    def plan(kv_len, mode):
        pages = (kv_len + 15) // 16
        qo = np.array([0, 1], dtype=np.int32)
        kv = np.array([0, pages], dtype=np.int32)
        last = np.array([kv_len - 16 * (pages - 1)], dtype=np.int32)
        buf = np.zeros(4096, dtype=np.int32)
        out = [C.c_int64(0) for _ in range(4)]
        return _rc("pie_hip_attention_prefill_plan", qo.ctypes.data, kv.ctypes.data, last.ctypes.data,
                   1, 16, 8, 2, 128, mode, buf.ctypes.data, buf.size, *[C.byref(o) for o in out])
    assert plan((1 << 30) - 1, 2)[0] == 0
    rc, msg = plan(1 << 30, 2)
    assert rc == 1 and "too long" in msg
    assert plan(1 << 30, 1)[0] == 0
    rc, msg = plan((1 << 31) - 1 + 16, 1)
    assert rc == 1
