"""CPU: the unchanged kernel sources built for the host against a HIP emulator (lanes as
threads, DPP/readlane emulated) under AddressSanitizer + UBSan, on exact-size buffers, and
compared with the C oracle. Catches out-of-bounds indexing before any GPU run."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

EMU = Path(__file__).resolve().parent / "hostemu"


@pytest.mark.skipif(not Path("/opt/rocm/llvm/bin/clang++").exists(), reason="needs ROCm clang++")
def test_kernels_under_host_emulation_and_asan():
    subprocess.run(["make", "-s", "-C", str(EMU)], check=True, timeout=600)
    res = subprocess.run([str(EMU / "_build" / "emu_main"), "all"], capture_output=True, text=True,
                         timeout=900)
    tail = "\n".join((res.stdout + res.stderr).splitlines()[-40:])
    assert res.returncode == 0, tail
    assert "all ok" in res.stdout, tail
