"""GPU: pie_hip_attention_decode_noalloc (split partials in the library's static device array)
against pie_hip_attention_decode (split partials in a caller workspace), bit for bit, called
through the C ABI: two calls in a row, the second with a smaller batch, so partials the first
call left in the shared array must not leak into the second. Also the full Qwen3-8B decode
shape (256 sequences) and the oversize rejection."""
from __future__ import annotations

import ctypes as C

import pytest
import torch

from pie_amd import _lib
from pie_amd import workloads as wl

pytestmark = pytest.mark.gpu


def _args(a, dev):
    """Device tensors and the common argument prefix (q .. splits excluded) of both entry points."""
    pb = a["batch"]
    q = a["q"].to(dev)
    cache = a["cache"].to(dev)
    P = pb.page_size
    Hkv, D = a["Hkv"], a["D"]
    tabs = [t.to(dev) for t in (pb.kv_indptr, pb.kv_indices, pb.kv_last_page_len)]
    assert a["layout"] == "NHD" and tuple(cache.shape[1:]) == (2, P, Hkv, D)
    kp = cache.data_ptr()
    vp = cache[:, 1].data_ptr()
    keep = (q, cache, tabs)
    return keep, q, kp, vp, cache.stride(0), cache.stride(2), cache.stride(3), cache.shape[0], tabs


def _run(a, dev, splits, noalloc, ws=None):
    keep, q, kp, vp, ps, ss, hs, npages, (ip, ix, ll) = _args(a, dev)
    B, Hq, Hkv, D = q.shape[0], a["Hq"], a["Hkv"], a["D"]
    out = torch.full((B, Hq, D), float("nan"), dtype=torch.bfloat16, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    common = (q.data_ptr(), q.stride(0), q.stride(1), kp, vp, ps, ss, hs, npages, ip.data_ptr(),
              ix.data_ptr(), ll.data_ptr(), B, Hq, Hkv, D, a["batch"].page_size,
              C.c_float(D ** -0.5), -1, None, splits)
    if noalloc:
        _lib.call("pie_hip_attention_decode_noalloc", *common, out.data_ptr(), out.stride(0),
                  out.stride(1), st)
    else:
        _lib.call("pie_hip_attention_decode", *common, ws.data_ptr(), ws.numel(), out.data_ptr(),
                  out.stride(0), out.stride(1), st)
    torch.cuda.synchronize()
    del keep
    return out


def _batch(B, seed, hi=900):
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(0, hi, (B,), generator=g).to(torch.int32)
    return wl.attn_batch(ctx, torch.ones(B, dtype=torch.int32), Hq=32, Hkv=8, D=128,
                         page_size=16, seed=seed)


@pytest.mark.parametrize("splits", [1, 3])
def test_noalloc_decode_matches_workspace_decode_twice(dev, splits):
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device=dev)
    for B, seed in ((40, 5), (7, 9)):  # second call smaller than the first
        print(f"noalloc decode B={B} splits={splits} seed={seed}", flush=True)
        a = _batch(B, seed)
        want = _run(a, dev, splits, False, ws)
        got = _run(a, dev, splits, True)
        assert not torch.isnan(want.float()).any()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"B={B}"


def test_noalloc_decode_full_decode_shape(dev):
    a = wl.attn_decode_cfg()
    print("noalloc decode 256 sequences, 2 splits", flush=True)
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device=dev)
    want = _run(a, dev, 2, False, ws)
    got = _run(a, dev, 2, True)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_noalloc_decode_rejects_oversize(dev):
    # 256 x 64 splits x 32 heads x 129 x 4 bytes = 270 MB > the 32 MiB array; rejected before launch
    lib = _lib.load()
    rc = lib.pie_hip_attention_decode_noalloc(16, 0, 0, 16, 16, 0, 0, 0, 1, 16, 16, 16, 256, 32, 8,
                                              128, 16, C.c_float(1.0), -1, None, 64, 16, 0, 0, None)
    assert rc == 1 and "static scratch" in lib.pie_hip_last_error().decode()


def test_noalloc_decode_refuses_overlap_on_another_stream(dev):
    """The static scratch is shared by every call on a GPU: an eager call (splits > 1) while a
    call on another stream is still running is refused (PIE_HIP_EBUSY) instead of racing; the
    same stream queues as usual, and after a synchronisation the other stream runs."""
    a = wl.attn_decode_cfg()
    keep, q, kp, vp, ps, ss, hs, npages, (ip, ix, ll) = _args(a, dev)
    B, Hq, Hkv, D = q.shape[0], a["Hq"], a["Hkv"], a["D"]
    out = torch.empty((B, Hq, D), dtype=torch.bfloat16, device=dev)
    common = (q.data_ptr(), q.stride(0), q.stride(1), kp, vp, ps, ss, hs, npages, ip.data_ptr(),
              ix.data_ptr(), ll.data_ptr(), B, Hq, Hkv, D, a["batch"].page_size,
              C.c_float(D ** -0.5), -1, None, 2, out.data_ptr(), out.stride(0), out.stride(1))
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    for _ in range(4):  # ~1.6 ms queued on s1
        _lib.call("pie_hip_attention_decode_noalloc", *common, s1.cuda_stream)
    with pytest.raises(_lib.PieHipError, match="another stream"):
        _lib.call("pie_hip_attention_decode_noalloc", *common, s2.cuda_stream)
    s1.synchronize()
    _lib.call("pie_hip_attention_decode_noalloc", *common, s2.cuda_stream)
    torch.cuda.synchronize()
    del keep
