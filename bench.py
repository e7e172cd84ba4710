"""Benchmark of the per-layer hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only main|ops|copy|chain] [--no-cpu]

One step = one pass of the fused residual-add + RMSNorm [8192, 4096] followed by SiLU-and-mul
[8192, 2x14336] (configuration 2, Llama-3-8B prefill), inputs resident in HBM. Prints ONE JSON
line: value = algorithmic HBM GB/s of the step; roofline = the dominant kernel (SiLU-and-mul)
timed with HIP events on the stream it runs on; cpu_baseline = torch-CPU running the
reference's own expressions (`residual + x`, F.rms_norm, F.silu(gate) * up) on a bounded
sample of the same workload; "ops" = every configuration's per-op µs / GB/s (steady state over
buffer sets larger than the 256 MB last-level cache, and one launch after a flush) and the
decode-chain µs (HIP-graph replay); "cpu_ops" = torch-CPU GB/s of each configuration's
expressions on bounded samples beside them.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0


def _events(fn, iters, flush=None):
    """Per-launch durations (ms) from HIP events on the current stream."""
    import torch
    out = []
    for _ in range(iters):
        if flush is not None:
            flush()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        out.append((a, b))
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in out]


def cpu_baseline(budget_s: float = 12.0) -> dict:
    """torch-CPU running the reference's expressions (llama3.py:586 `residual + down`,
    :555 fun.rms_norm, :569-572 fun.silu(gate) * up) on 256-row slices of configuration 2."""
    import torch
    import torch.nn.functional as F
    from pie_amd import workloads as wl
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    rows = 256
    c = wl.cfg2(T=rows)
    I = c["gate_up"].shape[1] // 2
    nbytes = sum(wl.cfg2_bytes(T=rows))

    def step():
        s = c["r"] + c["x"]
        F.rms_norm(s, [s.shape[1]], c["w"], c["eps"])
        g, u = torch.split(c["gate_up"], [I, I], -1)
        F.silu(g) * u

    for _ in range(2):
        step()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        step()
        n += 1
    dt = time.perf_counter() - t0
    return {"value": round(n * nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "reference",
            "sample": f"{n} x 256-row slices of config 2 (add+rms_norm [256,4096], silu*mul "
                      f"[256,2x14336]) in torch-CPU bf16, {dt:.1f} s"}


def cpu_ops(budget_each: float = 2.0) -> list:
    """torch-CPU timings beside the per-op GPU figures, on bounded samples with all host threads:
    RMSNorm (configuration 1, full size), add + RMSNorm and SiLU-and-mul (256-row slices of
    configuration 2) and the embedding (configuration 4, full size) run the reference's own
    torch expressions (kind "reference": llama3.py:555, :586, :569-572, :471). flashinfer has no
    CPU path, so Llama-3.1 RoPE and the paged append (configuration 3, 2048-token slices) run a
    torch restatement of flashinfer's semantics (kind "port"; the frequencies from oracle/).
    The GPU bench runs these on the GPU box's host cores after the timed GPU work."""
    import torch
    import torch.nn.functional as F
    import oracle
    from pie_amd import workloads as wl
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)

    def rate(name, kind, nbytes, fn, sample):
        fn()
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget_each:
            fn()
            n += 1
        dt = time.perf_counter() - t0
        return {"op": name, "kind": kind, "gbs": round(n * nbytes / dt / 1e9, 3),
                "us": round(dt / n * 1e6, 1), "cores": threads, "sample": sample}

    out = []
    c1 = wl.cfg1()
    out.append(rate("cfg1 rmsnorm [2048,2048]", "reference", 2 * 2048 * 2048 * 2 + 2048 * 2,
                    lambda: F.rms_norm(c1["x"], [2048], c1["w"], c1["eps"]), "full size"))
    c2 = wl.cfg2(T=256)
    b_add, b_silu = wl.cfg2_bytes(T=256)
    I = c2["gate_up"].shape[1] // 2
    out.append(rate("cfg2a add+rmsnorm", "reference", b_add,
                    lambda: F.rms_norm(c2["r"] + c2["x"], [4096], c2["w"], c2["eps"]), "256 rows"))
    g, u = torch.split(c2["gate_up"], [I, I], -1)
    out.append(rate("cfg2b silu_and_mul", "reference", b_silu, lambda: F.silu(g) * u, "256 rows"))
    c3 = wl.cfg3(B=4)  # four of configuration 3's requests (same generator), a 2048-token slice
    pb = c3["batch"]
    T = min(2048, int(pb.lens.sum()))
    q, k, v = wl.split_qkv(c3["qkv"][:T].clone(), 32, 8, 128)
    f = torch.tensor(oracle.inv_freq_llama31(128, **{kk: float(vv) for kk, vv in c3["rope"].items()}),
                     dtype=torch.float32)
    pos = pb.positions[:T].to(torch.float32)

    def rope():  # half-split pairs in fp32, written back in place (flashinfer_metal/ops.py:306-346)
        ang = pos[:, None] * f[None, :]
        cs, sn = ang.cos()[:, None, :], ang.sin()[:, None, :]
        for t in (q, k):
            x, y = t[..., :64].float(), t[..., 64:].float()
            t[..., :64] = (x * cs - y * sn).to(t.dtype)
            t[..., 64:] = (x * sn + y * cs).to(t.dtype)
    bts = wl.cfg3_bytes(T)
    out.append(rate("cfg3 llama31 rope", "port", bts["rope"], rope, f"{T} tokens"))
    cache = wl.sentinel_cache(c3["cache_shape"])
    bidx, bpos = pb.batch_indices[:T].long(), pb.positions[:T].long()
    pages = pb.kv_indices.long()[pb.kv_indptr.long()[bidx] + bpos // 16]
    slots = bpos % 16

    def append():  # cache[page, 0 / 1, slot] = k / v (flashinfer_metal/ops.py:349-389)
        cache[pages, 0, slots] = k
        cache[pages, 1, slots] = v
    out.append(rate("cfg3 paged append", "port", bts["append"], append, f"{T} tokens"))
    # configuration 5's per-head q/k norm (qwen3.py:651-662) and the whole decode chain in its
    # order (embedding, residual add + norm, q/k norm, RoPE, append, SiLU-and-mul); the table
    # has 4096 rows here (the gather touches 256 rows either way)
    c5 = wl.cfg5(V=4096)
    q5, k5, v5 = wl.split_qkv(c5["qkv"], 32, 8, 128)
    b5 = wl.cfg5_bytes()
    out.append(rate("cfg5 qk rmsnorm [256,32|8,128]", "reference", b5["qk_rmsnorm"],
                    lambda: (F.rms_norm(q5, [128], c5["q_norm"], c5["eps"]),
                             F.rms_norm(k5, [128], c5["k_norm"], c5["eps"])), "full size"))
    f5 = torch.tensor(oracle.inv_freq_std(128, 1.0, c5["theta"]), dtype=torch.float32)
    pb5 = c5["batch"]
    pos5 = pb5.positions.to(torch.float32)
    cache5 = wl.sentinel_cache(c5["cache_shape"])
    pages5 = pb5.kv_indices.long()[pb5.kv_indptr.long()[pb5.batch_indices.long()]
                                   + pb5.positions.long() // 16]
    slots5 = pb5.positions.long() % 16
    I5 = c5["gate_up"].shape[1] // 2
    ids5 = c5["ids"].long()

    def chain():
        hid = F.embedding(ids5, c5["W"])
        s = c5["residual"] + hid
        F.rms_norm(s, [4096], c5["w_norm"], c5["eps"])
        qn = F.rms_norm(q5, [128], c5["q_norm"], c5["eps"])
        kn = F.rms_norm(k5, [128], c5["k_norm"], c5["eps"])
        ang = pos5[:, None] * f5[None, :]
        cs, sn = ang.cos()[:, None, :], ang.sin()[:, None, :]
        for t in (qn, kn):
            x, y = t[..., :64].float(), t[..., 64:].float()
            t[..., :64] = (x * cs - y * sn).to(t.dtype)
            t[..., 64:] = (x * sn + y * cs).to(t.dtype)
        cache5[pages5, 0, slots5] = kn
        cache5[pages5, 1, slots5] = v5
        g5, u5 = torch.split(c5["gate_up"], [I5, I5], -1)
        F.silu(g5) * u5
    out.append(rate("cfg5 decode chain (256 x 1)", "port", sum(b5.values()), chain,
                    "full chain; reference torch expressions, RoPE and append as torch "
                    "restatements of flashinfer"))
    c4 = wl.cfg4()
    ids = c4["ids"].long()  # all 16384 ids: the 268 MB the op moves do not stay in host caches
    out.append(rate("cfg4 embedding", "reference", wl.cfg4_bytes(),
                    lambda: F.embedding(ids, c4["W"]), "full size"))
    return out


def _rotating(calls, iters=60, reps=3):
    """µs per launch over back-to-back launches that rotate through independent buffer sets
    (together larger than the 256 MB last-level cache), so each launch pays for its own HBM
    reads and for draining its writes. The launches are recorded into one HIP graph and
    replayed, so host-side launch cost (Python, ctypes) does not limit small ops; median over
    reps."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for c in calls:
            c()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(iters):
            calls[i % len(calls)]()
    g.replay()
    torch.cuda.synchronize()
    out = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        out.append(a.elapsed_time(b) * 1e3 / iters)
    del g
    return statistics.median(out)


def _copies(footprint_bytes):
    return max(2, -(-(768 << 20) // footprint_bytes))


def _entry(name, nbytes, steady_us, cold_ms):
    cold = statistics.median(cold_ms) * 1e3
    return {"op": name, "bytes": nbytes,
            "us": round(steady_us, 2), "gbs": round(nbytes / steady_us / 1e3, 1),
            "frac": round(nbytes / steady_us / 1e3 / HBM_PEAK_GBS, 3),
            "us_cold_single": round(cold, 2), "gbs_cold_single": round(nbytes / cold / 1e3, 1)}


def measure_ops(dev, cold_iters=20, only=None):
    """Every configuration's ops. "us"/"gbs"/"frac": back-to-back launches over rotating buffer
    sets (steady state, writes drained); "*_cold_single": one launch after a cache flush.
    Decode chain: µs per HIP-graph replay."""
    import torch

    scratch = torch.ones(1 << 28, dtype=torch.float32, device=dev)  # 1 GiB
    sink = torch.empty((), dtype=torch.float32, device=dev)

    def flush():
        # Reading 1 GiB evicts the 256 MB last-level cache and L2 with clean lines.
        torch.sum(scratch, dim=0, out=sink)

    def run(name, nbytes, make):
        calls = [make() for _ in range(_copies(nbytes))]
        e = _entry(name, nbytes, _rotating(calls), _events(calls[0], cold_iters, flush))
        del calls
        torch.cuda.empty_cache()
        return e

    res = []
    want = lambda tag: only is None or only == tag
    if want("cfg1"):
        res.extend(_ops_cfg1(dev, run))
    if want("cfg2"):
        res.extend(_ops_cfg2(dev, run))
    if want("cfg3"):
        res.extend(_ops_cfg3(dev, run))
    if want("cfg4"):
        res.extend(_ops_cfg4(dev, run))
    if want("variants"):
        res.extend(_ops_variants(dev, run))
    if want("attn"):
        res.extend(_ops_attention(dev, run))
    if want("sample"):
        res.extend(_ops_sampling(dev, run))
    if want("cfg5"):
        res.extend(measure_chain(dev, flush, cold_iters))
    if want("ceiling"):
        res.extend(_ops_ceiling(dev, run))
    del scratch
    return res


def _ops_ceiling(dev, run):
    """Measured ceilings for access patterns (pie_amd/probe/probe.hip, no arithmetic and no
    index logic): configuration 1's bytes as a plain copy (8 MiB read, 8 MiB written), the
    sampling softmax's bytes as a plain copy (one read and one write of [256, 128256] bf16), and
    configuration 3's paged append as a scatter of the same 2 KiB k / v rows from the same qkv
    rows to the same cache slots, the slot offsets computed beforehand (plus their 16 B per row)."""
    import ctypes as C

    import torch
    from pie_amd import build as B
    from pie_amd import workloads as wl
    lib = C.CDLL(str(B.PROBE_LIB))
    lib.pie_probe_copy.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_int, C.c_void_p]
    lib.pie_probe_scatter.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64,
                                      C.c_int64, C.c_void_p]
    st = lambda: torch.cuda.current_stream().cuda_stream
    n1 = 2048 * 2048 * 2

    def make_copy(nt):
        a = torch.empty(n1, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        return lambda: lib.pie_probe_copy(a.data_ptr(), b.data_ptr(), n1, nt, st())
    n_sm = 256 * 128256 * 2

    def make_copy_sm():
        a = torch.empty(n_sm, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        return lambda: lib.pie_probe_copy(a.data_ptr(), b.data_ptr(), n_sm, 1, st())
    lib.pie_probe_read.argtypes = [C.c_void_p, C.c_int64, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    sink = torch.empty(1 << 16, dtype=torch.int32, device=dev)

    def make_read(nbytes, threads, vpt):
        a = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        return lambda: lib.pie_probe_read(a.data_ptr(), nbytes, threads, vpt, sink.data_ptr(), st())
    # read-only ceilings (all of a work group's loads issued before any is used): the softmax's
    # read phase on its own rows (one 1024-thread work group per 250.5 KiB row, 16 vectors per
    # thread); the same shape over rows 256 KiB apart (a power-of-two stride, which measured
    # slower: every work group starts on the same memory channels); and the best read-only shape
    # measured (256-thread groups, 16 vectors each), over the softmax's bytes and over the
    # sampler's fp32 rows; and the sampler's own row layout (one work group per fp32 row)
    # the dense bf16 MFMA rate a kernel can reach (32x32x16, 2 work groups of 4 waves per CU,
    # 4 independent accumulator chains per wave), alone and with as much independent fp32 VALU
    # work interleaved: the matrix pipe's practical ceiling, and whether vector work overlaps it
    lib.pie_probe_mfma.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]
    mf_out = torch.empty(1 << 20, dtype=torch.float32, device=dev)
    mf_blocks, mf_iters = 2 * 256, 2000
    mf_flops = mf_blocks * 4 * mf_iters * 16 * 32768

    def make_mfma(valu):
        return lambda: lib.pie_probe_mfma(mf_out.data_ptr(), mf_blocks, mf_iters, valu, st())
    mf = []
    for valu, what in ((0, "alone"), (1, "with 128 independent fp32 fma per 16 MFMAs")):
        e = run(f"ceiling mfma 32x32x16 bf16, {what}", 1 << 30, lambda v=valu: make_mfma(v))
        for key in ("bytes", "gbs", "frac", "gbs_cold_single"):
            e[key] = None  # no memory traffic to speak of
        e["flops"] = mf_flops
        e["tflops"] = round(mf_flops / e["us"] / 1e6, 1)
        e["mfma_frac"] = round(mf_flops / e["us"] / 1e6 / 2500.0, 3)
        mf.append(e)
    n_rd = 256 * 1024 * 256  # 256 rows of 256 KiB (softmax rows are 250.5 KiB)
    n_rd2 = 2 * n_rd
    lib.pie_probe_read_rows.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int64, C.c_void_p, C.c_void_p]
    sm_vec = 128256 * 2 // 16  # a [256, 128256] bf16 row in 16-byte vectors (also its stride)

    def make_read_rows(vec):
        a = torch.empty(256 * vec * 16, dtype=torch.uint8, device=dev)
        return lambda: lib.pie_probe_read_rows(a.data_ptr(), 256, vec, vec, sink.data_ptr(), st())
    res = mf + [run("ceiling read [256, 128256] bf16 rows, 1 work group x 1024 threads x 16 vectors per row "
                    "(softmax read phase)", 256 * sm_vec * 16, lambda: make_read_rows(sm_vec)),
           run("ceiling read 64 MiB, 1 work group x 1024 threads x 16 vectors per 256 KiB (row stride a "
               "power of two)", n_rd, lambda: make_read(n_rd, 1024, 16)),
           run("ceiling read 64 MiB, 256 threads x 16 vectors per work group", n_rd, lambda: make_read(n_rd, 256, 16)),
           run("ceiling read 128 MiB (sampler rows' bytes), 256 threads x 16 vectors per work group", n_rd2,
               lambda: make_read(n_rd2, 256, 16)),
           run("ceiling read [256, 128256] fp32 rows, 1 work group x 1024 threads per row, two rounds of "
               "16 vectors (sampler rows)", 256 * 2 * sm_vec * 16, lambda: make_read_rows(2 * sm_vec))]
    res += [run("ceiling copy 8 MiB -> 8 MiB (cfg1 bytes), cached", 2 * n1, lambda: make_copy(0)),
           run("ceiling copy 8 MiB -> 8 MiB (cfg1 bytes), non-temporal", 2 * n1, lambda: make_copy(1)),
           run("ceiling copy 64 MB -> 64 MB (softmax bytes, [256,128256] bf16), non-temporal",
               2 * n_sm, make_copy_sm)]
    c = wl.cfg3()
    pb, T = c["batch"], c["qkv"].shape[0]
    Hq, Hkv, D, P = 32, 8, 128, pb.page_size
    row_b, kv_b = (Hq + 2 * Hkv) * D * 2, Hkv * D * 2
    page = pb.kv_indices.long()[pb.kv_indptr.long()[pb.batch_indices.long()] + pb.positions.long() // P]
    slot = pb.positions.long() % P
    t = torch.arange(T, dtype=torch.int64)
    dst_k = page * (2 * P * kv_b) + slot * kv_b
    src = torch.stack([t * row_b + Hq * D * 2, t * row_b + (Hq + Hkv) * D * 2], 1).reshape(-1).to(dev)
    dst = torch.stack([dst_k, dst_k + P * kv_b], 1).reshape(-1).to(dev)
    qkv0 = c["qkv"].to(dev)

    def make_scatter():
        qkv = qkv0.clone()
        cache = wl.sentinel_cache(c["cache_shape"]).to(dev)
        return lambda: lib.pie_probe_scatter(qkv.data_ptr(), src.data_ptr(), cache.data_ptr(),
                                             dst.data_ptr(), 2 * T, kv_b, st())
    res.append(run(f"ceiling scatter of the cfg3 append pattern T={T}", 2 * T * 2 * kv_b + 2 * T * 16,
                   make_scatter))
    # the fixed cost of one kernel inside a captured graph (what every launch of a decode step
    # pays besides its own work): 12 launches of a 16-byte copy in one graph, replayed back to back
    tiny = [torch.empty(16, dtype=torch.uint8, device=dev) for _ in range(24)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())

    def tiny_all():
        for i in range(12):
            lib.pie_probe_copy(tiny[2 * i].data_ptr(), tiny[2 * i + 1].data_ptr(), 16, 1, st())
    with torch.cuda.stream(side):
        tiny_all()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        tiny_all()
    per = _back_to_back(g.replay, 50) / 12
    res.append({"op": "ceiling graph launch: one 16-byte copy kernel, 12 per graph", "bytes": 32, "us": round(per, 2),
                "gbs": None, "frac": None})
    del g
    return res


def _ops_cfg1(dev, run):
    import torch
    from pie_amd import ops
    from pie_amd import workloads as wl
    c = wl.cfg1()
    x0, w = c["x"].to(dev), c["w"].to(dev)

    def make_cfg1():
        x, y = x0.clone(), torch.empty_like(x0)
        return lambda: ops.rmsnorm(x, w, c["eps"], out=y)
    return [run("cfg1 rmsnorm [2048,2048]", 2 * x0.numel() * 2 + w.numel() * 2, make_cfg1)]


def _ops_cfg2(dev, run):
    import torch
    from pie_amd import ops
    from pie_amd import workloads as wl
    c = wl.cfg2()
    x0, r0, w, gu0 = (c[k].to(dev) for k in ("x", "r", "w", "gate_up"))
    b_add, b_silu = wl.cfg2_bytes()

    def make_add():
        x, r = x0.clone(), r0.clone()
        y, s = torch.empty_like(x), torch.empty_like(x)
        return lambda: ops.add_rms_norm(x, r, w, c["eps"], out=y, residual_out=s)

    def make_silu():
        gu = gu0.clone()
        act = torch.empty((gu.shape[0], gu.shape[1] // 2), dtype=gu.dtype, device=dev)
        return lambda: ops.silu_and_mul(gu, out=act)
    return [run("cfg2a add+rmsnorm [8192,4096]", b_add, make_add),
            run("cfg2b silu_and_mul [8192,2x14336]", b_silu, make_silu)]


def _ops_cfg3(dev, run):
    from pie_amd import ops
    from pie_amd import workloads as wl
    c = wl.cfg3()
    pb, T = c["batch"], c["qkv"].shape[0]
    qkv0 = c["qkv"].to(dev)
    d = {n: getattr(pb, n).to(dev) for n in ("batch_indices", "positions", "kv_indices",
                                             "kv_indptr", "kv_last_page_len")}
    nb = wl.cfg3_bytes(T)

    def make_rope(kind):
        qkv = qkv0.clone()
        q, k, v = wl.split_qkv(qkv, 32, 8, 128)
        cache = wl.sentinel_cache(c["cache_shape"]).to(dev) if kind != "rope" else None
        if kind == "rope":
            return lambda: ops.apply_llama31_rope_pos_ids_inplace(q, k, d["positions"], **c["rope"])
        if kind == "append":
            return lambda: ops.append_paged_kv_cache(k, v, d["batch_indices"], d["positions"], cache,
                                                     d["kv_indices"], d["kv_indptr"],
                                                     d["kv_last_page_len"])
        return lambda: ops.apply_llama31_rope_pos_ids_and_append_paged_kv_cache(
            q, k, v, d["positions"], d["batch_indices"], d["positions"], cache, d["kv_indices"],
            d["kv_indptr"], d["kv_last_page_len"], **c["rope"])
    return [run(f"cfg3 llama31 rope T={T}", nb["rope"], lambda: make_rope("rope")),
            run(f"cfg3 paged append T={T}", nb["append"], lambda: make_rope("append")),
            run(f"cfg3 fused rope+append T={T}", nb["fused"], lambda: make_rope("fused"))]


def _ops_variants(dev, run):
    """The model-family variants at the same Llama-3-8B prefill shapes as configurations 2-4, so
    their bandwidth compares directly: Gemma add+RMSNorm and RMSNorm [8192, 4096], GELU-tanh-and-mul
    [8192, 2x14336], the scaled embedding, and RoPE from a [2048, 128] fp32 cos/sin table on
    configuration 3's q/k (the 1 MB table stays in cache; its reads are not counted)."""
    import torch
    from pie_amd import ops
    from pie_amd import workloads as wl
    c2 = wl.cfg2()
    x0, r0, gu0 = (c2[k].to(dev) for k in ("x", "r", "gate_up"))
    w = wl.normal((x0.shape[1],), 60, 0.0, 0.5).to(dev)
    b_add, b_act = wl.cfg2_bytes()
    b_norm = 2 * x0.numel() * 2 + w.numel() * 2

    def make_gemma_add():
        x, r = x0.clone(), r0.clone()
        y, s = torch.empty_like(x), torch.empty_like(x)
        return lambda: ops.gemma_add_rms_norm(x, r, w, 1e-6, out=y, residual_out=s)

    def make_gemma():
        x, y = x0.clone(), torch.empty_like(x0)
        return lambda: ops.gemma_rms_norm(x, w, 1e-6, out=y)

    def make_plain():
        x, y = x0.clone(), torch.empty_like(x0)
        return lambda: ops.rmsnorm(x, w, 1e-6, out=y)

    def make_gelu():
        gu = gu0.clone()
        act = torch.empty((gu.shape[0], gu.shape[1] // 2), dtype=gu.dtype, device=dev)
        return lambda: ops.gelu_tanh_and_mul(gu, out=act)
    res = [run("variant gemma add+rmsnorm [8192,4096]", b_add, make_gemma_add),
           run("variant gemma rmsnorm [8192,4096]", b_norm, make_gemma),
           run("rmsnorm [8192,4096] (the plain norm at the Gemma shape)", b_norm, make_plain),
           run("variant gelu_tanh_and_mul [8192,2x14336]", b_act, make_gelu)]
    del x0, r0, gu0
    c4 = wl.cfg4()
    W0, ids = c4["W"].to(dev), c4["ids"].to(dev)

    def make_embed():
        W = W0.clone()
        out = torch.empty((ids.numel(), W.shape[1]), dtype=W.dtype, device=dev)
        return lambda: ops.embedding(ids, W, out=out, scale=64.0)
    res.append(run("variant embedding x sqrt(H) [128256,4096] x16384", wl.cfg4_bytes(), make_embed))
    del W0
    c3 = wl.cfg3()
    T = c3["qkv"].shape[0]
    qkv0, pos = c3["qkv"].to(dev), c3["batch"].positions.to(dev)
    inv = 1e4 ** (-torch.arange(0, 128, 2, dtype=torch.float64) / 128)
    ang = torch.arange(2048, dtype=torch.float64)[:, None] * inv[None, :]
    cs = torch.cat([ang.cos(), ang.sin()], -1).float().to(dev)

    def make_rope_cs():
        qkv = qkv0.clone()
        q, k, _ = wl.split_qkv(qkv, 32, 8, 128)
        return lambda: ops.apply_rope_with_cos_sin_cache_inplace(pos, q, k, 128, cs)
    res.append(run(f"variant rope cos/sin table T={T}", wl.cfg3_bytes(T)["rope"], make_rope_cs))
    return res


def _ops_cfg4(dev, run):
    import torch
    from pie_amd import ops
    from pie_amd import workloads as wl
    c = wl.cfg4()
    W0, ids = c["W"].to(dev), c["ids"].to(dev)

    def make_embed():
        W = W0.clone()
        out = torch.empty((ids.numel(), W.shape[1]), dtype=W.dtype, device=dev)
        return lambda: ops.embedding(ids, W, out=out)
    return [run("cfg4 embedding [128256,4096] x16384", wl.cfg4_bytes(), make_embed)]


def _ops_attention(dev, run):
    """Paged decode attention at the Qwen3-8B decode-chain shape (256 sequences, contexts
    U[128, 4096], Hq 32 / Hkv 8 / D 128, page 16; the ~2.2 GB cache exceeds the last-level cache,
    so the launches share it and rotate only q / out). Bytes: q + out + every cached k/v row +
    page table (workloads.attn_bytes)."""
    import torch
    from pie_amd import attention
    from pie_amd import workloads as wl
    a = wl.attn_decode_cfg()
    pb = a["batch"]
    cache, q0 = a["cache"].to(dev), a["q"].to(dev)
    ws = torch.zeros(128 << 20, dtype=torch.uint8, device=dev)
    w = attention.BatchDecodeWithPagedKVCacheWrapper(ws, "NHD")
    w.plan(pb.kv_indptr.to(dev), pb.kv_indices.to(dev), pb.kv_last_page_len.to(dev), 32, 8, 128, 16)
    nbytes = wl.attn_bytes(pb, 32, 8, 128)

    def make():
        q, out = q0.clone(), torch.empty_like(q0)
        return lambda: w.run(q, cache, out=out)
    res = [run(f"attn decode B=256 ctx U[128,4096] (splits {w._plan['splits']})", nbytes, make)]
    del cache, w
    # causal prefill over configuration 3's ragged batch: MFMA-bound, reported as TFLOP/s of
    # the useful (causal-window) QK^T and PV flops
    a = wl.attn_prefill_cfg()
    pb = a["batch"]
    cache, q0 = a["cache"].to(dev), a["q"].to(dev)
    wp = attention.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    wp.plan(pb.qo_indptr.to(dev), pb.kv_indptr.to(dev), pb.kv_indices.to(dev),
            pb.kv_last_page_len.to(dev), 32, 8, 128, 16, causal=True)
    flops = wl.attn_flops(pb, 32, 128)

    def make_p():
        q, out = q0.clone(), torch.empty_like(q0)
        return lambda: wp.run(q, cache, out=out)
    e = run(f"attn prefill causal cfg3 T={q0.shape[0]}", wl.attn_bytes(pb, 32, 8, 128), make_p)
    e["flops"] = flops
    e["tflops"] = round(flops / e["us"] / 1e6, 1)
    e["mfma_frac"] = round(flops / e["us"] / 1e6 / 2500.0, 3)
    res.append(e)
    # the same causal window given as the custom mask Pie always passes (batching.py:226-228)
    blocks = []
    for b in range(pb.lens.numel()):
        qo, kv = int(pb.lens[b]), int(pb.seq_lens[b])
        blocks.append((torch.arange(kv, device=dev)[None, :] <=
                       (kv - qo + torch.arange(qo, device=dev))[:, None]).flatten())
    mask = torch.cat(blocks)
    del blocks
    wm = attention.BatchPrefillWithPagedKVCacheWrapper(ws, "NHD")
    wm.plan(pb.qo_indptr.to(dev), pb.kv_indptr.to(dev), pb.kv_indices.to(dev),
            pb.kv_last_page_len.to(dev), 32, 8, 128, 16, custom_mask=mask)

    def make_m():
        q, out = q0.clone(), torch.empty_like(q0)
        return lambda: wm.run(q, cache, out=out)
    e = run(f"attn prefill custom causal mask cfg3 T={q0.shape[0]}", wl.attn_bytes(pb, 32, 8, 128), make_m)
    e["flops"] = flops
    e["tflops"] = round(flops / e["us"] / 1e6, 1)
    e["mfma_frac"] = round(flops / e["us"] / 1e6 / 2500.0, 3)
    res.append(e)
    del mask
    del cache, ws
    return res


def _ops_sampling(dev, run):
    """The sampling path at Llama-3 vocabulary (128256) for 256 decode rows: safe_scaled_softmax
    on bf16 logits, and top-k + top-p sampling on fp32 probabilities. Bytes: one read (and for the
    softmax one write) of the rows; the sampler's later passes re-read rows from L2/MALL."""
    import torch
    from pie_amd import sampling
    B, V = 256, 128256
    g = torch.Generator().manual_seed(0)
    logits0 = (torch.randn(B, V, generator=g) * 3).to(torch.bfloat16).to(dev)
    temps = torch.full((B,), 0.8, device=dev)
    probs0 = torch.softmax(logits0.float(), -1)
    k = torch.full((B,), 50, dtype=torch.int32, device=dev)
    p = torch.full((B,), 0.9, device=dev)

    def make_softmax():
        x, out = logits0.clone(), torch.empty_like(logits0)
        return lambda: sampling.safe_scaled_softmax(x, temps, out=out)

    def make_sample():
        pr = probs0.clone()
        return lambda: sampling.top_k_top_p_sampling_from_probs(pr, k, p, seed=1, offset=0)
    # rows whose large probabilities sit in the vocabulary's last quarter: the one-read top_k
    # path's floor comes from a sample that spans every wave's segment, so these rows stay on
    # one read (the waves holding the large entries raise their own floors)
    skew = torch.randn(B, V, generator=g) * 3
    skew[:, : 3 * V // 4] -= 12.0
    probs_skew = torch.softmax(skew.to(dev), -1)

    def make_sample_skew():
        pr = probs_skew.clone()
        return lambda: sampling.top_k_top_p_sampling_from_probs(pr, k, p, seed=1, offset=0)
    mp = torch.full((B,), 0.1, device=dev)

    def make_mode(name):
        pr = probs0.clone()
        f = {"plain": lambda: sampling.sampling_from_probs(pr, seed=1, offset=0),
             "top_p": lambda: sampling.top_p_sampling_from_probs(pr, p, seed=1, offset=0),
             "top_k": lambda: sampling.top_k_sampling_from_probs(pr, k, seed=1, offset=0),
             "min_p": lambda: sampling.min_p_sampling_from_probs(pr, mp, seed=1, offset=0)}[name]
        return f
    return [run(f"safe_scaled_softmax bf16 [{B},{V}]", 2 * B * V * 2, make_softmax),
            run(f"top_k_top_p sampling fp32 [{B},{V}] (k 50, p 0.9)", B * V * 4, make_sample),
            run(f"sampling (plain) fp32 [{B},{V}]", B * V * 4, lambda: make_mode("plain")),
            run(f"top_p sampling fp32 [{B},{V}] (p 0.9: ~5.6k tokens kept per row)", B * V * 4,
                lambda: make_mode("top_p")),
            run(f"top_k sampling fp32 [{B},{V}] (k 50)", B * V * 4, lambda: make_mode("top_k")),
            run(f"min_p sampling fp32 [{B},{V}] (min_p 0.1)", B * V * 4, lambda: make_mode("min_p")),
            run(f"top_k_top_p sampling fp32 [{B},{V}], mass in the last quarter",
                B * V * 4, make_sample_skew)]


def _back_to_back(fn, n, reps=5):
    """µs per call over n back-to-back calls between two events (median of reps)."""
    import torch
    out = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        out.append(a.elapsed_time(b) * 1e3 / n)
    return statistics.median(out)


def measure_chain(dev, flush=None, cold_iters=20):
    """Configuration 5 (Qwen3-8B decode, 256 sequences): µs per chain.
    in_graph: one HIP graph holding the chain of CHAINS_PER_GRAPH instances in turn, each over its
    own activations (the table and the cache pool are shared), replayed back to back, divided by
    the chain count: the chain's GPU time inside a captured decode step, as Pie captures all
    layers of a decode pass in one graph (llama3.py:315-414); the instances' activations
    (~38 MB each) together exceed the 256 MB last-level cache, so each chain reads HBM.
    steady: back-to-back replays of a one-chain graph (bound by the host's graph-launch rate when
    the chain is short); single: one replay between two events (includes the launch latency);
    eager_steady: back-to-back run() calls (ops recorded and validated in Python each time);
    saved_steady (grouped): back-to-back relaunches of recorded groups, one library call each,
    over CHAINS_PER_GRAPH chains in turn like in_graph."""
    from pie_amd import workloads as wl
    from pie_amd.chain import DecodeChain
    c = wl.cfg5()
    chain_bytes = sum(wl.cfg5_bytes().values())
    res = []
    for mode, launches in (("grouped", 1), ("fused", 4), ("unfused", 6)):
        fused = mode != "unfused"
        grouped = mode == "grouped"
        ch = DecodeChain(c, dev, fused=fused, grouped=grouped)
        if grouped:
            # recorded groups relaunched with one library call per chain, no graph: CHAINS_PER_GRAPH
            # chains over their own activations in turn (as in_graph, so each reads HBM)
            svs = [DecodeChain(c, dev, saved=True, share=ch) for _ in range(CHAINS_PER_GRAPH)]
            for sv in svs:
                sv.run()

            def _saved_round():
                for sv in svs:
                    sv.run()
            saved_steady = _back_to_back(_saved_round, 10) / len(svs)
            del svs
        g = ch.capture()
        for _ in range(20):
            g.replay()
        steady = _back_to_back(g.replay, 100)
        single = statistics.median(_events(g.replay, 200)) * 1e3
        chains = [ch] + [DecodeChain(c, dev, fused=fused, grouped=grouped, share=ch)
                         for _ in range(CHAINS_PER_GRAPH - 1)]
        big = _capture_all(chains)
        for _ in range(3):
            big.replay()
        in_graph = _back_to_back(big.replay, 20) / len(chains)
        e = {"op": f"cfg5 decode chain ({mode}, {launches} launch{'es' if launches > 1 else ''})",
             "bytes": chain_bytes, "us_in_graph": round(in_graph, 2),
             "gbs_in_graph": round(chain_bytes / in_graph / 1e3, 1),
             "frac_in_graph": round(chain_bytes / in_graph / 1e3 / HBM_PEAK_GBS, 3),
             "chains_per_graph": len(chains),
             "us_steady": round(steady, 2),
             "us_single_replay": round(single, 2),
             "us_eager_steady": round(_back_to_back(ch.run, 50), 2), "launches": launches}
        if grouped:
            e["us_saved_steady"] = round(saved_steady, 2)
        if flush is not None and grouped:
            e["us_single_replay_cold"] = round(statistics.median(_events(g.replay, cold_iters, flush)) * 1e3, 2)
        res.append(e)
        del ch, g, chains, big
    return res


CHAINS_PER_GRAPH = 12


def _capture_all(chains):
    """One HIP graph running every chain once, in order (warm-up pass first, on a side stream)."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for ch in chains:
            ch.run()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for ch in chains:
            ch.run()
    torch.cuda.synchronize()
    return g


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", choices=["all", "main", "ops", "copy", "chain"], default="all")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--op", choices=["cfg1", "cfg2", "cfg3", "cfg4", "cfg5", "variants", "attn", "sample", "ceiling"], default=None,
                    help="with --only ops: measure one configuration")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the "
              "ops are independent per token/head and shard without exchange", file=sys.stderr)
        sys.exit(2)

    import torch
    from pie_amd import ops
    from pie_amd import workloads as wl
    dev = torch.device("cuda:0")

    if args.only == "copy":  # calibration kernel for the FETCH_SIZE / WRITE_SIZE counters
        a = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        b = torch.empty_like(a)
        for _ in range(args.steps):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy", "bytes_read": a.numel(), "bytes_written": b.numel(),
                          "launches": args.steps}))
        return

    if args.only == "chain":  # decode chain alone (also for kernel traces)
        print(json.dumps({"chain": measure_chain(dev)}))
        return

    ops_res = None
    if args.only in ("all", "ops"):
        ops_res = measure_ops(dev, only=args.op)
        if args.only == "ops":
            print(json.dumps({"ops": ops_res}))
            return

    c = wl.cfg2()
    x, r, w, gu = (c[k].to(dev) for k in ("x", "r", "w", "gate_up"))
    y, s = torch.empty_like(x), torch.empty_like(x)
    act = torch.empty((gu.shape[0], gu.shape[1] // 2), dtype=gu.dtype, device=dev)
    b_add, b_silu = wl.cfg2_bytes()

    def step(ev=None):
        ops.add_rms_norm(x, r, w, c["eps"], out=y, residual_out=s)
        if ev is not None:
            ev[0].record()
        ops.silu_and_mul(gu, out=act)
        if ev is not None:
            ev[1].record()

    for _ in range(args.warmup):
        step()
    # Timed region: exactly K steps, synchronised on both sides, nothing else in the stream.
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    # Second pass over K steps with HIP events around every SiLU-and-mul launch (on the stream
    # the kernels run on): the dominant kernel's average launch duration for the roofline.
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    for i in range(args.steps):
        step(evs[i])
    torch.cuda.synchronize()
    silu_ms = statistics.mean(a.elapsed_time(b) for a, b in evs)
    ms_per_step = dt * 1e3 / args.steps
    step_bytes = b_add + b_silu
    achieved = b_silu / (silu_ms * 1e-3) / 1e9

    # HBM bytes per launch from the committed counter runs (profiles/traffic.json records the
    # command, the calibration, the date and the commit they were measured at)
    traffic = traffic_src = None
    tf = ROOT / "profiles" / "traffic.json"
    if tf.exists():
        tj = json.loads(tf.read_text())
        traffic, traffic_src = tj.get("silu_and_mul_cfg2"), tj.get("silu_and_mul_cfg2_source")

    line = {
        "metric": "achieved HBM GB/s (% of MI355X peak) per fused op; µs per decode-step layer chain",
        "value": round(step_bytes * args.steps / dt / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (seeded N(0,1)/N(1,0.1)/N(0,2) as in the configs)",
        "config": {"workload": "cfg2: fused residual-add+RMSNorm [8192,4096] eps 1e-5 then "
                               "SiLU-and-mul [8192,2x14336] (Llama-3-8B prefill), bf16",
                   "bytes_per_step": step_bytes, "parallelism": "single GPU"},
        "roofline": {"kernel": "silu_and_mul_vec", "bound": "hbm", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "traffic_source": traffic_src,
                     "avg_launch_us": round(silu_ms * 1e3, 2),
                     "algorithmic_bytes": b_silu},
        "cpu_baseline": None if args.no_cpu else cpu_baseline(),
    }
    if not args.no_cpu:
        line["cpu_ops"] = cpu_ops()
    if ops_res is not None:
        line["ops"] = ops_res
    print(json.dumps(line))


if __name__ == "__main__":
    main()
