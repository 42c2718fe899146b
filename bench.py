"""Benchmark of the GRM hot path on one MI355X.

Headline (value): the north-star shape - fused
chunk-update + query application, bf16 q/k/v, fp32 state, B*H = 8 x 8 = 64
sequences, T = 8192, d_k = d_v = 128, chunk = 64, with the 128 per-chunk state
snapshots of every sequence.  One step = one launch of grm_hip_chunk_update_fwd
over the whole batch, inputs resident in HBM, outputs preallocated.
value = tokens/s = 64 * 8192 / (seconds per step); roofline = algorithmic bytes
per launch / average launch duration (HIP events around the timed launches).

Also reported (secondary): config 2 (64 x 2048 tokens), config 2 backward,
config 3 routing (score + top-k + softmax), fused retrieval and the materialised
top-k gather of 128x128 fp32 states (GB/s against HBM peak), config 5 update and
retrieval, config 4 model forward and training step, the reference's published
microbenchmark shape, and the torch-CPU port of the reference's CPU path on the
host (cpu_baseline, the headline workload in full plus slices of the others).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-gather] [--no-cpu]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
FP32_PEAK_TFLOPS = 157.3    # MI355X dense fp32 MFMA
METRIC = "chunk-update+query tokens/s & %MFMA peak; top-k gather GB/s & %HBM, 1 GPU"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def c2_counts(BH=64, T=2048, dk=128, dv=128, C=64, in_b=2, out_b=2):
    """Algorithmic FLOPs and compulsory HBM bytes of one config-2 step."""
    tokens = BH * T
    flops = tokens * (2 * C * (dk + dv) + 4 * dk * dv)
    bytes_ = tokens * (2 * dk + dv) * in_b + tokens * dv * out_b + BH * dv * dk * 4 + BH * (T // C) * dv * dk * 4
    return flops, bytes_


def make_c2(dev, torch, BH=64, T=2048, D=128, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(BH, T, D, generator=g), dim=-1).to(torch.bfloat16)
    k = torch.nn.functional.normalize(torch.randn(BH, T, D, generator=g), dim=-1).to(torch.bfloat16)
    v = torch.randn(BH, T, D, generator=g).to(torch.bfloat16)
    m = torch.randn(BH, D, D, generator=g) * 0.02
    return k, v, q, m


def timed_launches(torch, fn, steps: int, warmup: int, stream):
    """Run fn warmup times, then `steps` times back to back between two events on `stream`.
    Returns the host wall time and [mean seconds per call].  One event pair around all calls:
    an event pair around each call of a short kernel also times the idle gap before the host
    submits it, which is not the kernel's."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        fn()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, [ev0.elapsed_time(ev1) * 1e-3 / steps]


def bench_scan(torch, dev, steps, warmup, BH=64, T=2048, D=128, seed=0, C=64):
    """One grm_hip_chunk_update_fwd launch per step over BH sequences x T tokens (bf16 q/k/v,
    fp32 state, chunk 64, the T/64 per-chunk snapshots written), inputs resident and outputs
    preallocated.  One timed loop of `steps` back-to-back launches after `warmup` untimed ones,
    read by two clocks: the host clock between two synchronisations (wall time per step) and two
    HIP events on the kernel's stream around the same launches (average launch duration, with no
    per-launch event overhead, which is what a kernel trace of these launches reports).  Both
    come from the same launches because the box's clocks drift under sustained load."""
    from rnn_with_grm_amd import capi

    lib = capi.load()
    k, v, q, m = [t.to(dev) for t in make_c2(dev, torch, BH=BH, T=T, D=D, seed=seed)]
    hidden = torch.empty((BH, T, D), dtype=torch.bfloat16, device=dev)
    mem_out = torch.empty((BH, D, D), dtype=torch.float32, device=dev)
    snaps = torch.empty((BH, T // C, D, D), dtype=torch.float32, device=dev)
    wsb = capi.fwd_workspace_bytes(BH, T, D, D, C)
    ws = torch.empty(max(wsb // 4, 1), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    args = (P(k), P(v), P(q), P(m), P(hidden), P(mem_out), P(snaps), P(ws), wsb, BH, T, D, D, capi.BF16, capi.F32,
            0.97, C, sp)

    def step():
        rc = lib.grm_hip_chunk_update_fwd(*args)
        if rc != 0:
            raise RuntimeError(capi.last_error())

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    if not (bool(torch.isfinite(snaps[:, -1]).all()) and torch.equal(snaps[:, -1], mem_out)):
        raise RuntimeError(f"scan {BH}x{T}: last snapshot differs from the final state")
    flops, bytes_ = c2_counts(BH=BH, T=T, dk=D, dv=D, C=C)
    us = ev0.elapsed_time(ev1) * 1e3 / steps
    del k, v, q, m, hidden, snaps, ws, mem_out
    # The box's rate for a stream as large: a device copy moving the same number of bytes
    # (half read, half written), right after the timed launches.
    copy_us, copy_bytes = copy_rate(torch, dev, bytes_, steps, stream)
    return {"wall_s": wall, "us": us, "tokens": BH * T, "flops": flops, "bytes": bytes_,
            "copy_us": copy_us, "copy_bytes": copy_bytes}


def scan_record(r, what):
    """The roofline / MFMA / copy-ceiling record of one bench_scan result."""
    gbs = r["bytes"] / r["us"] / 1e3
    tf = r["flops"] / r["us"] / 1e6
    return {"what": what, "us": round(r["us"], 1), "tokens/s": round(r["tokens"] / r["us"] * 1e6),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_launch": r["bytes"]},
            "mfma": {"TFLOP/s": round(tf, 2), "peak": BF16_PEAK_TFLOPS, "frac": round(tf / BF16_PEAK_TFLOPS, 5),
                     "flops_per_launch": r["flops"]},
            "copy_ceiling": {"what": "a device copy of the same byte count (half read, half written) right after "
                                     "the timed launches, events around the same number of copies",
                             "us": round(r["copy_us"], 1), "GB/s": round(r["copy_bytes"] / r["copy_us"] / 1e3, 1),
                             "kernel_time_vs_copy": round(r["copy_us"] / r["us"], 4)}}


def copy_rate(torch, dev, nbytes, steps, stream):
    """Microseconds per device copy of nbytes in total (nbytes / 2 read, nbytes / 2 written),
    events around `steps` back-to-back copies: the practical ceiling of a stream of that size."""
    n = nbytes // 8
    src = torch.empty(n, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    ev0c, ev1c = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0c.record(stream)
    for _ in range(steps):
        dst.copy_(src)
    ev1c.record(stream)
    torch.cuda.synchronize()
    us = ev0c.elapsed_time(ev1c) * 1e3 / steps
    del src, dst
    return us, 8 * n


def bench_c2_bwd(torch, dev, steps, warmup):
    """chunk_update_backward at config 2 through the C ABI: the forward recompute of the
    chunk states, the adjoint pass and the per-chunk MFMA gradients, timed with events
    around `steps` back-to-back calls."""
    from rnn_with_grm_amd import capi

    k, v, q, m = [t.to(dev) for t in make_c2(dev, torch)]
    BH, T, D = k.shape
    g = torch.Generator().manual_seed(5)
    dh = (torch.randn(BH, T, D, generator=g) * 0.01).to(torch.bfloat16).to(dev)
    dmo = (torch.randn(BH, D, D, generator=g) * 0.01).to(dev)
    stream = torch.cuda.current_stream(dev)

    def step():
        return capi.chunk_update_bwd(dh, dmo, k, v, q, m, 0.97)

    for _ in range(warmup):
        out = step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(steps):
        out = step()
    ev1.record(stream)
    torch.cuda.synchronize()
    if not all(bool(torch.isfinite(t.float()).all()) for t in out):
        raise RuntimeError("config-2 backward produced non-finite gradients")
    return {"ms": ev0.elapsed_time(ev1) / steps, "tokens": BH * T}


def near_ties(torch, lib, capi, q, keys, BH, Q, S, D, K, scale, sp):
    """Rows whose k-th and (k+1)-th routing scores differ by less than 1e-6: one extra
    top-(k+1) call of the same routing kernel, outside every timed region."""
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    dev = q.device
    idx = torch.empty((BH, Q, K + 1), dtype=torch.int64, device=dev)
    sc = torch.empty((BH, Q, K + 1), dtype=torch.float32, device=dev)
    gt = torch.empty((BH, Q, K + 1), dtype=torch.float32, device=dev)
    if lib.grm_hip_topk_route(P(q), P(keys), P(idx), P(sc), P(gt), BH, Q, S, D, capi.BF16, K + 1, scale, 1.0,
                              sp) != 0:
        raise RuntimeError(capi.last_error())
    gap = sc[..., K - 1] - sc[..., K]
    return {"rows": BH * Q, "gap_below_1e-6": int((gap < 1e-6).sum()), "gap_zero": int((gap == 0).sum()),
            "min_gap": float(gap.min())}


def bench_c3(torch, dev, steps, warmup):
    """Routing over the archive summaries; the fused retrieval (gather_apply + fusion); the
    materialised gather."""
    from rnn_with_grm_amd import capi

    lib = capi.load()
    BH, Q, S, D, K = 64, 2048, 256, 128, 8
    g = torch.Generator().manual_seed(1)
    q = torch.nn.functional.normalize(torch.randn(BH, Q, D, generator=g), dim=-1).to(torch.bfloat16).to(dev)
    keys = torch.nn.functional.normalize(torch.randn(BH, S, D, generator=g), dim=-1).to(torch.bfloat16).to(dev)
    states = (torch.randn(BH, S, D, D, device=dev) * 0.02)
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    idx = torch.empty((BH, Q, K), dtype=torch.int64, device=dev)
    sc = torch.empty((BH, Q, K), dtype=torch.float32, device=dev)
    gt = torch.empty((BH, Q, K), dtype=torch.float32, device=dev)
    scale = 1.0 / D ** 0.5

    def route():
        rc = lib.grm_hip_topk_route(P(q), P(keys), P(idx), P(sc), P(gt), BH, Q, S, D, capi.BF16, K, scale, 1.0, sp)
        if rc != 0:
            raise RuntimeError(capi.last_error())

    r_wall, r_per = timed_launches(torch, route, max(3, steps), warmup, stream)
    ties = near_ties(torch, lib, capi, q, keys, BH, Q, S, D, K, scale, sp)
    out = torch.empty((BH, Q, K, D, D), dtype=torch.float32, device=dev)

    def gather():
        rc = lib.grm_hip_batched_gather(P(states), P(idx), P(out), BH, S, Q * K, D * D, 4, None, sp)
        if rc != 0:
            raise RuntimeError(capi.last_error())

    # The fused path: route -> gather_apply -> residual + LayerNorm, no materialised states.
    retrieved = torch.empty((BH, Q, K, D), dtype=torch.float32, device=dev)
    wsb = int(lib.grm_hip_gather_apply_workspace(BH, S, Q * K))
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    online = torch.randn(BH, D, D, device=dev) * 0.02
    h_online = torch.bmm(q.float(), online.transpose(1, 2).contiguous()).reshape(BH * Q, D).contiguous()
    ln_w = torch.ones(D, device=dev)
    ln_b = torch.zeros(D, device=dev)
    fused_out = torch.empty((BH * Q, D), dtype=torch.float32, device=dev)

    def gather_apply():
        rc = lib.grm_hip_gather_apply(P(states), P(idx), P(q), P(retrieved), P(ws), wsb, BH, S, Q, K, D, D, capi.F32,
                                      capi.BF16, capi.F32, None, sp)
        if rc != 0:
            raise RuntimeError(capi.last_error())

    def fuse():
        rc = lib.grm_hip_fuse_residual(P(h_online), P(retrieved), P(gt), P(ln_w), P(ln_b), P(fused_out), BH * Q, K, D,
                                       capi.F32, 1e-5, sp)
        if rc != 0:
            raise RuntimeError(capi.last_error())

    rfb = int(lib.grm_hip_retrieve_fuse_workspace(BH, S, Q * K, D))
    rfws = torch.empty(rfb, dtype=torch.uint8, device=dev)
    h3 = h_online.view(BH, Q, D)
    fused3 = torch.empty_like(h3)

    def retrieve_fuse():
        rc = lib.grm_hip_retrieve_fuse(P(states), P(idx), P(q), P(gt), P(h3), P(ln_w), P(ln_b), P(fused3), P(rfws),
                                       rfb, BH, S, Q, K, D, D, capi.F32, capi.BF16, capi.F32, 1e-5, None, sp)
        if rc != 0:
            raise RuntimeError(capi.last_error())

    def retrieval():
        route()
        retrieve_fuse()

    def composition():
        route()
        gather_apply()
        fuse()

    ga_wall, ga_per = timed_launches(torch, gather_apply, max(3, steps), warmup, stream)
    fu_wall, fu_per = timed_launches(torch, fuse, max(3, steps), warmup, stream)
    rf_wall, rf_per = timed_launches(torch, retrieve_fuse, max(3, steps), warmup, stream)
    rt_wall, rt_per = timed_launches(torch, retrieval, max(3, steps), warmup, stream)
    cp_wall, cp_per = timed_launches(torch, composition, max(3, steps), warmup, stream)
    assert torch.allclose(fused3.view(BH * Q, D), fused_out, rtol=2e-3, atol=2e-3), "retrieve_fuse spot check failed"
    # spot check of the fused path against the materialised composition for one query
    b, qi = 7, 1500
    sel = states[b, idx[b, qi]]                                    # [K, D, D]
    r_ref = torch.einsum("rhk,k->rh", sel, q[b, qi].float())
    assert torch.allclose(retrieved[b, qi], r_ref, rtol=1e-4, atol=1e-6), "gather_apply spot check failed"
    del retrieved, ws, online, h_online, fused_out, rfws, fused3

    g_steps = max(3, min(steps, 10))
    g_wall, g_per = timed_launches(torch, gather, g_steps, min(warmup, 2), stream)
    # spot check: one (b, q, r) row against the archive
    b, qi, r = 5, 777, 3
    s = int(idx[b, qi, r])
    assert torch.equal(out[b, qi, r], states[b, s]), "gather spot check failed"
    # The box's write ceiling for the same 64 GiB: torch's fill kernel over the output.
    f_wall, f_per = timed_launches(torch, out.zero_, 3, 1, stream)
    del out
    route_bytes = q.numel() * 2 + keys.numel() * 2 + idx.numel() * 8 + 2 * sc.numel() * 4
    gather_bytes = BH * Q * K * D * D * 4 + BH * S * D * D * 4 + idx.numel() * 8
    return {
        "route": {"ms": statistics.mean(r_per) * 1e3, "bytes": route_bytes, "near_ties": ties,
                  "flops": 2 * BH * Q * S * D},
        "gather_apply": {"ms": statistics.mean(ga_per) * 1e3,
                         "bytes": BH * S * D * D * 4 + BH * Q * K * D * 4 + q.numel() * 2 + idx.numel() * 8,
                         "flops": 2 * BH * Q * K * D * D},
        "fuse": {"ms": statistics.mean(fu_per) * 1e3},
        "retrieve_fuse": {"ms": statistics.mean(rf_per) * 1e3,
                          "bytes": BH * S * D * D * 4 + q.numel() * 2 + idx.numel() * 8 + gt.numel() * 4 +
                                   2 * BH * Q * D * 4,
                          "intermediate_bytes": 2 * (BH * Q * K * D * 2 + BH * Q * K * 4)},
        "retrieval": {"ms": statistics.mean(rt_per) * 1e3},
        "composition": {"ms": statistics.mean(cp_per) * 1e3},
        "gather": {"ms": statistics.mean(g_per) * 1e3, "bytes": gather_bytes,
                   "fill_ms": statistics.mean(f_per) * 1e3, "fill_bytes": BH * Q * K * D * D * 4},
    }


def bench_routes(torch, dev, steps, warmup):
    """Routing alone (score + top-k + softmax through the C ABI): config 3 (64 sequences x 2048
    queries over 256 keys, top-8) and config 5 (16 heads x 65536 queries over 512 keys, top-16),
    the latter also with causal segment windows (128-token segments)."""
    from rnn_with_grm_amd import capi

    lib = capi.load()
    nrm = torch.nn.functional.normalize
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    out = {}
    for name, (BH, Q, S, D, K) in (("c3", (64, 2048, 256, 128, 8)), ("c5", (16, 65536, 512, 128, 16))):
        g = torch.Generator().manual_seed(1)
        q = nrm(torch.randn(BH, Q, D, generator=g), dim=-1).to(torch.bfloat16).to(dev)
        keys = nrm(torch.randn(BH, S, D, generator=g), dim=-1).to(torch.bfloat16).to(dev)
        idx = torch.empty((BH, Q, K), dtype=torch.int64, device=dev)
        sc = torch.empty((BH, Q, K), dtype=torch.float32, device=dev)
        gt = torch.empty((BH, Q, K), dtype=torch.float32, device=dev)

        def topk():
            rc = lib.grm_hip_topk_route(P(q), P(keys), P(idx), P(sc), P(gt), BH, Q, S, D, capi.BF16, K,
                                        1.0 / D ** 0.5, 1.0, sp)
            if rc != 0:
                raise RuntimeError(capi.last_error())

        def causal():
            rc = lib.grm_hip_segment_route(P(q), P(keys), P(idx), P(sc), P(gt), BH, Q, S, D, capi.BF16, K, 128, 0, S,
                                           1.0 / D ** 0.5, 1.0, sp)
            if rc != 0:
                raise RuntimeError(capi.last_error())

        runs = [(name + "_topk_route", topk)] + ([(name + "_causal_route", causal)] if name == "c5" else [])
        for label, fn in runs:
            _, per = timed_launches(torch, fn, max(3, steps), warmup, stream)
            out[label] = {"us": round(statistics.mean(per) * 1e6, 1), "rows": BH * Q, "keys": S, "top_k": K,
                          "bytes": q.numel() * 2 + keys.numel() * 2 + idx.numel() * 8 + 2 * sc.numel() * 4,
                          "flops": 2 * BH * Q * S * D}
        del q, keys, idx, sc, gt
    return out


def bench_published(torch, dev):
    """The reference's only published figure is its chunk-update microbenchmark
    (examples/benchmark_cuda_chunk_update.py defaults: B=4, 256 tokens, d_v=256, d_k=64, fp32,
    decay 0.97, q and k L2-normalised, memory N(0,1); 10 warm-up and 50 timed calls of the
    cuda_ops entry point, host clock; GRM_Architecture_Blueprint_v2.1.md:266-272 gives 0.219 ms
    native and 0.724 ms for the PyTorch fallback on an unspecified NVIDIA GPU).  The same
    protocol through this repository's cuda_ops entry point, native and fallback."""
    from rnn_with_grm_amd import cuda_ops

    g = torch.Generator().manual_seed(0)
    B, T, H, K = 4, 256, 256, 64
    keys = torch.nn.functional.normalize(torch.randn(B, T, K, generator=g), p=2, dim=-1, eps=1e-6).to(dev)
    queries = torch.nn.functional.normalize(torch.randn(B, T, K, generator=g), p=2, dim=-1, eps=1e-6).to(dev)
    values = torch.randn(B, T, H, generator=g).to(dev)
    memory = torch.randn(B, H, K, generator=g).to(dev)

    def run(debug_fallback):
        for _ in range(10):
            cuda_ops.cuda_chunk_update(keys, values, queries, memory, memory_decay=0.97, enabled=True,
                                       debug_fallback=debug_fallback)
            torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(50):
            cuda_ops.cuda_chunk_update(keys, values, queries, memory, memory_decay=0.97, enabled=True,
                                       debug_fallback=debug_fallback)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / 50 * 1e3

    native, fallback = run(False), run(True)
    return {"what": "the reference's published chunk-update microbenchmark (B=4, 256 tokens, d_v=256, d_k=64, fp32, "
                    "cuda_ops entry point, 50 calls, host clock), same protocol here; published: 0.219 ms native, "
                    "0.724 ms fallback, unspecified NVIDIA GPU",
            "native_ms": round(native, 4), "fallback_ms": round(fallback, 4),
            "native_tokens/s": round(B * T / native * 1e3), "published_native_ms": 0.219,
            "published_fallback_ms": 0.724, "native_vs_published": round(0.219 / native, 2)}


def bench_c5(torch, dev, steps, warmup, update_warmup):
    """Config 5: one whole-sequence update call (16 heads x 65536 tokens, a snapshot every 128
    tokens, 512 per head), then retrieval of k=16 archived states per token over those
    snapshots: route -> gather_apply -> residual + LayerNorm, twice: every token over all 512
    states (the reference's chunk routing has no causal mask), and with causal windows (the
    tokens of segment s over snapshots 0..s-1, the archive of the model's segment loop).
    The update takes the headline's warm-up (update_warmup launches): like the headline
    scan it is timed at the settled clock, after the power controller's dip (about 2.5 to
    10 ms into sustained launches of these kernels)."""
    from rnn_with_grm_amd import capi

    lib = capi.load()
    BH, T, D, SEG, K = 16, 65536, 128, 128, 16
    S = T // SEG
    nrm = torch.nn.functional.normalize
    g = torch.Generator().manual_seed(5)
    q = nrm(torch.randn(BH, T, D, generator=g), dim=-1).to(torch.bfloat16).to(dev)
    k = nrm(torch.randn(BH, T, D, generator=g), dim=-1).to(torch.bfloat16).to(dev)
    v = torch.randn(BH, T, D, generator=g).to(torch.bfloat16).to(dev)
    m0 = (torch.randn(BH, D, D, generator=g) * 0.02).to(dev)
    summaries = nrm(torch.randn(BH, S, D, generator=g), dim=-1).to(torch.bfloat16).to(dev)
    hidden = torch.empty(BH, T, D, dtype=torch.bfloat16, device=dev)
    snaps = torch.empty(BH, S, D, D, device=dev)
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    wsb = int(lib.grm_hip_chunk_update_fwd_workspace(BH, T, D, D, SEG))
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)

    def update():
        rc = lib.grm_hip_chunk_update_fwd(P(k), P(v), P(q), P(m0), P(hidden), None, P(snaps), P(ws), wsb, BH, T, D,
                                          D, capi.BF16, capi.F32, 0.97, SEG, sp)
        if rc != 0:
            raise RuntimeError(capi.last_error())

    u_wall, u_per = timed_launches(torch, update, max(3, steps), update_warmup, stream)
    idx = torch.empty((BH, T, K), dtype=torch.int64, device=dev)
    sc = torch.empty((BH, T, K), dtype=torch.float32, device=dev)
    gt = torch.empty((BH, T, K), dtype=torch.float32, device=dev)
    retrieved = torch.empty((BH, T, K, D), dtype=torch.float32, device=dev)
    wsb2 = int(lib.grm_hip_gather_apply_workspace(BH, S, T * K))
    ws2 = torch.empty(wsb2, dtype=torch.uint8, device=dev)
    h_online = hidden.float().reshape(BH * T, D).contiguous()
    ln_w = torch.ones(D, device=dev)
    ln_b = torch.zeros(D, device=dev)
    fused_out = torch.empty((BH * T, D), dtype=torch.float32, device=dev)

    def route():
        rc = lib.grm_hip_topk_route(P(q), P(summaries), P(idx), P(sc), P(gt), BH, T, S, D, capi.BF16, K,
                                    1.0 / D ** 0.5, 1.0, sp)
        if rc != 0:
            raise RuntimeError(capi.last_error())

    def gather_apply():
        rc = lib.grm_hip_gather_apply(P(snaps), P(idx), P(q), P(retrieved), P(ws2), wsb2, BH, S, T, K, D, D,
                                      capi.F32, capi.BF16, capi.F32, None, sp)
        if rc != 0:
            raise RuntimeError(capi.last_error())

    def fuse():
        rc = lib.grm_hip_fuse_residual(P(h_online), P(retrieved), P(gt), P(ln_w), P(ln_b), P(fused_out), BH * T, K,
                                       D, capi.F32, 1e-5, sp)
        if rc != 0:
            raise RuntimeError(capi.last_error())

    rfb = int(lib.grm_hip_retrieve_fuse_workspace(BH, S, T * K, D))
    rfws = torch.empty(rfb, dtype=torch.uint8, device=dev)
    h5 = h_online.view(BH, T, D)
    fused5 = torch.empty_like(h5)

    def retrieve_fuse():
        rc = lib.grm_hip_retrieve_fuse(P(snaps), P(idx), P(q), P(gt), P(h5), P(ln_w), P(ln_b), P(fused5), P(rfws),
                                       rfb, BH, S, T, K, D, D, capi.F32, capi.BF16, capi.F32, 1e-5, None, sp)
        if rc != 0:
            raise RuntimeError(capi.last_error())

    def retrieval():
        route()
        retrieve_fuse()

    def composition():
        route()
        gather_apply()
        fuse()

    def route_causal():
        # segment s (128 tokens) sees the snapshots of segments < s, as in the model's segment loop
        rc = lib.grm_hip_segment_route(P(q), P(summaries), P(idx), P(sc), P(gt), BH, T, S, D, capi.BF16, K, SEG, 0,
                                       S, 1.0 / D ** 0.5, 1.0, sp)
        if rc != 0:
            raise RuntimeError(capi.last_error())

    def retrieval_causal():
        route_causal()
        retrieve_fuse()  # empty slots (index -1) contribute nothing

    n = max(3, min(steps, 10))
    r_wall, r_per = timed_launches(torch, route, n, min(warmup, 2), stream)
    ties = near_ties(torch, lib, capi, q, summaries, BH, T, S, D, K, 1.0 / D ** 0.5, sp)
    ga_wall, ga_per = timed_launches(torch, gather_apply, n, min(warmup, 2), stream)
    fu_wall, fu_per = timed_launches(torch, fuse, n, min(warmup, 2), stream)
    rf_wall, rf_per = timed_launches(torch, retrieve_fuse, n, min(warmup, 2), stream)
    rt_wall, rt_per = timed_launches(torch, retrieval, n, min(warmup, 2), stream)
    cp_wall, cp_per = timed_launches(torch, composition, n, min(warmup, 2), stream)
    # spot checks: one token's retrieval against the composition, and its last snapshot
    b, t = 3, 40000
    r_ref = torch.einsum("rhk,k->rh", snaps[b, idx[b, t]], q[b, t].float())
    assert torch.allclose(retrieved[b, t], r_ref, rtol=1e-4, atol=1e-6), "c5 gather_apply spot check failed"
    assert torch.allclose(fused5.view(BH * T, D)[b * T + t], fused_out[b * T + t], rtol=2e-3, atol=2e-3), \
        "c5 retrieve_fuse spot check failed"
    assert bool(torch.isfinite(snaps[:, -1]).all()), "c5 snapshots not finite"
    rc_wall, rc_per = timed_launches(torch, route_causal, n, min(warmup, 2), stream)
    rtc_wall, rtc_per = timed_launches(torch, retrieval_causal, n, min(warmup, 2), stream)
    assert int(idx[b, t].max()) < t // SEG and int(idx[b, t].min()) >= 0, "c5 causal window violated"
    tokens = BH * T
    upd_bytes = tokens * (2 * D + D) * 2 + tokens * D * 2 + BH * D * D * 4 + BH * S * D * D * 4
    out = {
        "update": {"us": statistics.mean(u_per) * 1e6, "bytes": upd_bytes, "tokens": tokens},
        "route": {"ms": statistics.mean(r_per) * 1e3, "flops": 2 * tokens * S * D, "near_ties": ties},
        "gather_apply": {"ms": statistics.mean(ga_per) * 1e3,
                         "bytes": BH * S * D * D * 4 + tokens * K * D * 4 + q.numel() * 2 + idx.numel() * 8,
                         "flops": 2 * tokens * K * D * D},
        "fuse": {"ms": statistics.mean(fu_per) * 1e3},
        "retrieve_fuse": {"ms": statistics.mean(rf_per) * 1e3,
                          "bytes": BH * S * D * D * 4 + q.numel() * 2 + idx.numel() * 8 + gt.numel() * 4 +
                                   2 * tokens * D * 4,
                          "intermediate_bytes": 2 * (tokens * K * D * 2 + tokens * K * 4)},
        "retrieval": {"ms": statistics.mean(rt_per) * 1e3, "tokens": tokens},
        "composition": {"ms": statistics.mean(cp_per) * 1e3},
        "route_causal": {"ms": statistics.mean(rc_per) * 1e3},
        "retrieval_causal": {"ms": statistics.mean(rtc_per) * 1e3},
    }
    del retrieved, h_online, fused_out, ws2, idx, sc, gt, snaps, hidden, q, k, v, rfws, fused5
    return out


def bench_c4_archive(torch, dev, steps, warmup):
    """Config 4's per-segment retrieval (B=4, hidden 512, d_k 64, 64-token segments, k=8, a full
    64-segment float16 archive), two ways:
      reference style - the retriever's own composition (paper_grm.py:227-229,301-313): stack the
                        64 archived states, widen to float32, gather [B,64,8,512,64], apply;
      device archive  - DeviceSegmentArchive.retrieve_from_indices: the float16 ring read in place
                        by one fused gather + apply with float32 widening on load."""
    from types import SimpleNamespace

    from rnn_with_grm_amd import cuda_ops
    from rnn_with_grm_amd.archive import DeviceSegmentArchive

    B, H, K, SEG, R, CAP, DIN = 4, 512, 64, 64, 8, 64, 512
    g = torch.Generator().manual_seed(4)
    mems = [(torch.randn(B, H, K, generator=g) * 0.02).to(torch.float16).to(dev) for _ in range(CAP)]
    summ = torch.randn(B, CAP, DIN, generator=g).to(dev)
    arch = DeviceSegmentArchive(H, K, DIN, CAP, torch.float16).to(dev)
    arch.push_segments(torch.stack(mems, 1), summ)
    cell = SimpleNamespace(query_proj=torch.nn.Linear(DIN, K).to(dev))
    x = torch.randn(B, SEG, DIN, generator=g).to(dev)
    idx = torch.randint(0, CAP, (B, SEG, R), generator=g).to(dev)
    stream = torch.cuda.current_stream(dev)

    def reference_style():
        allm = torch.stack(mems, dim=0).to(torch.float32).permute(1, 0, 2, 3).contiguous()
        sel = cuda_ops.cuda_batched_memory_gather(allm, idx)
        q = torch.nn.functional.normalize(cell.query_proj(x), p=2, dim=-1, eps=1e-6).to(sel.dtype)
        return cuda_ops.cuda_apply_query(sel, q)

    def device_archive():
        return arch.retrieve_from_indices(x, idx, None, cell, dev, 0.97)

    with torch.no_grad():
        a, b = reference_style(), device_archive()
        assert torch.allclose(a, b, rtol=1e-4, atol=1e-5), "c4 archive retrieval mismatch"
        r_wall, r_per = timed_launches(torch, reference_style, max(3, steps), warmup, stream)
        d_wall, d_per = timed_launches(torch, device_archive, max(3, steps), warmup, stream)
    return {"reference_style_ms": statistics.mean(r_per) * 1e3, "device_archive_ms": statistics.mean(d_per) * 1e3}


class SegmentMemoryLM:
    """Config 4's language model: Embedding(32000, 512) -> HierarchicalSegmentMemoryModel
    (4 layers, hidden 512, d_k 64, 64-token segments, capacity 64, top-8, float16 archive)
    -> Linear(512, 32000), the composition of the reference's SegmentMemoryLanguageModel
    (grm/utils/train.py:192-229).  Random init, bfloat16 weights."""

    def __init__(self, torch, dev, vocab=32000, dim=512, layers=4, dk=64, seg=64, top_k=8):
        from rnn_with_grm_amd.segment_model import HierarchicalSegmentMemoryModel

        torch.manual_seed(0)
        self.embedding = torch.nn.Embedding(vocab, dim)
        self.grm = HierarchicalSegmentMemoryModel(dim, dim, dim, num_layers=layers, segment_length=seg,
                                                  memory_capacity_segments=64, retrieval_top_k=top_k,
                                                  memory_key_dim=dk, dropout=0.0, recomputation_ratio=0.0)
        self.head = torch.nn.Linear(dim, vocab)
        for m in (self.embedding, self.grm, self.head):
            m.to(device=dev, dtype=torch.bfloat16).eval()

    def __call__(self, ids):
        from rnn_with_grm_amd import segment_model

        x = self.embedding(ids)
        segment_model._mark("embedding", x)
        out, _, _, _ = self.grm(x, reset_memory=True)
        segment_model._mark("other (between phases)", out)
        logits = self.head(out)
        segment_model._mark("LM head GEMM (512 -> 32000)", logits)
        return logits


def bench_c4_model(torch, dev, steps, warmup):
    """Config 4 end to end: one forward over 4 x 8192 token ids, every layer as whole-sequence
    launches (scan, segment routing, gather_apply, fusion), the archive reset each step."""
    B, T = 4, 8192
    lm = SegmentMemoryLM(torch, dev)
    g = torch.Generator().manual_seed(7)
    ids = torch.randint(0, 32000, (B, T), generator=g).to(dev)
    stream = torch.cuda.current_stream(dev)
    with torch.no_grad():
        logits = lm(ids)
        assert logits.shape == (B, T, 32000) and torch.isfinite(logits.float()).all(), "c4 forward not finite"
        wall, per = timed_launches(torch, lambda: lm(ids), max(3, min(steps, 10)), max(1, min(warmup, 3)), stream)
        # Per-phase breakdown of one more forward, from events at the phase boundaries
        # (summed over the 4 layers); the timed forwards above record none.
        from rnn_with_grm_amd import segment_model

        segment_model.PHASE_EVENTS = []
        segment_model._mark("start", ids)
        lm(ids)
        torch.cuda.synchronize()
        phases = segment_model.phase_times_ms()
        segment_model.PHASE_EVENTS = None
    ms = statistics.mean(per) * 1e3
    return {"ms": ms, "tokens": B * T, "phases_ms": phases}


def host_cpu_info():
    """The host's CPU model, logical CPU count, the CPUs this process may run on and its
    cgroup CPU quota; `usable` is the smallest of these, the thread count the CPU legs use."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    count = os.cpu_count() or 1
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else count
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
            if q != "max":
                quota = float(q) / float(period)
    except (OSError, ValueError):
        pass
    usable = min(count, affinity, int(quota) if quota and quota >= 1 else count)
    return {"cpu_model": model, "os_cpu_count": count, "affinity_cpus": affinity, "cgroup_cpu_quota": quota,
            "usable": max(1, usable)}


def _median_seconds(fn, min_runs=5, budget_s=4.0):
    """One warm-up call, then at least min_runs timed calls (more while within budget_s)."""
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baseline(torch):
    """The torch-CPU port of the reference's CPU path on the host, at the usable core count
    and at one thread: config 1 and config 2 at full shape, configs 3 and 5 on slices whose
    time is scaled linearly to the full configuration (stated per leg)."""
    from oracle import torch_port

    host = host_cpu_info()
    nrm = torch.nn.functional.normalize
    g = torch.Generator().manual_seed(0)
    # config 1: fp32, B*H = 8, T = 512, d = 64, chunk 64, zero initial state
    k1 = nrm(torch.randn(8, 512, 64, generator=g), dim=-1)
    v1 = torch.randn(8, 512, 64, generator=g)
    q1 = nrm(torch.randn(8, 512, 64, generator=g), dim=-1)
    m1 = torch.zeros(8, 64, 64)
    k2, v2, q2, m2 = make_c2(None, torch)
    kn, vn, qn, mn = make_c2(None, torch, BH=64, T=8192, seed=3)
    # config 3 slice: one of the 64 (b, h) sequences, 256 of its 2048 queries (x 512 to the full batch)
    q3 = nrm(torch.randn(1, 256, 128, generator=g), dim=-1).to(torch.bfloat16)
    keys3 = nrm(torch.randn(1, 256, 128, generator=g), dim=-1).to(torch.bfloat16)
    st3 = torch.randn(1, 256, 128, 128, generator=g) * 0.02
    h3 = torch.randn(256, 128, generator=g)
    # config 5 slices: the update over one head's first 4096 tokens (x 256 to 16 heads x 65536), and
    # the retrieval of 256 tokens of one head over its 512 snapshots (x 4096)
    k5 = nrm(torch.randn(1, 4096, 128, generator=g), dim=-1).to(torch.bfloat16)
    v5 = torch.randn(1, 4096, 128, generator=g).to(torch.bfloat16)
    q5 = nrm(torch.randn(1, 4096, 128, generator=g), dim=-1).to(torch.bfloat16)
    m5 = torch.randn(1, 128, 128, generator=g) * 0.02
    keys5 = nrm(torch.randn(1, 512, 128, generator=g), dim=-1).to(torch.bfloat16)
    st5 = torch.randn(1, 512, 128, 128, generator=g) * 0.02
    ln_w, ln_b = torch.ones(128), torch.zeros(128)

    def retrieval(q, keys, states, h, top_k):
        gates, idx, _ = torch_port.route(q, keys, top_k, 1.0 / 128 ** 0.5)
        sel = torch_port.gather(states, idx)
        r = torch_port.apply_query(sel, q.float())
        return torch_port.fuse_residual(h, r[0], gates[0], ln_w, ln_b)

    legs = [
        ("n1", "full north-star shape (64 x 8192 tokens, d=128, chunk 64, bf16 inputs, fp32 math, 128 snapshots "
               "per sequence)", 64 * 8192, 1, lambda: torch_port.segment_scan(kn, vn, qn, mn, 0.97, 64)),
        ("c1", "full config 1 (fp32, 8 x 512 tokens, d=64, chunk 64)", 8 * 512, 1,
         lambda: torch_port.segment_scan(k1, v1, q1, m1, 0.97, 64)),
        ("c2", "full config 2 (64 x 2048 tokens, d=128, bf16 inputs, fp32 math)", 64 * 2048, 1,
         lambda: torch_port.segment_scan(k2, v2, q2, m2, 0.97, 64)),
        ("c3_retrieval", "config 3 slice: 256 queries of 1 of 64 sequences, route top-8 of 256, gather, apply, "
         "fuse; time x 512 for the full 64 x 2048 queries", 256, 512, lambda: retrieval(q3, keys3, st3, h3, 8)),
        ("c5_update", "config 5 slice: 4096 tokens of 1 of 16 heads, chunk 128; time x 256 for 16 x 65536 tokens",
         4096, 256, lambda: torch_port.segment_scan(k5, v5, q5, m5, 0.97, 128)),
        ("c5_retrieval", "config 5 slice: 256 tokens of 1 of 16 heads, route top-16 of 512, gather, apply, fuse; "
         "time x 4096 for 16 x 65536 tokens", 256, 4096,
         lambda: retrieval(q5[:, :256], keys5, st5, h3, 16)),
    ]
    out = {}
    for threads in (host["usable"], 1):
        torch.set_num_threads(threads)
        res = {}
        for name, what, tokens, scale, fn in legs:
            sec, runs = _median_seconds(fn, budget_s=2.0 if threads > 1 else 3.0)
            res[name] = {"sample": what, "slice_seconds": round(sec, 6), "runs": runs,
                         "full_config_seconds": round(sec * scale, 4),
                         "tokens/s": round(tokens / sec)}
        out[threads] = res
    threads = host["usable"]
    n1 = out[threads]["n1"]
    return {"value": n1["tokens/s"], "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"the headline workload in full: north-star shape (64 x 8192 tokens, d=128, chunk 64, fp32 math "
                      f"on bf16-rounded inputs, the 128 snapshots per sequence kept), one _vectorized_chunk_update "
                      f"per 64-token segment (cuda_ops.py:218-254), median of {n1['runs']} runs of "
                      f"{n1['slice_seconds']:.2f} s on {threads} threads (the host's usable CPUs: min of "
                      f"os.cpu_count(), affinity and cgroup quota)",
            "host": host, "one_thread": out[1], "legs": out[threads]}


def bench_c4_train(torch, dev, steps, warmup):
    """Config 4 training forward + backward (no optimizer step): the same LM and token ids,
    cross-entropy over next-token targets, loss.backward() through the scan's MFMA backward,
    the routing, and the retrieval with its LayerNorm residual as one autograd function (the
    transposed apply per query and route, no gathered states, no per-route rows kept).
    Returns the mean step and the generic-path calls the steps made."""
    from rnn_with_grm_amd import cuda_ops

    B, T, V = 4, 8192, 32000
    lm = SegmentMemoryLM(torch, dev)
    params = [p for m in (lm.embedding, lm.grm, lm.head) for p in m.parameters()]
    g = torch.Generator().manual_seed(7)
    ids = torch.randint(0, V, (B, T), generator=g).to(dev)
    targets = torch.roll(ids, -1, dims=1)
    stream = torch.cuda.current_stream(dev)
    torch.cuda.reset_peak_memory_stats(dev)  # this leg's own peak, not the earlier legs'

    def step():
        for p in params:
            p.grad = None
        logits = lm(ids)
        loss = torch.nn.functional.cross_entropy(logits.view(B * T, V).float(), targets.view(-1))
        loss.backward()

    step()
    torch.cuda.synchronize()
    grads = [p.grad for p in params if p.grad is not None]
    assert len(grads) > len(params) // 2 and all(torch.isfinite(t.float()).all() for t in grads), \
        "c4 training gradients missing or not finite"
    generic0 = cuda_ops.get_grm_cuda_runtime_status()["hip"]["generic_path_calls"]
    wall, per = timed_launches(torch, step, max(3, min(steps, 8)), max(1, min(warmup, 2)), stream)
    generic = cuda_ops.get_grm_cuda_runtime_status()["hip"]["generic_path_calls"] - generic0
    return {"ms": statistics.mean(per) * 1e3, "tokens": B * T, "generic_path_calls": generic,
            "peak_gib": torch.cuda.max_memory_allocated(dev) / 2 ** 30}


def retrieval_roofline(ms, flops, alg_bytes, rows_bytes=None):
    """Roofline of a fused retrieval launch: max(F / P, B / BW) with F the float32-semantics FLOPs of the
    gathered applies (2 per multiply-add of every selected 128 x 128 state with its query) against the
    dense float32 MFMA peak, and B its algorithmic HBM bytes against 8 TB/s.  The kernel computes the
    float32 products as three bf16 MFMA products (hi*hi + hi*lo + lo*hi), so the bf16 rate it issues is
    reported beside it."""
    t_f = flops / (FP32_PEAK_TFLOPS * 1e12)
    t_b = alg_bytes / (HBM_PEAK_GBS * 1e9)
    t = ms * 1e-3
    rec = {"bound": "mfma_fp32" if t_f >= t_b else "hbm", "achieved": round(max(t_f, t_b) / t, 4), "peak": 1.0,
           "unit": "fraction of roofline time", "frac": round(max(t_f, t_b) / t, 4),
           "fp32_TFLOP/s": round(flops / t / 1e12, 1), "fp32_peak_TFLOP/s": FP32_PEAK_TFLOPS,
           "fp32_floor_ms": round(t_f * 1e3, 4), "hbm_GB/s": round(alg_bytes / t / 1e9, 1),
           "hbm_floor_ms": round(t_b * 1e3, 4), "algorithmic_bytes": alg_bytes, "flops": flops,
           "bf16x3_issued_TFLOP/s": round(3 * flops / t / 1e12, 1)}
    if rows_bytes is not None:
        rec["traffic"] = {"float16_rows_written_and_read": rows_bytes, "over_algorithmic": round(
            (alg_bytes + rows_bytes) / alg_bytes, 3)}
    return rec


def committed_traffic(name, source):
    """HBM bytes per launch from a committed counter summary (profiles/<name>: FETCH_SIZE and
    WRITE_SIZE of the kernel, scaled by a copy of known size), with the sha256 of the kernel
    source it was measured on.  A summary measured on other source is stale: None, and a note."""
    import hashlib

    f = REPO / "profiles" / name
    if not f.exists():
        return None, f"no counter summary {f.name}"
    try:
        rec = json.loads(f.read_text())
    except ValueError:
        return None, f"{f.name} unreadable"
    src = REPO / "rnn_with_grm_amd" / "csrc" / source
    sha = hashlib.sha256(src.read_bytes()).hexdigest()[:16]
    if rec.get("source_sha256_16") != sha:
        return None, f"{f.name} was measured on another {source} ({rec.get('source_sha256_16')} vs {sha})"
    return rec.get("hbm_bytes_per_launch"), f"profiles/{f.name}: {rec.get('command', '')}"


def settle(torch) -> None:
    """Between legs: drain the GPU, hand cached blocks back and idle for two seconds, so
    that each leg starts from the same clock and allocator state (the legs before config
    4 write 64 GiB and more, after which the box's clocks step down for a while)."""
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    time.sleep(2.0)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # 120 warm-up launches of the headline scan (about 30 ms): the board's power controller lowers the
    # clocks for the first tens of back-to-back launches of this kernel and then restores them, so the
    # timed launches start once the rate has settled (measured: 233-250 us, a dip to 270-287 us over
    # launches 10-25, 240 us around launch 100, then 238 us from launch 120 on, steady over 600 launches).
    ap.add_argument("--warmup", type=int, default=120)
    ap.add_argument("--no-gather", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--c2-only", action="store_true", help="only the headline kernel (quick sweeps)")
    ap.add_argument("--c4-only", action="store_true", help="the headline kernel and the config-4 model forward")
    ap.add_argument("--train-only", action="store_true",
                    help="the headline kernel and the config-4 training forward + backward")
    ap.add_argument("--bwd-only", action="store_true", help="the headline kernel and the config-2 backward")
    ap.add_argument("--route-only", action="store_true", help="the headline kernel and config 3 / 5 routing")
    ap.add_argument("--probe", action="store_true",
                    help="counter runs: a 256 MiB device copy (calibration), then launches of one scan shape only")
    ap.add_argument("--probe-shape", choices=("n1", "c2", "c5"), default="n1",
                    help="the scan shape of --probe: the north-star shape (the headline), config 2 or config 5")
    a = ap.parse_args()
    if a.c2_only or a.probe or a.c4_only or a.bwd_only or a.route_only or a.train_only:
        a.no_gather = a.no_cpu = True
    if a.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {a.gpus} is not supported in this build "
              "(the hot path shards with zero communication over (b,h) sequences; see the design notes)",
              file=sys.stderr)
        return 2
    import torch

    from rnn_with_grm_amd import cuda_ops

    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    if not cuda_ops.load_grm_cuda_extension():
        raise RuntimeError(f"GRM HIP extension not loaded: {cuda_ops.extension_load_error()}")
    dev = torch.device("cuda:0")

    if a.probe:
        # Calibration for HBM byte counters: a plain copy of a known size.
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"probe copy: {src.numel()} bytes read and written")
        del src, dst
        if a.probe_shape != "n1":
            shape = {"c2": dict(BH=64, T=2048, seed=0), "c5": dict(BH=16, T=65536, seed=5, C=128)}[a.probe_shape]
            r = bench_scan(torch, dev, a.steps, min(a.warmup, 5), **shape)
            log(f"probe {a.probe_shape}: {r['us']:.1f} us/launch, {r['bytes'] / r['us'] / 1e3:.0f} GB/s")
            return 0

    # Headline: the north-star shape (B=8 x H=8 sequences x 8192 tokens, d = 128, chunk 64).
    log(f"north-star shape fused chunk-update+query (64 x 8192 tokens): warmup {a.warmup}, steps {a.steps}")
    n1 = bench_scan(torch, dev, a.steps, a.warmup, BH=64, T=8192, seed=3)
    sec_w = min(a.warmup, 5)  # warm-up of the secondary legs
    t_step = n1["wall_s"] / a.steps
    t_kernel = n1["us"] * 1e-6
    tokens, flops, bytes_ = n1["tokens"], n1["flops"], n1["bytes"]
    achieved_gbs = bytes_ / t_kernel / 1e9
    tflops = flops / t_kernel / 1e12
    log(f"n1: {n1['us']:.1f} us/launch (events around {a.steps} launches), {t_step * 1e6:.1f} us/step (wall), "
        f"{achieved_gbs:.0f} GB/s; a copy of the same bytes {n1['copy_us']:.1f} us "
        f"({n1['copy_bytes'] / n1['copy_us'] / 1e3:.0f} GB/s)")
    traffic, traffic_note = committed_traffic("scan_vsplit_n1_traffic.json", "chunk_scan_vsplit.hip")

    secondary = {}
    if not a.probe:
        log("config 2 fused chunk-update+query (64 x 2048 tokens)")
        c2 = bench_scan(torch, dev, a.steps, sec_w, BH=64, T=2048, seed=0)
        secondary["c2_update"] = scan_record(
            c2, "BASELINE config 2: fused chunk-update + query, 64 sequences x 2048 tokens, d_k=d_v=128, chunk 64, "
                "bf16 q/k/v, fp32 state, 32 snapshots per sequence; one launch per step (scan_vsplit_kernel)")
        c2_tr, c2_note = committed_traffic("scan_vsplit_c2_traffic.json", "chunk_scan_vsplit.hip")
        secondary["c2_update"]["roofline"]["traffic"] = c2_tr
        secondary["c2_update"]["roofline"]["traffic_note"] = c2_note
        log(f"c2: {c2['us']:.1f} us/launch, {c2['bytes'] / c2['us'] / 1e3:.0f} GB/s")
    if a.route_only:
        log("routing only: config 3 and config 5")
        for label, r in bench_routes(torch, dev, a.steps, sec_w).items():
            secondary[label] = dict(r, **{"GB/s": round(r["bytes"] / r["us"] / 1e3, 1),
                                          "TFLOP/s": round(r["flops"] / r["us"] / 1e6, 2)})
            log(f"{label}: {r['us']:.1f} us")
    if not a.no_gather or a.bwd_only:
        log("config 2 backward (chunk_update_backward: recompute, adjoint pass, per-chunk MFMA gradients)")
        bw = bench_c2_bwd(torch, dev, max(3, a.steps // 2), 2)
        secondary["c2_backward"] = {
            "what": "chunk_update_backward at config 2 (bf16 q/k/v, fp32 state): forward recompute of the 32 "
                    "chunk states, adjoint pass, per-chunk MFMA gradients; events around back-to-back calls",
            "ms": round(bw["ms"], 4), "tokens/s": round(bw["tokens"] / bw["ms"] * 1e3)}
        log(f"c2 backward: {bw['ms']:.3f} ms per call")
    if not a.no_gather:
        settle(torch)
        log("config 3 routing + materialised gather (64 GiB output)")
        c3 = bench_c3(torch, dev, a.steps, sec_w)
        r, gth = c3["route"], c3["gather"]
        secondary["c3_topk_route"] = {"ms": round(r["ms"], 4), "GB/s": round(r["bytes"] / r["ms"] / 1e6, 1),
                                      "TFLOP/s": round(r["flops"] / r["ms"] / 1e9, 2), "near_ties": r["near_ties"]}
        gbs = gth["bytes"] / gth["ms"] / 1e6
        secondary["c3_gather"] = {"ms": round(gth["ms"], 3), "GB/s": round(gbs, 1),
                                  "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                                  "bytes": gth["bytes"], "bytes_convention": "compulsory: out write + archive read + idx",
                                  "write_ceiling": {"what": "torch fill of the same 64 GiB output",
                                                    "ms": round(gth["fill_ms"], 3),
                                                    "GB/s": round(gth["fill_bytes"] / gth["fill_ms"] / 1e6, 1),
                                                    "gather_time_vs_fill": round(gth["fill_ms"] / gth["ms"], 4)}}
        log(f"c3 gather: {gth['ms']:.2f} ms, {gbs:.0f} GB/s (fill of the output: {gth['fill_ms']:.2f} ms)")
        ga, rt = c3["gather_apply"], c3["retrieval"]
        secondary["c3_retrieval_fused"] = {
            "what": "route -> retrieve_fuse (gather + apply + gate-weighted sum + residual + LayerNorm, no "
                    "materialised states, row-scaled float16 per-route rows), per config-3 batch; the two-kernel "
                    "composition (gather_apply in float32, then fuse_residual) beside it",
            "ms": round(rt["ms"], 4), "route_ms": round(r["ms"], 4),
            "retrieve_fuse_ms": round(c3["retrieve_fuse"]["ms"], 4),
            "retrieve_fuse_roofline": retrieval_roofline(c3["retrieve_fuse"]["ms"], ga["flops"],
                                                         c3["retrieve_fuse"]["bytes"],
                                                         c3["retrieve_fuse"]["intermediate_bytes"]),
            "composition_ms": round(c3["composition"]["ms"], 4), "gather_apply_ms": round(ga["ms"], 4),
            "fuse_ms": round(c3["fuse"]["ms"], 4),
            "gather_apply_GB/s": round(ga["bytes"] / ga["ms"] / 1e6, 1),
            "gather_apply_TFLOP/s_fp32": round(ga["flops"] / ga["ms"] / 1e9, 2),
            "speedup_vs_materialised_gather_alone": round(gth["ms"] / rt["ms"], 2)}
        log(f"c3 fused retrieval: {rt['ms']:.3f} ms (route {r['ms']:.3f}, retrieve_fuse "
            f"{c3['retrieve_fuse']['ms']:.3f}); composition {c3['composition']['ms']:.3f} (gather_apply "
            f"{ga['ms']:.3f}, fuse {c3['fuse']['ms']:.3f})")

    if not a.no_gather:
        settle(torch)
        log("config 5: whole-sequence update (16 x 65536 tokens, 512 snapshots) + k=16 retrieval per token")
        c5 = bench_c5(torch, dev, a.steps, sec_w, a.warmup)
        u, rt5, ga5 = c5["update"], c5["retrieval"], c5["gather_apply"]
        ugbs = u["bytes"] / u["us"] / 1e3
        secondary["c5_update"] = {"us": round(u["us"], 1), "tokens/s": round(u["tokens"] / u["us"] * 1e6),
                                  "GB/s": round(ugbs, 1), "hbm_frac": round(ugbs / HBM_PEAK_GBS, 4),
                                  "bytes": u["bytes"], "warmup_launches": a.warmup}
        rf5 = c5["retrieve_fuse"]
        secondary["c5_retrieval_fused"] = {
            "what": "route (top-16 of 512 snapshots per token) -> retrieve_fuse (gather + apply + gate-weighted sum "
                    "+ residual + LayerNorm), every token routed over all 512 states (no causal mask, as the "
                    "reference's chunk path); the two-kernel composition (gather_apply float32 rows, then "
                    "fuse_residual) beside it",
            "ms": round(rt5["ms"], 3), "tokens/s": round(rt5["tokens"] / rt5["ms"] * 1e3),
            "route_ms": round(c5["route"]["ms"], 3), "route_near_ties": c5["route"]["near_ties"],
            "retrieve_fuse_ms": round(rf5["ms"], 3),
            "retrieve_fuse_roofline": retrieval_roofline(rf5["ms"], ga5["flops"], rf5["bytes"],
                                                         rf5["intermediate_bytes"]),
            "composition_ms": round(c5["composition"]["ms"], 3), "gather_apply_ms": round(ga5["ms"], 3),
            "fuse_ms": round(c5["fuse"]["ms"], 3),
            "route_TFLOP/s": round(c5["route"]["flops"] / c5["route"]["ms"] / 1e9, 1),
            "gather_apply_GB/s": round(ga5["bytes"] / ga5["ms"] / 1e6, 1),
            "gather_apply_TFLOP/s_fp32": round(ga5["flops"] / ga5["ms"] / 1e9, 1)}
        secondary["c5_retrieval_causal"] = {
            "what": "the same retrieval with causal windows (segment routing: the tokens of segment s route over "
                    "snapshots 0..s-1, as in the model's segment loop), route -> retrieve_fuse",
            "ms": round(c5["retrieval_causal"]["ms"], 3),
            "tokens/s": round(rt5["tokens"] / c5["retrieval_causal"]["ms"] * 1e3),
            "route_ms": round(c5["route_causal"]["ms"], 3)}
        log(f"c5 update: {u['us']:.1f} us ({ugbs:.0f} GB/s); retrieval {rt5['ms']:.2f} ms (route "
            f"{c5['route']['ms']:.2f}, retrieve_fuse {rf5['ms']:.2f}); composition {c5['composition']['ms']:.2f} "
            f"(gather_apply {ga5['ms']:.2f}, fuse {c5['fuse']['ms']:.2f})")

    if not a.no_gather:
        c4 = bench_c4_archive(torch, dev, a.steps, sec_w)
        secondary["c4_segment_retrieval"] = {
            "what": "one 64-token segment's retrieval at config 4 (B=4, d_v=512, d_k=64, k=8, 64 float16 "
                    "archived states): the retriever's stack + widen + gather + apply vs DeviceSegmentArchive",
            "reference_style_ms": round(c4["reference_style_ms"], 4),
            "device_archive_ms": round(c4["device_archive_ms"], 4),
            "speedup": round(c4["reference_style_ms"] / c4["device_archive_ms"], 2)}
        log(f"c4 segment retrieval: reference style {c4['reference_style_ms']:.3f} ms, device archive "
            f"{c4['device_archive_ms']:.3f} ms")

    if not a.no_gather or a.c4_only:
        settle(torch)
        log("config 4 end-to-end forward (4 layers, 4 x 8192 tokens)")
        m4 = bench_c4_model(torch, dev, a.steps, sec_w)
        secondary["c4_model_forward"] = {
            "what": "config 4 LM forward, bf16 weights, random init: Embedding -> 4 x SegmentRecurrentMemoryLayer "
                    "(hidden 512, d_k 64, segment 64, capacity 64, top-8, float16 archive) -> Linear(512, 32000); "
                    "whole-sequence launches per layer, archive reset each forward",
            "ms": round(m4["ms"], 3), "tokens/s": round(m4["tokens"] / m4["ms"] * 1e3),
            "breakdown_ms": {k: round(v, 3) for k, v in sorted(m4["phases_ms"].items(), key=lambda kv: -kv[1])},
            "breakdown_note": "one extra forward with events at the phase boundaries, summed over the 4 layers"}
        log(f"c4 forward: {m4['ms']:.2f} ms, {m4['tokens'] / m4['ms'] * 1e3:.3e} tokens/s")
        for k, v in sorted(m4["phases_ms"].items(), key=lambda kv: -kv[1]):
            log(f"  c4 phase {k}: {v:.3f} ms")

    if not a.no_gather or a.train_only:
        settle(torch)
        log("config 4 training forward + backward")
        t4 = bench_c4_train(torch, dev, a.steps, sec_w)
        secondary["c4_model_train_step"] = {
            "what": "config 4 LM forward + cross-entropy + backward (no optimizer step), same model and ids; "
                    "native scan backward, routing, and retrieval + LayerNorm residual as one autograd function "
                    "whose backward never forms the gathered states or the per-route rows",
            "ms": round(t4["ms"], 3), "tokens/s": round(t4["tokens"] / t4["ms"] * 1e3),
            "generic_path_calls": t4["generic_path_calls"], "peak_memory_gib": round(t4["peak_gib"], 1)}
        log(f"c4 train step: {t4['ms']:.2f} ms, {t4['tokens'] / t4['ms'] * 1e3:.3e} tokens/s, generic path calls "
            f"{t4['generic_path_calls']}, peak {t4['peak_gib']:.1f} GiB")

    if not a.no_gather:
        pub = bench_published(torch, dev)
        secondary["published_microbench"] = pub
        log(f"published microbench shape: native {pub['native_ms']:.4f} ms (published 0.219), fallback "
            f"{pub['fallback_ms']:.4f} ms (published 0.724)")

    cpu = None
    if not a.no_cpu:
        log("cpu baseline (torch-CPU port: north-star shape, configs 1 and 2 full, configs 3 and 5 slices)")
        cpu = cpu_baseline(torch)
        log(f"cpu: {cpu['value']:.3e} tokens/s on {cpu['cores']} threads ({cpu['host']}); one thread "
            f"{cpu['one_thread']['n1']['tokens/s']:.3e}")

    line = {
        "metric": METRIC,
        "value": tokens / t_step,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": t_step * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q,k,v with q,k L2-normalised, state N(0,0.02))",
        "config": {"workload": "north-star shape (BASELINE north_star): fused chunk-update + query, B=8 x H=8 = 64 "
                               "sequences x 8192 tokens, d_k=d_v=128, chunk 64, bf16 q/k/v, fp32 state, 128 "
                               "snapshots per sequence",
                   "global_batch": 64, "seq_len": 8192, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved_gbs / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_note": traffic_note,
                     "kernel": "scan_vsplit_kernel<BF16,128,4>: the one launch of a grm_hip_chunk_update_fwd call",
                     "algorithmic_bytes_per_launch": bytes_,
                     "kernel_us": round(t_kernel * 1e6, 2),
                     "copy_ceiling": {"what": "a device copy of the same byte count (half read, half written) "
                                              "right after the timed launches, events around the same number of "
                                              "copies",
                                      "us": round(n1["copy_us"], 2),
                                      "GB/s": round(n1["copy_bytes"] / n1["copy_us"] / 1e3, 1),
                                      "kernel_time_vs_copy": round(n1["copy_us"] / (t_kernel * 1e6), 4)},
                     "mfma": {"TFLOP/s": round(tflops, 2), "peak": BF16_PEAK_TFLOPS,
                              "frac": round(tflops / BF16_PEAK_TFLOPS, 5), "flops_per_launch": flops}},
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
