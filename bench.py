#!/usr/bin/env python3
"""Benchmark of the MI355X sparse flash attention path.

One step = one pass of the hot path over one batch of synthetic input.  The
headline (``value``) is the DeepSeek-V3.2-style MLA prefill forward:
B=1, S=32768, Hq=128, one latent KV head, d_qk=576, d_v=512 (V = first 512
dims of K), top-k=2048, bf16, reported as effective TFLOP/s over the valid
top-k pairs (2·(d_qk+d_v) FLOP per head per pair).  The other workloads are
measured in the same run and reported under ``workloads``:

* ``prefill``     MQA fwd, S=4096, Hq=16, d=128, top-k 512        (TFLOP/s)
* ``train_gqa``   GQA fwd + bwd (deterministic and atomic dK/dV), B=2, S=8192,
                  Hq=32, Hkv=2, top-k 1024
* ``mla_decode``  B=64 x 1 query, KV [64, 65536, 1, 576], top-k 2048, split-k
                  + combine, caches flushed (by a 1 GiB read) before every step (GB/s);
                  ``paged``: the same cache as a 64-row-page pool (4.8 GB, pages
                  shuffled) read through a block table
* ``indexer``     top-k index producer for the prefill: S=32768 causal queries,
                  64 index heads, d=128, top-k 2048 (scores + selection; TFLOP/s
                  over the visible (query, key) pairs, 2 H d FLOP each);
                  ``layer_ms``: indexer + MLA forward on the indices it produced
                  (the whole sparse attention layer of the prefill)
* ``mla_bwd``     shared-KV (MLA) backward at the full prefill shape (S=32768,
                  128 heads, d_qk 576 / d_v 512, top-k 2048; TFLOP/s over valid
                  pairs): dQ and the merged dK + dV of the shared rows
* ``shim``        the reference's own signature (SBHD q, one shared kv, sink):
                  S=4096, H=64, D=128, top-k 2048, fwd and bwd

Inputs are resident in HBM before timing.  Timing uses HIP events on the
stream the kernels run on (torch's current stream).  ``cpu_baseline`` times
the CPU oracle (PyTorch eager, fp32) on a bounded sample of the same
workload on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA: 256 CU x 4096 FLOP/clk x 2.4 GHz
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
# vector L1 / texture path: one 64-byte line per clock per CU, 256 CUs at 2.4 GHz
PEAK_TEX_GBS = 256 * 64 * 2.4


def texture(gather_gbs):
    """The d = 128 kernels' binding resource: the gathered K / V row bytes
    against the texture path's nominal rate (their counters show TD 0.87-0.94
    busy while MFMA is 0.1-0.4 busy)."""
    return {"gather_gbs": gather_gbs, "peak_gbs": PEAK_TEX_GBS, "frac": gather_gbs / PEAK_TEX_GBS,
            "bytes_per_cu_clk_at_2p4ghz": gather_gbs * 1e9 / (256 * 2.4e9)}
METRIC = "SFA fwd/bwd effective TFLOP/s (top-k FLOPs) + decode gather GB/s, % roofline"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def valid_pairs(w):
    import torch
    idx = w.idx.long()
    bound = w.kv_lens.long().view(-1, 1, 1, 1) if w.kv_lens is not None else w.k.shape[1]
    return int(((idx >= 0) & (idx < bound)).sum().item())


def fwd_flops(w, pairs):
    G = w.q.shape[2] // w.k.shape[2]
    return pairs * G * 2.0 * (w.q.shape[3] + w.v.shape[3])


def bwd_flops(w, pairs):
    G = w.q.shape[2] // w.k.shape[2]
    return pairs * G * 2.0 * (3 * w.q.shape[3] + 2 * w.v.shape[3])


def gathered_bytes(w, pairs):
    """K and V rows read per valid pair (one read per pair serves the G
    query heads); with G = 16 and d = 128 this stream, served mostly from
    L2 / MALL, rather than the MFMA rate bounds the d = 128 kernels."""
    return pairs * (w.q.shape[3] + w.v.shape[3]) * w.q.element_size()


def decode_bytes(w, pairs):
    """Algorithmic bytes of a decode step: the gathered K rows (V is their
    prefix) + q + out + lse + idx."""
    B, _, Hq, Dqk = w.q.shape
    Dv = w.v.shape[3]
    return pairs * Dqk * 2 + w.q.numel() * 2 + B * Hq * Dv * 2 + B * Hq * 4 + w.idx.numel() * 4


def time_steps(fn, steps, warmup, before=None):
    """Per-step HIP-event durations (ms) on the current stream."""
    import torch
    for _ in range(warmup):
        if before:
            before()
        fn()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        if before:
            before()
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    return [s.elapsed_time(e) for s, e in zip(starts, ends)], wall


def cpu_model():
    """The host CPU as /proc/cpuinfo names it: model name, family / model /
    stepping numbers (a virtualised host may shorten the name) and the
    logical CPU count of the host."""
    fields, n = {}, 0
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k = k.strip()
                if k == "processor":
                    n += 1
                elif k in ("model name", "cpu family", "model", "stepping") and k not in fields:
                    fields[k] = v.strip()
    except OSError:
        pass
    if not fields:
        import platform
        return platform.processor() or "unknown"
    return (f"{fields.get('model name', '?')} (family {fields.get('cpu family', '?')}, model "
            f"{fields.get('model', '?')}, stepping {fields.get('stepping', '?')}; {n} logical CPUs on the host)")


def _cpu_threads():
    import torch
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    return cores


def _cpu_copy(w, rows=None):
    """CPU copies of a workload's tensors, optionally only query rows ``rows``
    (a slice of dim 1) of q / idx / dout."""
    sl = slice(None) if rows is None else rows
    cp = lambda t: None if t is None else t[:, sl].cpu() if t.dim() == 4 else t.cpu()
    return dict(q=cp(w.q), k=w.k.cpu(), idx=cp(w.idx), dout=cp(w.dout),
                kv_lens=None if w.kv_lens is None else w.kv_lens.cpu())


def cpu_baseline_mla(w, seconds):
    """Oracle forward on a strided sample of query rows, until ~``seconds`` of
    CPU work; the rate (valid-pair TFLOP/s) extrapolates to the full step."""
    from oracle.sfa_oracle import sfa_forward
    cores = _cpu_threads()
    k = w.k.cpu()
    v = k[..., : w.v.shape[3]]
    S = w.q.shape[1]
    chunk = 16
    starts = list(range(S - chunk, 0, -max(chunk, S // 256)))  # late (full top-k) rows first
    done_pairs, elapsed, nrows = 0, 0.0, 0
    for s0 in starts:
        q = w.q[:, s0:s0 + chunk].cpu()
        idx = w.idx[:, s0:s0 + chunk].cpu()
        t0 = time.perf_counter()
        sfa_forward(q, k, v, idx, w.scale)
        elapsed += time.perf_counter() - t0
        done_pairs += int((idx >= 0).sum())
        nrows += chunk
        if elapsed >= seconds:
            break
    flops = fwd_flops(w, done_pairs)
    rate = flops / elapsed / 1e12
    return {"value": rate, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"oracle fp32 fwd on {nrows} query rows ({done_pairs} valid pairs) of the mla_prefill "
                      f"workload, {elapsed:.1f} s; sfa_forward chunks of {chunk} rows",
            "extrapolated_step_s": fwd_flops(w, valid_pairs(w)) / (rate * 1e12)}


def cpu_fwd_bwd(w, rows=None, bwd=True):
    """Oracle forward (+ backward) on query rows ``rows`` of workload ``w``
    (all rows if None); returns seconds and the valid pairs covered."""
    from oracle.sfa_oracle import sfa_backward, sfa_forward
    c = _cpu_copy(w, rows)
    k = c["k"]
    v = k[..., : w.v.shape[3]] if w.v.data_ptr() == w.k.data_ptr() else w.v.cpu()
    t0 = time.perf_counter()
    out, lse = sfa_forward(c["q"], k, v, c["idx"], w.scale, kv_lens=c["kv_lens"])
    t_fwd = time.perf_counter() - t0
    t_bwd = None
    if bwd:
        t0 = time.perf_counter()
        sfa_backward(c["q"], k, v, c["idx"], out, lse, c["dout"], w.scale, kv_lens=c["kv_lens"])
        t_bwd = time.perf_counter() - t0
    bound = c["kv_lens"].long().view(-1, 1, 1, 1) if c["kv_lens"] is not None else k.shape[1]
    pairs = int(((c["idx"] >= 0) & (c["idx"].long() < bound)).sum())
    return t_fwd, t_bwd, pairs


# per-workload CPU rates wait until every GPU timing is done: the oracle's
# threads busy the host cores, and a launching thread that loses its core
# for a few ms in a timed step moves a short step's mean (the decode step)
_CPU_PENDING = []


def cpu_rate(name, w):
    """CPU (oracle, PyTorch eager fp32) rate of workload ``name`` on this
    host's cores: full runs where they take seconds, a bounded sample of query
    rows otherwise (the rate is per valid pair, so it extrapolates)."""
    _cpu_threads()
    if name == "tiny":
        tf, tb, pairs = cpu_fwd_bwd(w)
        return {"value": (fwd_flops(w, pairs) + bwd_flops(w, pairs)) / (tf + tb) / 1e12, "unit": "TFLOP/s",
                "fwd_s": tf, "bwd_s": tb, "sample": "full fwd+bwd (B=1, S=256, Hq=4, d=64, top-k 64, fp32)"}
    if name == "prefill":
        tf, _, pairs = cpu_fwd_bwd(w, bwd=False)
        return {"value": fwd_flops(w, pairs) / tf / 1e12, "unit": "TFLOP/s", "fwd_s": tf,
                "sample": "full fwd (B=1, S=4096, Hq=16, d=128, top-k 512)"}
    if name == "train_gqa":
        S = w.q.shape[1]
        r0 = S - 512
        tf, tb, pairs = cpu_fwd_bwd(w, rows=slice(r0, S))
        full = valid_pairs(w)
        rate_f, rate_b = fwd_flops(w, pairs) / tf / 1e12, bwd_flops(w, pairs) / tb / 1e12
        return {"value": (fwd_flops(w, pairs) + bwd_flops(w, pairs)) / (tf + tb) / 1e12, "unit": "TFLOP/s",
                "fwd_tflops": rate_f, "bwd_tflops": rate_b, "fwd_s": tf, "bwd_s": tb,
                "extrapolated_step_s": fwd_flops(w, full) / (rate_f * 1e12) + bwd_flops(w, full) / (rate_b * 1e12),
                "sample": f"fwd+bwd on query rows {r0}..{S - 1} of both sequences ({pairs} valid pairs, full "
                          f"top-k); rate per valid pair, extrapolated to the full step"}
    if name == "mla_decode":
        tf, _, pairs = cpu_fwd_bwd(w, bwd=False)
        return {"value": decode_bytes(w, pairs) / tf / 1e9, "unit": "GB/s", "tflops": fwd_flops(w, pairs) / tf / 1e12,
                "fwd_s": tf, "sample": "full decode step (64 sequences x 128 heads, top-k 2048)"}
    raise KeyError(name)


def bench_mla_prefill(args):
    import torch
    import ops_amd
    from ops_amd.workloads import make_workload
    log("generating mla_prefill workload (S=32768, Hq=128, top-k 2048)")
    w = make_workload("mla_prefill", device="cuda")
    pairs = valid_pairs(w)
    flops = fwd_flops(w, pairs)
    out = torch.empty(w.q.shape[:3] + (w.v.shape[3],), dtype=w.q.dtype, device="cuda")
    lse = torch.empty(w.q.shape[:3], dtype=torch.float32, device="cuda")
    fn = lambda: ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale, out=out, lse=lse)
    log("timing mla_prefill")
    times, wall = time_steps(fn, args.steps, args.warmup)
    ms = sum(times) / len(times)
    achieved = flops / (ms * 1e-3) / 1e12
    res = {
        "ms_per_step": wall / args.steps,
        "kernel_ms": ms,
        "value": flops / (wall / args.steps * 1e-3) / 1e12,
        "achieved_tflops": achieved,
        "valid_pairs": pairs,
        "flops_per_step": flops,
    }
    # the same forward on rows already in ascending order, declared so
    # (SFA_FWD_IDX_SORTED: what rows of the index producer take): no sort pass
    big = torch.iinfo(torch.int32).max
    srt = torch.sort(torch.where(w.idx >= 0, w.idx, torch.full_like(w.idx, big)), dim=-1).values
    srt = torch.where(srt == big, torch.full_like(srt, -1), srt)
    st, _ = time_steps(lambda: ops_amd.sfa_forward(w.q, w.k, w.v, srt, w.scale, out=out, lse=lse, idx_sorted=True),
                       max(2, args.steps // 2), 2)
    res["presorted_ms"] = sum(st) / len(st)
    del srt
    return w, res


def bench_tiny(args):
    """Config 1 (fp32, generic kernels): fwd + bwd TFLOP/s."""
    import ops_amd
    from ops_amd.workloads import make_workload
    w = make_workload("tiny", device="cuda")
    pairs = valid_pairs(w)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
    ft, _ = time_steps(lambda: ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale), args.steps * 4, args.warmup)
    bt, _ = time_steps(lambda: ops_amd.sfa_backward(w.q, w.k, w.v, w.idx, out, lse, w.dout, w.scale),
                       args.steps * 4, args.warmup)
    fms, bms = sum(ft) / len(ft), sum(bt) / len(bt)
    res = {"metric": "fwd+bwd effective TFLOP/s", "value": (fwd_flops(w, pairs) + bwd_flops(w, pairs)) /
           ((fms + bms) * 1e-3) / 1e12, "unit": "TFLOP/s", "fwd_ms": fms, "bwd_ms": bms, "valid_pairs": pairs,
           "dtype": "f32", "config": {"B": 1, "S": 256, "Hq": 4, "Hkv": 1, "d": 64, "topk": 64}}
    if not args.no_cpu:
        _CPU_PENDING.append((res, "tiny", w))
    return res


def bench_prefill(args):
    import ops_amd
    from ops_amd.workloads import make_workload
    w = make_workload("prefill", device="cuda")
    pairs = valid_pairs(w)
    flops = fwd_flops(w, pairs)
    times, _ = time_steps(lambda: ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale), args.steps * 4, args.warmup)
    ms = sum(times) / len(times)
    tf = flops / (ms * 1e-3) / 1e12
    res = {"metric": "fwd effective TFLOP/s", "value": tf, "unit": "TFLOP/s", "ms": ms, "valid_pairs": pairs,
           "frac_of_peak": tf / PEAK_BF16_TFLOPS, "gather_gbs": gathered_bytes(w, pairs) / (ms * 1e-3) / 1e9,
           "config": {"B": 1, "S": 4096, "Hq": 16, "Hkv": 1, "d": 128, "topk": 512}}
    res["texture"] = texture(res["gather_gbs"])
    if not args.no_cpu:
        _CPU_PENDING.append((res, "prefill", w))
    return res


def bench_train_gqa(args):
    import ops_amd
    from ops_amd.workloads import make_workload
    w = make_workload("train_gqa", device="cuda")
    pairs = valid_pairs(w)
    ff = fwd_flops(w, pairs)
    times, _ = time_steps(lambda: ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale), args.steps, args.warmup)
    ms = sum(times) / len(times)
    res = {"metric": "fwd effective TFLOP/s", "value": ff / (ms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms": ms,
           "valid_pairs": pairs, "hot_share": w.meta.get("hot_share"),
           "gather_gbs": gathered_bytes(w, pairs) / (ms * 1e-3) / 1e9,
           "config": {"B": 2, "S": 8192, "Hq": 32, "Hkv": 2, "d": 128, "topk": 1024}}
    res["frac_of_peak"] = res["value"] / PEAK_BF16_TFLOPS
    res["texture"] = texture(res["gather_gbs"])
    if not args.no_bwd:
        out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
        bf = bwd_flops(w, pairs)
        res["bwd"] = {}
        for mode in ("csr", "atomic"):
            bt, _ = time_steps(lambda: ops_amd.sfa_backward(w.q, w.k, w.v, w.idx, out, lse, w.dout, w.scale,
                                                            dkv_mode=mode), max(1, args.steps // 2), 1)
            bms = sum(bt) / len(bt)
            res["bwd"][mode] = {"value": bf / (bms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms": bms,
                                "frac_of_peak": bf / (bms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS}
            if mode == "csr":
                # the dQ pass re-gathers the K and V rows of every pair (bwd_dq_kernel)
                res["bwd"][mode]["dq_pass_gather_bytes"] = gathered_bytes(w, pairs)
        res["bwd"]["note"] = ("TFLOP/s over valid pairs (pairs * G * 2 (3 d_qk + 2 d_v)); 'csr' = deterministic "
                              "dK/dV (the default), 'atomic' = fp32 atomics")
    if not args.no_cpu:
        _CPU_PENDING.append((res, "train_gqa", w))
    return res


def decode_flush():
    """A 1 GiB buffer whose READ before every step evicts the KV rows from the
    256 MB Infinity Cache and L2 without leaving dirty lines behind (a
    write-flush makes the next kernel pay for write-backs it did not cause)."""
    import torch
    flush = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
    return lambda: flush.sum()


def prepared_forward(w, out, lse):
    """One sfa_fwd call through the C ABI with its argument struct and
    workspace built once: the host work between a step's start event and the
    kernel launch is a single ctypes call, so a host stall there is unlikely
    to stretch a 60 us step (the GPU is still busy with the cache flush
    queued before it).  Same arguments as ops_amd.sfa_forward."""
    import ctypes
    import torch
    from ops_amd import _lib, sfa
    lib = _lib.load()
    q, k, v, idx, kv_lens, _ = sfa._prep(w.q, w.k, w.v, w.idx, w.kv_lens, None)
    a = sfa._fwd_args(q, k, v, idx, out, lse, w.scale, kv_lens, None, 0)
    ws = lib.sfa_fwd_workspace_size(ctypes.byref(a))
    wbuf = torch.empty(max(ws, 1), dtype=torch.uint8, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ref = ctypes.byref(a)
    wptr = ctypes.c_void_p(wbuf.data_ptr())

    def fn():
        _lib.check(lib.sfa_fwd(ref, wptr, ws, stream))

    fn.keep = (q, k, v, idx, kv_lens, a, wbuf)  # (the tensors the struct points to stay alive)
    return fn


def bench_mla_decode(args):
    import torch
    import ops_amd
    from ops_amd.workloads import make_workload
    w = make_workload("mla_decode", device="cuda")
    pairs = valid_pairs(w)
    B, _, Hq, Dqk = w.q.shape
    Dv = w.v.shape[3]
    nbytes = decode_bytes(w, pairs)
    flush = decode_flush()
    out = torch.empty((B, 1, Hq, Dv), dtype=w.q.dtype, device="cuda")
    lse = torch.empty((B, 1, Hq), dtype=torch.float32, device="cuda")
    fn = prepared_forward(w, out, lse)
    times, _ = time_steps(fn, args.steps * 4, args.warmup, before=flush)
    us = sum(times) / len(times) * 1e3
    gbs = nbytes / (us * 1e-6) / 1e9
    # "us" is the mean over the timed steps; the median and the slowest step
    # beside it show whether one stalled step moved the mean
    res = {"metric": "decode GB/s (algorithmic bytes, cache flushed)", "value": gbs, "unit": "GB/s", "us": us,
           "us_median": statistics.median(times) * 1e3, "us_max": max(times) * 1e3, "bytes": nbytes,
           "frac_of_peak": gbs / PEAK_HBM_GBS, "tflops": fwd_flops(w, pairs) / (us * 1e-6) / 1e12,
           "config": {"B": 64, "Skv": 65536, "Hq": 128, "d_qk": 576, "d_v": 512, "topk": 2048}}
    # the same step over a paged cache (block table of 64-row pages)
    from ops_amd.workloads import page_kv
    kp, vp, bt = page_kv(w.k, w.v, 64, seed=1)
    pbytes = nbytes + pairs * 4  # one block-table entry per valid slot
    fnp = lambda: ops_amd.sfa_forward_paged(w.q, kp, vp, bt, w.idx, w.scale, kv_lens=w.kv_lens, out=out, lse=lse)
    times, _ = time_steps(fnp, args.steps * 4, args.warmup, before=flush)
    pus = sum(times) / len(times) * 1e3
    res["paged"] = {"value": pbytes / (pus * 1e-6) / 1e9, "unit": "GB/s", "us": pus,
                    "us_median": statistics.median(times) * 1e3, "us_max": max(times) * 1e3, "bytes": pbytes,
                    "frac_of_peak": pbytes / (pus * 1e-6) / 1e9 / PEAK_HBM_GBS, "page_size": 64,
                    "pool_bytes": kp.numel() * kp.element_size()}
    del kp, vp
    # a decode step's sparse-attention layer: the index producer over the
    # same contexts (64 index heads, d = 128, bf16), then this decode on the
    # index rows it produced
    qi, ki, wi, lens = indexer_inputs("decode")
    assert torch.equal(lens, w.kv_lens)

    def layer():
        idx = ops_amd.indexer_topk(qi, ki, wi, w.idx.shape[-1], kv_lens=lens)
        ops_amd.sfa_forward(w.q, w.k, w.v, idx, w.scale, kv_lens=w.kv_lens, out=out, lse=lse)

    times, _ = time_steps(layer, args.steps * 2, args.warmup, before=flush)
    res["layer_us"] = sum(times) / len(times) * 1e3
    res["layer_note"] = "index producer (64 heads, d 128, bf16 keys) + this decode on its rows, caches flushed"
    del qi, ki, wi
    if not args.no_cpu:
        _CPU_PENDING.append((res, "mla_decode", w))
    return res


def bench_mla_bwd(args):
    """Shared-KV (MLA) backward at the full prefill shape (S = 32768, 128
    heads, d_qk 576 / d_v 512, top-k 2048): dQ and the gradient of the shared
    rows (dK + dV, as the reference sums them, SFA.py:849-853) on the MFMA
    path; TFLOP/s over valid pairs, pairs * G * 2 (3 d_qk + 2 d_v)."""
    import ops_amd
    from ops_amd.workloads import make_workload
    w = make_workload("mla_prefill", device="cuda", with_dout=True)
    pairs = valid_pairs(w)
    out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
    res = {"metric": "bwd effective TFLOP/s", "valid_pairs": pairs, "unit": "TFLOP/s",
           "config": {"B": 1, "S": 32768, "Hq": 128, "Hkv": 1, "d_qk": 576, "d_v": 512, "topk": 2048}}
    for mode in ("auto", "atomic"):
        fn = lambda: ops_amd.sfa_backward(w.q, w.k, w.v, w.idx, out, lse, w.dout, w.scale, merge_kv=True,
                                          dkv_mode=mode)
        bt, _ = time_steps(fn, max(2, args.steps // 4), 1)
        ms = sum(bt) / len(bt)
        tf = bwd_flops(w, pairs) / (ms * 1e-3) / 1e12
        if mode == "auto":
            res.update({"value": tf, "ms": ms, "frac_of_peak": tf / PEAK_BF16_TFLOPS,
                        "kernels": "mla_map_kernel + mla_bwd_dq_kernel + mla_bwd_dkv_kernel<true> + "
                                   "mla_bwd_reduce_kernel (deterministic: per-slot bf16 rows summed per key "
                                   "in query order)"})
        else:
            res["atomic"] = {"value": tf, "ms": ms, "frac_of_peak": tf / PEAK_BF16_TFLOPS,
                             "kernels": "mla_bwd_dq_kernel + mla_bwd_dkv_kernel<false> (fp32 atomic adds of "
                                        "every slot's row, SFA.py:853's scheme)"}
    return res


def bench_shim(args):
    """The reference's own operator signature and shape class:
    ``SparseFlashAttentionTriton.apply(q [S, B, H, D], kv [S_kv, B, D],
    attn_sink [H], topk_idxs [S, B, K], sm_scale)`` (SFA.py:69-164) with one
    kv row serving as K and V, at S = 4096, B = 1, H = 64, D = 128, top-k 2048
    (the query, the 255 before it and uniform draws from the rest of the
    causal prefix), bf16, a sink: forward, then backward (dQ, kv's gradient
    dK + dV, dsink) through the shim's strided views.  G = 64 query heads per
    kv row: the d = 128 MFMA kernels in head groups of 16, the deterministic
    dK/dV."""
    import torch
    import ops_amd
    from ops_amd.workloads import make_workload
    w = make_workload("prefill", device="cuda", S=4096, Hq=64, K=2048, with_dout=True)
    q = w.q.permute(1, 0, 2, 3).detach().requires_grad_(True)   # [S, B, H, D]
    kv = w.k[:, :, 0].permute(1, 0, 2).detach().requires_grad_(True)  # [S_kv, B, D]
    idx = w.idx[:, :, 0].permute(1, 0, 2)                          # [S, B, K]
    sink = torch.linspace(-1.0, 1.0, 64, device="cuda").requires_grad_(True)
    dout = w.dout.permute(1, 0, 2, 3)
    pairs = valid_pairs(w)
    G = 64
    ff = pairs * G * 2.0 * (128 + 128)
    bf = pairs * G * 2.0 * (3 * 128 + 2 * 128)
    with torch.no_grad():
        ft, _ = time_steps(lambda: ops_amd.SparseFlashAttentionTriton.apply(q, kv, sink, idx, w.scale),
                           args.steps, args.warmup)
    out = ops_amd.SparseFlashAttentionTriton.apply(q, kv, sink, idx, w.scale)
    bt, _ = time_steps(lambda: torch.autograd.grad(out, (q, kv, sink), dout, retain_graph=True),
                       max(2, args.steps // 2), 1)
    fms, bms = sum(ft) / len(ft), sum(bt) / len(bt)
    return {"metric": "fwd / bwd effective TFLOP/s (reference signature)", "value": ff / (fms * 1e-3) / 1e12,
            "unit": "TFLOP/s", "fwd_ms": fms, "frac_of_peak": ff / (fms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
            "gather_gbs": pairs * 2 * 128 * 2 * 4 / (fms * 1e-3) / 1e9,
            "texture": texture(pairs * 2 * 128 * 2 * 4 / (fms * 1e-3) / 1e9),
            "bwd": {"value": bf / (bms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms": bms,
                    "frac_of_peak": bf / (bms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS},
            "valid_pairs": pairs,
            "note": "gather_gbs: K and V row bytes per valid pair and 16-head group (4 groups re-gather a row)",
            "config": {"api": "SparseFlashAttentionTriton.apply (SBHD, shared kv, sink)", "B": 1, "S": 4096,
                       "H": 64, "D": 128, "topk": 2048}}


def indexer_inputs(kind):
    """Index-producer inputs (64 index heads, d = 128, bf16 q / k, fp32
    weights): "prefill" = one causal sequence of 32768 queries over its own
    keys; "decode" = one query for each of 64 sequences over a 65536-key
    cache whose lengths are the decode workload's (16K-64K)."""
    import torch
    H = 64
    if kind == "prefill":
        B, Sq, Skv, kv_lens = 1, 32768, 32768, None
    else:
        from ops_amd.workloads import decode_context_lens
        B, Sq, Skv = 64, 1, 65536
        kv_lens = decode_context_lens(device="cuda")
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    q = torch.randn(B, Sq, H, 128, generator=g, device="cuda").bfloat16()
    k = torch.randn(B, Skv, 128, generator=g, device="cuda").bfloat16()
    w = torch.randn(B, Sq, H, generator=g, device="cuda") / math.sqrt(H)
    return q, k, w, kv_lens


def bench_indexer(args, mla=None):
    import torch
    import ops_amd
    B, S, H, K = 1, 32768, 64, 2048
    q, k, w, _ = indexer_inputs("prefill")
    fn = lambda: ops_amd.indexer_topk(q, k, w, K)
    times, _ = time_steps(fn, max(2, args.steps // 2), 1)
    ms = sum(times) / len(times)
    flops = S * (S + 1) // 2 * H * 128 * 2.0
    tf = flops / (ms * 1e-3) / 1e12
    res = {"metric": "indexer scores + top-k, effective TFLOP/s (visible pairs)", "value": tf, "unit": "TFLOP/s",
           "ms": ms, "frac_of_peak": tf / PEAK_BF16_TFLOPS,
           "config": {"B": B, "S": S, "H_index": H, "d_index": 128, "topk": K, "causal": True}}
    # the same scores from fp8 e4m3 q / k (per-token k scales, q scales
    # folded into the weights), as DeepSeek-V3.2 stores the indexer inputs
    f8 = torch.float8_e4m3fn
    ks = k.float().abs().amax(-1).clamp_min(1e-6) / 448.0
    k8 = (k.float() / ks[..., None]).to(f8)
    qs = q.float().abs().amax(-1).clamp_min(1e-6) / 448.0
    q8 = (q.float() / qs[..., None]).to(f8)
    w8 = (w * qs).contiguous()
    ft, _ = time_steps(lambda: ops_amd.indexer_topk(q8, k8, w8, K, k_scale=ks), max(2, args.steps // 2), 1)
    fms = sum(ft) / len(ft)
    res["fp8"] = {"value": flops / (fms * 1e-3) / 1e12, "unit": "TFLOP/s", "ms": fms,
                  "note": "fp8 e4m3 q / k, per-token k scales; TFLOP/s over the same visible pairs"}
    del q8, k8
    # a decode step's index rows: one query for each of 64 sequences over
    # 16K-64K keys (HBM-bound: every visible key row is read once)
    qd, kd, wd, lens = indexer_inputs("decode")
    dt, _ = time_steps(lambda: ops_amd.indexer_topk(qd, kd, wd, K, kv_lens=lens), max(5, args.steps), 2,
                       before=decode_flush())
    dms = sum(dt) / len(dt)
    key_bytes = int(lens.sum()) * 128 * 2
    res["decode"] = {"ms": dms, "key_gbs": key_bytes / (dms * 1e-3) / 1e9,
                     "frac_of_hbm": key_bytes / (dms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                     "note": "key rows read (bf16, 256 B per visible key) per second; caches flushed per step",
                     "config": {"B": 64, "Sq": 1, "Skv": 65536, "kv_lens": "16384-65536", "H_index": 64,
                                "d_index": 128, "topk": K}}
    # the same step from fp8 index keys (128 B per key row)
    ksd = kd.float().abs().amax(-1).clamp_min(1e-6) / 448.0
    kd8 = (kd.float() / ksd[..., None]).to(f8)
    qsd = qd.float().abs().amax(-1).clamp_min(1e-6) / 448.0
    qd8 = (qd.float() / qsd[..., None]).to(f8)
    wd8 = (wd * qsd).contiguous()
    dt8, _ = time_steps(lambda: ops_amd.indexer_topk(qd8, kd8, wd8, K, kv_lens=lens, k_scale=ksd), max(5, args.steps),
                        2, before=decode_flush())
    d8 = sum(dt8) / len(dt8)
    res["decode"]["fp8"] = {"ms": d8, "key_gbs": key_bytes / 2 / (d8 * 1e-3) / 1e9,
                            "frac_of_hbm": key_bytes / 2 / (d8 * 1e-3) / 1e9 / PEAK_HBM_GBS}
    del qd, kd, wd, qd8, kd8, wd8
    if mla is not None:
        out = torch.empty(mla.q.shape[:3] + (mla.v.shape[3],), dtype=mla.q.dtype, device="cuda")
        lse = torch.empty(mla.q.shape[:3], dtype=torch.float32, device="cuda")

        def layer():
            # (the producer writes ascending rows: no sort pass before the forward)
            idx = ops_amd.indexer_topk(q, k, w, K)
            ops_amd.sfa_forward(mla.q, mla.k, mla.v, idx, mla.scale, out=out, lse=lse, idx_sorted=True)

        lt, _ = time_steps(layer, max(2, args.steps // 2), 1)
        res["layer_ms"] = sum(lt) / len(lt)
    return res


def profile_targets(name):
    """(fn, before) of one workload's kernels, for counter runs that time
    nothing: ``python bench.py --profile NAME --steps N`` launches fn N times
    (before() ahead of each, e.g. the decode cache flush)."""
    import torch
    import ops_amd
    from ops_amd.workloads import make_workload, page_kv
    if name == "mla_prefill":
        w = make_workload("mla_prefill", device="cuda")
        return lambda: ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale), None
    if name == "prefill":
        w = make_workload("prefill", device="cuda")
        return lambda: ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale), None
    if name in ("train_gqa_fwd", "train_gqa_bwd_csr", "train_gqa_bwd_atomic"):
        w = make_workload("train_gqa", device="cuda")
        if name == "train_gqa_fwd":
            return lambda: ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale), None
        out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
        mode = name.rsplit("_", 1)[1]
        return lambda: ops_amd.sfa_backward(w.q, w.k, w.v, w.idx, out, lse, w.dout, w.scale, dkv_mode=mode), None
    if name in ("mla_decode", "mla_decode_paged"):
        w = make_workload("mla_decode", device="cuda")
        flush = decode_flush()
        if name == "mla_decode":
            return lambda: ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale, kv_lens=w.kv_lens), flush
        kp, vp, bt = page_kv(w.k, w.v, 64, seed=1)
        return lambda: ops_amd.sfa_forward_paged(w.q, kp, vp, bt, w.idx, w.scale, kv_lens=w.kv_lens), flush
    if name == "mla_bwd":
        w = make_workload("mla_prefill", device="cuda", with_dout=True)
        out, lse = ops_amd.sfa_forward(w.q, w.k, w.v, w.idx, w.scale)
        return lambda: ops_amd.sfa_backward(w.q, w.k, w.v, w.idx, out, lse, w.dout, w.scale, merge_kv=True), None
    if name in ("shim_fwd", "shim_bwd"):
        # the reference-signature shape of bench_shim: S = 4096, H = 64 on one
        # kv row, D = 128, top-k 2048, a sink (SBHD views of the BSHD workload)
        w = make_workload("prefill", device="cuda", S=4096, Hq=64, K=2048, with_dout=True)
        q = w.q.permute(1, 0, 2, 3).contiguous()
        kv = w.k[:, :, 0].permute(1, 0, 2).contiguous()
        idx = w.idx[:, :, 0].permute(1, 0, 2).contiguous()
        sink = torch.linspace(-1.0, 1.0, q.shape[2], device="cuda")
        if name == "shim_fwd":
            return lambda: ops_amd.SparseFlashAttentionTriton.apply(q, kv, sink, idx, w.scale), None
        qg, kvg, sg = q.requires_grad_(True), kv.requires_grad_(True), sink.requires_grad_(True)
        out = ops_amd.SparseFlashAttentionTriton.apply(qg, kvg, sg, idx, w.scale)
        dout = w.dout.permute(1, 0, 2, 3).contiguous()
        return lambda: torch.autograd.grad(out, (qg, kvg, sg), dout, retain_graph=True), None
    if name in ("indexer_prefill", "indexer_decode"):
        q, k, w, kv_lens = indexer_inputs(name.split("_")[1])
        return lambda: ops_amd.indexer_topk(q, k, w, 2048, kv_lens=kv_lens), None
    raise SystemExit(f"unknown --profile target {name!r}")


def run_probe(name, args):
    """Hardware ceilings the design's decisions rest on, from committed code
    (one JSON line per measurement):
      gemm           the vendor bf16 GEMM (hipBLASLt via torch.matmul) on
                     N(0,1) operands at 4096^3, 8192^3, 16384^3: the dense
                     MFMA rate this power-limited part sustains;
      decode_gather  the 64 x 64K decode's data movement without its MFMA
                     work (libsfa_probe.so: the library's row gather, LDS
                     DMA, two 32-row tiles in flight, one barrier per tile),
                     caches flushed before each step as in the decode bench,
                     in the work layouts the decode design compares; the
                     same rows read into registers with as many loads in
                     flight as 1-32 waves per CU allow (no LDS, no tiles:
                     the ceiling of random 1152-byte rows on the part), a
                     contiguous read of the same bytes (the streaming
                     reference); the real decode step (prepared sfa_fwd
                     call) is timed beside them."""
    import ctypes
    import torch
    if name == "gemm":
        for n in (4096, 8192, 16384):
            g = torch.Generator(device="cuda").manual_seed(n)
            a = torch.randn(n, n, device="cuda", generator=g).bfloat16()
            b = torch.randn(n, n, device="cuda", generator=g).bfloat16()
            t, _ = time_steps(lambda: torch.matmul(a, b), max(3, args.steps), 2)
            ms = statistics.median(t)
            print(json.dumps({"probe": "gemm_bf16", "n": n, "ms": round(ms, 4),
                              "tflops": round(2 * n ** 3 / (ms * 1e-3) / 1e12, 1),
                              "frac_of_peak": round(2 * n ** 3 / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}),
                  flush=True)
            del a, b
        return
    if name != "decode_gather":
        raise SystemExit(f"unknown --probe {name!r} (gemm, decode_gather)")
    from ops_amd.workloads import make_workload
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ops_amd", "libsfa_probe.so")
    if not os.path.exists(path):
        raise SystemExit(f"{path} is not built: python -m ops_amd.build")
    lib = ctypes.CDLL(path)
    lib.sfa_probe_gather.restype = ctypes.c_int
    lib.sfa_probe_gather.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                     ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    w = make_workload("mla_decode", device="cuda")
    B, _, Hq, Dqk = w.q.shape
    Skv, K = w.k.shape[1], w.idx.shape[-1]
    assert w.k.is_contiguous() and w.q.is_contiguous() and w.k.shape[2] == 1 and Dqk == 576
    idx = w.idx.reshape(B, K).contiguous()
    gathered = valid_pairs(w) * Dqk * 2
    flush = decode_flush()
    part = torch.empty(B * 4 * 128 * 1024, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    qrow = Hq * Dqk * 2
    layouts = [  # (what, key splits, head groups, Q bytes per workgroup, partial rows per workgroup)
        ("4 key splits x 128 heads: gather only", 4, 1, 0, 0),
        ("4 key splits x 128 heads: gather + Q", 4, 1, qrow, 0),
        ("4 key splits x 128 heads: gather + Q + bf16 partial rows", 4, 1, qrow, 128),
        ("2 key splits x 2 groups of 64 heads: gather + Q + partial rows", 2, 2, qrow // 2, 64),
        ("1 split x 4 groups of 32 heads (no partials): gather + Q", 1, 4, qrow // 4, 0),
    ]
    for what, splits, hg, qb, rows in layouts:
        fn = lambda: lib.sfa_probe_gather(ctypes.c_void_p(w.k.data_ptr()), ctypes.c_void_p(w.q.data_ptr()), qrow,
                                          ctypes.c_void_p(idx.data_ptr()), ctypes.c_void_p(part.data_ptr()), B, Skv,
                                          K, splits, hg, qb, rows, ctypes.c_void_p(stream))
        rc = fn()
        if rc != 0:
            raise SystemExit(f"sfa_probe_gather failed: {rc}")
        t, _ = time_steps(fn, args.steps * 4, args.warmup, before=flush)
        us = sum(t) / len(t) * 1e3
        print(json.dumps({"probe": "decode_gather", "layout": what, "workgroups": B * splits * hg,
                          "us": round(us, 2), "us_median": round(statistics.median(t) * 1e3, 2),
                          "gathered_gbs": round(gathered * hg / (us * 1e-6) / 1e9, 1),
                          "algorithmic_gbs": round(gathered / (us * 1e-6) / 1e9, 1)}), flush=True)
    lib.sfa_probe_rowread.restype = ctypes.c_int
    lib.sfa_probe_rowread.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    sink = torch.empty(2048 * 256, dtype=torch.int32, device="cuda")
    for contiguous in (0, 1):
        for wgs in (256, 512, 1024, 2048):
            fn = lambda: lib.sfa_probe_rowread(ctypes.c_void_p(w.k.data_ptr()), ctypes.c_void_p(idx.data_ptr()),
                                               ctypes.c_void_p(sink.data_ptr()), B, Skv, K, wgs, contiguous,
                                               ctypes.c_void_p(stream))
            rc = fn()
            if rc != 0:
                raise SystemExit(f"sfa_probe_rowread failed: {rc}")
            t, _ = time_steps(fn, args.steps * 4, args.warmup, before=flush)
            us = sum(t) / len(t) * 1e3
            what = ("contiguous read of the same bytes" if contiguous else
                    "the rows into registers (ceiling: no LDS, no tiles)")
            print(json.dumps({"probe": "decode_gather", "layout": f"{what}, {wgs // 64} waves per CU",
                              "workgroups": wgs, "us": round(us, 2), "us_median": round(statistics.median(t) * 1e3, 2),
                              "algorithmic_gbs": round(gathered / (us * 1e-6) / 1e9, 1)}), flush=True)
    out = torch.empty((B, 1, Hq, w.v.shape[3]), dtype=w.q.dtype, device="cuda")
    lse = torch.empty((B, 1, Hq), dtype=torch.float32, device="cuda")
    fn = prepared_forward(w, out, lse)
    t, _ = time_steps(fn, args.steps * 4, args.warmup, before=flush)
    print(json.dumps({"probe": "decode_gather", "layout": "the decode step itself (sfa_fwd, 4 splits + combine)",
                      "us": round(sum(t) / len(t) * 1e3, 2), "us_median": round(statistics.median(t) * 1e3, 2)}),
          flush=True)


# Counter passes of the per-workload counter summaries (one rocprofv3 run
# each; every pass stays within one run's per-block counter limits).
PMC_PASSES = (
    "SQ_VALU_MFMA_BUSY_CYCLES SQ_WAVE_CYCLES SQ_WAIT_INST_ANY SQ_INSTS_MFMA SQ_INSTS_VALU SQ_INSTS_LDS "
    "SQ_INSTS_SALU SQ_INSTS_VMEM GRBM_GUI_ACTIVE GRBM_COUNT",
    "FETCH_SIZE TCC_HIT_sum TA_BUSY_avr TA_BUFFER_READ_LDS_WAVEFRONTS_sum TD_TD_BUSY_sum TD_TC_STALL_sum "
    "TCP_TCC_READ_REQ_LATENCY_sum TCP_TCC_READ_REQ_sum TCP_PENDING_STALL_CYCLES_sum TCP_TOTAL_CACHE_ACCESSES_sum "
    "GRBM_GUI_ACTIVE",
    "WRITE_SIZE TCC_EA0_RDREQ_sum TCC_EA0_RDREQ_32B_sum GRBM_GUI_ACTIVE",
    "TCC_MISS_sum TCC_REQ_sum TCC_EA0_RDREQ_DRAM_sum TCC_EA0_RDREQ_DRAM_32B_sum SQ_LDS_BANK_CONFLICT "
    "SQ_LDS_IDX_ACTIVE SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS SQ_INST_LEVEL_VMEM SQ_INSTS_VMEM_WR "
    "SQ_INSTS_VMEM_RD SQ_INSTS_SMEM GRBM_GUI_ACTIVE",
)
N_XCD, N_CU, N_SIMD = 8, 256, 1024


def _short_kernel(name):
    import re
    m = re.match(r"_ZN3sfa12_GLOBAL__N_1(\d+)", name)
    if m:  # a mangled name (some tracer records): identifier + the bf16 / float template argument
        n = int(m.group(1))
        ident = name[m.end():m.end() + n]
        rest = name[m.end() + n:]
        targ = "<bf16>" if rest.startswith("IDF16b") else "<float>" if rest.startswith("IfE") else ""
        return ident + targ
    n = name.replace("void ", "").replace("sfa::(anonymous namespace)::", "").replace("sfa::", "")
    n = re.sub(r"\(.*\)$", "", n)
    return n.replace("FwdCfg<32, 576, 512, 4, 1, true, 18, true>", "CfgMla")


def pmc_summary(root, copy_mib):
    """Summarise rocprofv3 counter CSVs laid out as ROOT/<target>_<pass>/
    (pass = 1-based index into PMC_PASSES; target "copy" is the
    ``--copy-probe COPY_MIB`` run that calibrates the byte counters) into
    per-dispatch means and derived figures per (target, kernel, grid).
    Cycle-based figures use GRBM_GUI_ACTIVE / 8 (one XCD's busy cycles) as
    the kernel's clock count; SQ wave counters count quad-cycles."""
    import csv
    import glob
    import re
    raw = {}
    for d in sorted(glob.glob(os.path.join(root, "*_[0-9]"))):
        target, ps = os.path.basename(d).rsplit("_", 1)
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            disp = {}
            with open(f) as fh:
                for r in csv.DictReader(fh):
                    e = disp.setdefault(r["Dispatch_Id"], {"c": {}})
                    e["c"][r["Counter_Name"]] = float(r["Counter_Value"])
                    e["ns"] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
                    wg = int(r["Workgroup_Size"])
                    e["key"] = (_short_kernel(r["Kernel_Name"]), int(r["Grid_Size"]) // max(wg, 1), wg)
                    e["res"] = {"vgpr": int(r["VGPR_Count"]), "agpr": int(r["Accum_VGPR_Count"]),
                                "lds": int(r["LDS_Block_Size"])}
            for e in disp.values():
                k = raw.setdefault(target, {}).setdefault(e["key"], {"res": e["res"], "passes": {}})
                k["passes"].setdefault(int(ps), []).append(e)
    def mean_pass(k, ps):
        es = k["passes"].get(ps, [])
        if not es:
            return None, None
        names = set().union(*[e["c"].keys() for e in es])
        return ({n: sum(e["c"].get(n, 0.0) for e in es) / len(es) for n in names},
                sum(e["ns"] for e in es) / len(es))
    # calibration from the copy probe (its largest reader)
    cal = {"copy_bytes": copy_mib << 20, "fetch_scale": None, "write_scale": None, "bytes_per_rdreq": None}
    if "copy" in raw:
        best = max(raw["copy"].values(), key=lambda k: (mean_pass(k, 2)[0] or {}).get("FETCH_SIZE", 0))
        c2, _ = mean_pass(best, 2)
        c3, _ = mean_pass(best, 3)
        if c2 and c2.get("FETCH_SIZE"):
            cal["fetch_scale"] = cal["copy_bytes"] / (c2["FETCH_SIZE"] * 1024)
        if c3 and c3.get("WRITE_SIZE"):
            cal["write_scale"] = cal["copy_bytes"] / (c3["WRITE_SIZE"] * 1024)
        if c3 and c3.get("TCC_EA0_RDREQ_sum"):
            cal["bytes_per_rdreq"] = cal["copy_bytes"] / c3["TCC_EA0_RDREQ_sum"]
    out = {"calibration": cal, "targets": {}}
    for target, kernels in raw.items():
        rows = []
        for (name, grid, wg), k in kernels.items():
            row = {"kernel": name, "workgroups": grid, "wg_threads": wg, **k["res"]}
            dispatches = max(len(v) for v in k["passes"].values())
            row["dispatches_per_pass"] = dispatches
            for ps in sorted(k["passes"]):
                c, ns = mean_pass(k, ps)
                row[f"pass{ps}_us"] = round(ns / 1e3, 2)
                g = c.get("GRBM_GUI_ACTIVE", 0.0) / N_XCD
                if ps == 1 and g:
                    row["clock_ghz"] = round(g / ns, 3)
                    row["mfma_busy"] = round(c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0) / (g * N_SIMD), 4)
                    row["waves_per_simd"] = round(4 * c.get("SQ_WAVE_CYCLES", 0) / (g * N_SIMD), 3)
                    if c.get("SQ_WAVE_CYCLES"):
                        row["wait_inst_frac"] = round(c.get("SQ_WAIT_INST_ANY", 0) / c["SQ_WAVE_CYCLES"], 3)
                    for n in ("MFMA", "VALU", "LDS", "SALU", "VMEM"):
                        row[f"insts_{n.lower()}"] = c.get(f"SQ_INSTS_{n}")
                if ps == 2:
                    fs = c.get("FETCH_SIZE", 0) * 1024
                    row["fetch_size_kib_raw"] = c.get("FETCH_SIZE")
                    if cal["fetch_scale"]:
                        row["fetch_bytes"] = fs * cal["fetch_scale"]
                        row["fetch_gbs"] = round(row["fetch_bytes"] / ns, 1)
                    if g:
                        row["ta_busy"] = round(c.get("TA_BUSY_avr", 0) / g, 3)
                        row["td_busy"] = round(c.get("TD_TD_BUSY_sum", 0) / (g * N_CU), 3)
                        row["td_tc_stall"] = round(c.get("TD_TC_STALL_sum", 0) / (g * N_CU), 3)
                        row["tcp_pending_stall"] = round(c.get("TCP_PENDING_STALL_CYCLES_sum", 0) / (g * N_CU), 3)
                    if c.get("TCP_TCC_READ_REQ_sum"):
                        row["l2_read_latency_cyc"] = round(c["TCP_TCC_READ_REQ_LATENCY_sum"] / c["TCP_TCC_READ_REQ_sum"], 1)
                    row["lds_dma_wavefronts"] = c.get("TA_BUFFER_READ_LDS_WAVEFRONTS_sum")
                    row["tcc_hit"] = c.get("TCC_HIT_sum")
                if ps == 3:
                    row["write_size_kib_raw"] = c.get("WRITE_SIZE")
                    row["ea_rdreq"] = c.get("TCC_EA0_RDREQ_sum")
                    if cal["write_scale"]:
                        row["write_bytes"] = c.get("WRITE_SIZE", 0) * 1024 * cal["write_scale"]
                        row["write_gbs"] = round(row["write_bytes"] / ns, 1)
                    if cal["bytes_per_rdreq"]:
                        row["rdreq_bytes"] = c.get("TCC_EA0_RDREQ_sum", 0) * cal["bytes_per_rdreq"]
                if ps == 4:
                    row["tcc_miss"] = c.get("TCC_MISS_sum")
                    row["tcc_req"] = c.get("TCC_REQ_sum")
                    if cal["bytes_per_rdreq"]:
                        row["dram_read_bytes"] = c.get("TCC_EA0_RDREQ_DRAM_sum", 0) * cal["bytes_per_rdreq"]
                    if c.get("SQ_LDS_IDX_ACTIVE"):
                        row["lds_bank_conflict_frac"] = round(c.get("SQ_LDS_BANK_CONFLICT", 0) / c["SQ_LDS_IDX_ACTIVE"], 4)
                    for n in ("VMEM_RD", "VMEM_WR", "SMEM"):
                        row[f"insts_{n.lower()}"] = c.get(f"SQ_INSTS_{n}")
            if row.get("tcc_hit") is not None and row.get("tcc_miss") is not None:
                row["l2_hit_frac"] = round(row["tcc_hit"] / max(row["tcc_hit"] + row["tcc_miss"], 1.0), 3)
            rows.append(row)
        rows.sort(key=lambda r: -r.get("pass1_us", 0) * r["dispatches_per_pass"])
        out["targets"][target] = rows
    return out


def _is_library_kernel(name):
    return (not name or name.startswith("at::") or name.startswith("__amd") or "at::native" in name
            or name.startswith("rocprim::"))


def pmc_markdown(summary, targets=None):
    """The summary as markdown tables: per target (all, or those named),
    this library's kernels (input generation, cache flushes and copies made
    by torch / the HIP runtime are left out)."""
    def f(x, nd=3):
        if x is None:
            return "-"
        if isinstance(x, float) and (abs(x) >= 1e5 or (x and abs(x) < 1e-3)):
            return f"{x:.4g}"
        return f"{x:.{nd}f}" if isinstance(x, float) else str(x)
    cal = summary["calibration"]
    lines = [f"Calibration (plain copy of {cal['copy_bytes'] >> 20} MiB): FETCH_SIZE x {f(cal['fetch_scale'])}, "
             f"WRITE_SIZE x {f(cal['write_scale'])}, {f(cal['bytes_per_rdreq'], 1)} B per TCC_EA0_RDREQ", ""]
    for target, rows in summary["targets"].items():
        if target == "copy" or (targets and target not in targets):
            continue
        rows = [r for r in rows if not _is_library_kernel(r["kernel"])]
        lines += [f"### {target}", "",
                  "| kernel | WGs x thr | LDS B | us | GHz | waves/SIMD | MFMA busy | wait-inst | "
                  "MFMA / VALU / LDS / SALU / VMEM insts | fetch GB (GB/s) | RDREQ GB | write GB (GB/s) | "
                  "L2 hit | L2 lat | TA / TD busy | LDS confl |",
                  "|" + "---|" * 16]
        for r in rows:
            ins = " / ".join(f(r.get(f"insts_{n}"), 0) if r.get(f"insts_{n}") is not None else "-"
                             for n in ("mfma", "valu", "lds", "salu", "vmem"))
            gb = lambda b: f"{b / 1e9:.3f}" if b is not None else "-"
            lines.append(
                f"| {r['kernel'][:60]} | {r['workgroups']} x {r['wg_threads']} | {r['lds']} | "
                f"{f(r.get('pass1_us'), 1)} | {f(r.get('clock_ghz'), 2)} | {f(r.get('waves_per_simd'), 2)} | "
                f"{f(r.get('mfma_busy'))} | {f(r.get('wait_inst_frac'))} | {ins} | "
                f"{gb(r.get('fetch_bytes'))} ({f(r.get('fetch_gbs'), 0)}) | {gb(r.get('rdreq_bytes'))} | "
                f"{gb(r.get('write_bytes'))} ({f(r.get('write_gbs'), 0)}) | {f(r.get('l2_hit_frac'))} | "
                f"{f(r.get('l2_read_latency_cyc'), 0)} | {f(r.get('ta_busy'))} / {f(r.get('td_busy'))} | "
                f"{f(r.get('lds_bank_conflict_frac'))} |")
        lines.append("")
    return "\n".join(lines)


def trace_summary(root):
    """Per (kernel, grid) duration statistics of the rocprofv3
    ``--kernel-trace`` CSVs under ROOT, as a markdown table (library kernels
    of torch and the HIP runtime left out).  Several workloads share a
    kernel instance, so the grid tells them apart."""
    import csv
    import glob
    import statistics
    groups = {}
    for f in glob.glob(os.path.join(root, "**", "*kernel_trace.csv"), recursive=True):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                name = _short_kernel(r["Kernel_Name"])
                if _is_library_kernel(name):
                    continue
                wg = int(r.get("Workgroup_Size_X", r.get("Workgroup_Size", 1)) or 1)
                grid = int(r.get("Grid_Size_X", r.get("Grid_Size", 0)) or 0) // max(wg, 1)
                # (registers, spills and occupancy: `python -m ops_amd.build --resource-usage`, from
                # the compiler; the trace's register columns leave out the accumulation registers)
                key = (name, grid, wg, r.get("LDS_Block_Size", r.get("Group_Segment_Size", "")))
                groups.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    lines = ["| kernel | workgroups x threads | LDS B | launches | total ms | avg us | min | median | max |",
             "|" + "---|" * 9]
    for (name, grid, wg, lds), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| {name} | {grid} x {wg} | {lds} | {len(d)} | {sum(d) / 1e3:.2f} | "
                     f"{statistics.mean(d):.1f} | {min(d):.1f} | {statistics.median(d):.1f} | {max(d):.1f} |")
    return "\n".join(lines)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--extra", default="tiny,prefill,train_gqa,mla_decode,indexer,mla_bwd,shim",
                    help="comma list of additional workloads to measure ('' for none)")
    ap.add_argument("--no-bwd", action="store_true", help="skip the train_gqa backward timing")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--profile", default="", metavar="NAME",
                    help="only launch workload NAME's kernels `steps` times (for counter runs) and exit: "
                         "mla_prefill, prefill, train_gqa_fwd, train_gqa_bwd_csr, train_gqa_bwd_atomic, "
                         "mla_decode, mla_decode_paged, mla_bwd, shim_fwd, shim_bwd")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("DIR", "OUT_JSON"),
                    help="summarise counter CSVs under DIR/<target>_<pass>/ (passes = PMC_PASSES) into "
                         "OUT_JSON, print markdown tables, and exit (needs no GPU)")
    ap.add_argument("--pmc-copy-mib", type=int, default=1024, help="size of the calibrating copy probe")
    ap.add_argument("--pmc-targets", default="", help="comma list: print only these targets' tables")
    ap.add_argument("--pmc-passes", action="store_true", help="print PMC_PASSES, one line each, and exit")
    ap.add_argument("--trace-summary", metavar="DIR",
                    help="print per-(kernel, grid) durations of the --kernel-trace CSVs under DIR and exit")
    ap.add_argument("--probe", default="", metavar="NAME",
                    help="measure a hardware ceiling the design rests on and exit: gemm (bf16 GEMM rate), "
                         "decode_gather (the decode's data movement without its MFMA work, per work layout)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB `steps` times (calibrates the "
                         "FETCH_SIZE / WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.pmc_passes:
        print("\n".join(PMC_PASSES))
        return
    if args.trace_summary:
        print(trace_summary(args.trace_summary), flush=True)
        return
    if args.pmc_summary:
        summ = pmc_summary(args.pmc_summary[0], args.pmc_copy_mib)
        with open(args.pmc_summary[1], "w") as fh:
            json.dump(summ, fh, indent=1)
        print(pmc_markdown(summ, [t for t in args.pmc_targets.split(",") if t]), flush=True)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the sparse attention path runs on a single MI355X "
              "(multi-GPU sharding is described as a design only, not implemented)", file=sys.stderr)
        sys.exit(2)
    import torch
    assert torch.cuda.is_available(), "no GPU"
    torch.backends.cuda.matmul.allow_tf32 = False
    if args.copy_probe:
        n = args.copy_probe << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n, "launches": args.steps}), flush=True)
        return
    if args.probe:
        run_probe(args.probe, args)
        return
    if args.profile:
        fn, before = profile_targets(args.profile)
        torch.cuda.synchronize()
        for i in range(args.steps):
            if before:
                before()
            fn()
        torch.cuda.synchronize()
        print(json.dumps({"profile": args.profile, "launches": args.steps}), flush=True)
        return

    w, head = bench_mla_prefill(args)
    extra = {}
    for name in [x for x in args.extra.split(",") if x]:
        log(f"measuring {name}")
        if name == "indexer":
            extra[name] = bench_indexer(args, w)
        else:
            extra[name] = {"tiny": bench_tiny, "prefill": bench_prefill, "train_gqa": bench_train_gqa,
                           "mla_decode": bench_mla_decode, "mla_bwd": bench_mla_bwd,
                           "shim": bench_shim}[name](args)
        torch.cuda.empty_cache()
    cpu = None
    if not args.no_cpu:
        for res, name, wl in _CPU_PENDING:
            res["cpu"] = cpu_rate(name, wl)
        _CPU_PENDING.clear()
        log("cpu baseline (oracle) on a bounded sample")
        cpu = cpu_baseline_mla(w, args.cpu_seconds)
        cpu["cpu_model"] = cpu_model()
        cpu["per_config"] = {n: r.pop("cpu") for n, r in extra.items() if isinstance(r, dict) and "cpu" in r}
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_mla_prefill.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("bytes_per_launch")
    line = {
        "metric": METRIC,
        "value": round(head["value"], 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/kv; causal top-k indices with recency bias)",
        "config": {"workload": "mla_prefill", "B": 1, "S": 32768, "Hq": 128, "Hkv": 1, "d_qk": 576, "d_v": 512,
                   "topk": 2048, "valid_pairs": head["valid_pairs"]},
        "roofline": {"bound": "mfma", "achieved": round(head["achieved_tflops"], 3), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(head["achieved_tflops"] / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic, "kernel": "idx_sort_kernel + fwd_mfma_kernel<MLA> (one sfa_fwd call)",
                     "kernel_ms": round(head["kernel_ms"], 4),
                     "presorted_ms": round(head["presorted_ms"], 4)},
        "cpu_baseline": cpu,
        "workloads": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
