#!/usr/bin/env python3
"""Benchmark of the SSLA hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Headline workload (config 2, C2): chunked GLA forward, B=8 sequences x
T=4096 tokens, H=8, K=V=64, chunk 64, bf16 q/k/v/o, fp32 g/h0/ht.  One
"step" = one call of ssla_gla_chunk_fwd over the whole batch with inputs
already resident in HBM.  Three input sets (3 x 203 MB) rotate, so each
call's inputs were last touched 406 MB of traffic earlier -- more than the
256 MB Infinity Cache holds -- and the timed loop streams from HBM.

Secondary lines (same JSON object): config 1 (the recurrent GLA call the
reference runs on the CPU), the per-site sparse GLA scan (config 3, 64 bins
per pass, bin by bin and in one call), the scatter-max pooling (config 4,
1e6 events, in shuffled order and sorted by cell), the asynchronous forward
step (config 5, 20 windows x 50k events with carried per-site states), the
chunk GLA backward at config 2, and the first stage of the MOS_S backbone
(ingest, preprocess, two MosAttention layers, SparseMaxPool,
TemporalDropout) on 8 synthetic Gen1 windows.

CPU baselines (``cpu_baseline`` of the main line and of the config 1, 3, 4
and 5 lines) time this build's PyTorch / fp64 restatements of the
reference's CPU-capable paths (oracle/) on the host's cores after the GPU
measurements, with the thread count, host CPU count and CPU model recorded.

Prints ONE JSON line.  Kernel durations come from HIP events recorded on
the stream the kernels are launched on (torch's current stream, which is
the stream handed to the C-ABI).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
FP32_PEAK_TFLOPS = 157.3       # MI355X fp32, TFLOP/s

C2 = dict(B=8, T=4096, H=8, D=64)


def c2_bytes():
    Tt, H, D = C2["B"] * C2["T"], C2["H"], C2["D"]
    # q, k, v bf16 + g fp32 read, o bf16 written, h0 read + ht written fp32
    return 3 * Tt * H * D * 2 + Tt * H * D * 4 + Tt * H * D * 2 + 2 * C2["B"] * H * D * D * 4


def c2_flops():
    Tt, H, D = C2["B"] * C2["T"], C2["H"], C2["D"]
    BT = 64
    # causal-useful: T*H*[(BT+1)(K+V) + 4KV]
    return Tt * H * ((BT + 1) * (D + D) + 4 * D * D)


def _source_sha(rel):
    import hashlib
    return hashlib.sha256((ROOT / rel).read_bytes()).hexdigest()[:16]


def _traffic_from_profile(name, source):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by the copy-kernel calibration), read from the
    committed summary profiles/<name>, with the note that says where it came
    from.  The summary records the sha256 (first 16 hex digits) of the
    kernel source it was measured on; when that is not the current source
    the figure is stale and None is returned."""
    p = ROOT / "profiles" / name
    if not p.exists():
        return None, f"profiles/{name} missing"
    val, sha = None, None
    for line in p.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                val = float(line.split(":", 1)[1].strip().split()[0])
            except ValueError:
                val = None
        elif line.startswith("source_sha256_16:"):
            sha = line.split(":", 1)[1].strip().split()[0]
    cur = _source_sha(source)
    if sha != cur:
        return None, (f"profiles/{name} was measured on {source} sha {sha}, the current source is {cur}: "
                      "stale, not reported")
    return val, f"rocprofv3 --pmc FETCH_SIZE + WRITE_SIZE from profiles/{name} ({source} sha {cur})"


def _cpu_info():
    """Host-core facts recorded with every CPU baseline."""
    import torch
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"host_cpus": os.cpu_count(), "torch_threads": torch.get_num_threads(), "cpu_model": model}


def _cpu_threads():
    """Threads for the CPU legs: the box's CPU share (OMP_NUM_THREADS is set
    to it there), never more than the host reports."""
    n = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    return max(1, min(n, os.cpu_count() or 1))


def _median_time(fn, runs=3):
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2], ts


def _flush_mall(torch, dev, buf=[]):
    """Write 512 MiB so that nothing of the previous pass stays in the
    256 MB Infinity Cache (used between timed passes, outside the timing)."""
    if not buf:
        buf.append(torch.empty(512 * 2**20 // 4, dtype=torch.float32, device=dev))
    buf[0].zero_()


def bench_chunk(torch, lib, steps, warmup, dev):
    from ssla_amd import _lib, synthetic
    sets = []
    for seed in (0, 1, 2):
        x = synthetic.chunk_gla_inputs(seed=seed, device=dev)
        x["o"] = torch.empty_like(x["v"])
        x["ht"] = torch.empty_like(x["initial_state"])
        sets.append(x)
    Tt, H, D = C2["B"] * C2["T"], C2["H"], C2["D"]
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    ws_bytes = lib.ssla_gla_chunk_workspace_size(C2["B"], Tt, H, D, D)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)

    def launch(x):
        st = lib.ssla_gla_chunk_fwd(
            x["q"].data_ptr(), x["k"].data_ptr(), x["v"].data_ptr(), x["g"].data_ptr(), _lib.SSLA_F32,
            x["cu_seqlens"].data_ptr(), C2["B"], Tt, H, D, D, float(x["scale"]),
            x["initial_state"].data_ptr(), x["o"].data_ptr(), x["ht"].data_ptr(), _lib.SSLA_BF16,
            ws.data_ptr(), ws_bytes, sh)
        _lib.check(st, "ssla_gla_chunk_fwd")

    for i in range(warmup):
        launch(sets[i % len(sets)])
    torch.cuda.synchronize()
    # one HIP event pair on the launch stream around the K timed calls (no
    # per-call markers inside the timed region): the average call time
    # includes the gaps between calls
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        launch(sets[i % len(sets)])
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    avg_ms = e0.elapsed_time(e1) / steps
    return dict(wall_s=wall, kernel_avg_ms=avg_ms, tokens=Tt, sample=sets[0])


C3_STEP_BYTES = 4 * (2 * 4 * 32 * 32 + 3 * 4 * 32 + 2 * 4 * 32) + 4   # state in + out, q k g v o, index


def _c3_sets(torch, dev, n_sets=2):
    """Config-3 inputs on the device, n_sets independent draws (state table
    74.7 MB + the bins' q, k, v, g, o about 146 MB per set)."""
    from ssla_amd import synthetic
    sets = []
    for seed in range(n_sets):
        sb = synthetic.sparse_scan_bins(seed=seed)
        bins = [dict(s=torch.from_numpy(sb.sites[b]).to(dev), q=sb.q[b].to(dev), k=sb.k[b].to(dev),
                     v=sb.v[b].to(dev), g=sb.g[b].to(dev), o=torch.empty(sb.sites[b].size, 4, 32, device=dev))
                for b in range(len(sb.sites))]
        sets.append(dict(sb=sb, bins=bins, state=sb.state0.to(dev).contiguous()))
    return sets


def cpu_sparse(sb, n_bins=64, runs=5):
    """CPU leg of config 3: the per-bin torch loop (gather the active states,
    decay-and-add update, o, scatter back) over the pass's n_bins bins."""
    import torch
    from oracle import torch_ref
    torch.set_num_threads(_cpu_threads())
    sites = [torch.from_numpy(s).long() for s in sb.sites[:n_bins]]
    steps = sum(int(s.numel()) for s in sites)
    torch_ref.sparse_scan_bins(sb.state0.clone(), sites[:2], sb.q, sb.k, sb.v, sb.g, sb.scale)   # warm-up
    med, ts = _median_time(lambda: torch_ref.sparse_scan_bins(sb.state0.clone(), sites, sb.q, sb.k, sb.v, sb.g,
                                                              sb.scale), runs)
    return {"value": steps / med, "unit": "site-steps/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{n_bins} bins ({steps} site-steps), torch fp32 per-bin index_select / "
                      f"update / einsum / index_copy_; median of {len(ts)} runs {[round(t, 3) for t in ts]} s",
            **_cpu_info()}


def bench_sparse(torch, lib, reps, dev, sets=None, cpu=True):
    """Config 3: 64 bins of per-site GLA updates, bin by bin (one
    ssla_sparse_gla_step launch per bin).  Two independent input sets
    alternate and 512 MiB are written between passes (outside the timing),
    so every pass starts with nothing in the Infinity Cache; within a pass
    a state row read by several bins may stay cached, as it would in use."""
    from ssla_amd import _lib
    sets = sets or _c3_sets(torch, dev)
    stream = torch.cuda.current_stream(dev)
    n_sites = sets[0]["sb"].n_sites
    scale = float(sets[0]["sb"].scale)

    def one_pass(x, sh):
        for b in x["bins"]:
            st = lib.ssla_sparse_gla_step(b["s"].data_ptr(), b["s"].numel(), b["q"].data_ptr(), b["k"].data_ptr(),
                                          b["v"].data_ptr(), b["g"].data_ptr(), x["state"].data_ptr(), n_sites, 4, 32,
                                          32, scale, b["o"].data_ptr(), None, sh)
            _lib.check(st, "ssla_sparse_gla_step")

    def timed(run, n):
        tot = 0.0
        for i in range(n):
            _flush_mall(torch, dev)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            run(sets[i % len(sets)])
            e1.record(stream)
            torch.cuda.synchronize()
            tot += e0.elapsed_time(e1)
        return tot / n

    for x in sets:
        one_pass(x, stream.cuda_stream)
    torch.cuda.synchronize()
    ms = timed(lambda x: one_pass(x, stream.cuda_stream), reps)
    # the same pass captured once per set as a HIP graph and replayed (no launch gaps)
    side = torch.cuda.Stream(dev)
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        for x in sets:
            one_pass(x, side.cuda_stream)
    stream.wait_stream(side)
    graphs = []
    for x in sets:
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            one_pass(x, torch.cuda.current_stream(dev).cuda_stream)
        graphs.append(gr)
    for gr in graphs:
        gr.replay()
    torch.cuda.synchronize()
    gidx = {id(x): i for i, x in enumerate(sets)}
    ms_graph = timed(lambda x: graphs[gidx[id(x)]].replay(), reps)
    steps = sets[0]["sb"].site_steps
    gbs = steps * C3_STEP_BYTES / (ms * 1e-3) / 1e9
    gbs_graph = steps * C3_STEP_BYTES / (ms_graph * 1e-3) / 1e9
    return {"workload": "sparse_gla_step config 3: 76x60 sites, 64 bins, H=4, K=V=32, fp32",
            "metric": "sparse scan site-steps/s", "value": steps / (ms * 1e-3), "unit": "site-steps/s",
            "ms_per_pass": ms, "site_steps_per_pass": steps, "launches_per_pass": len(sets[0]["bins"]),
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "bytes_per_site_step": C3_STEP_BYTES,
                         "note": "per-pass average over 64 launches (launch gaps included); 2 input sets "
                                 "(2 x 221 MB) alternate and the Infinity Cache is flushed before every pass"},
            "graph": {"value": steps / (ms_graph * 1e-3), "ms_per_pass": ms_graph, "achieved": gbs_graph,
                      "frac": gbs_graph / HBM_PEAK_GBS,
                      "note": "the 64 launches captured once as a HIP graph and replayed"},
            **({"cpu_baseline": cpu_sparse(sets[0]["sb"])} if cpu else {})}


def bench_sparse_batched(torch, lib, reps, dev):
    """Config 3 with all 64 bins in one call (sparse_gla_scan ->
    ssla_gla_recurrent_fwd with state_idx): the same site-steps regrouped
    site-major, stable in time (outside the timing), so each active site's
    state is read and written once per pass instead of once per step.  Two
    input sets alternate; the state is restored and 512 MiB are written
    before every call, outside the events."""
    import numpy as np
    from ssla_amd import _lib, synthetic
    sets = []
    for seed in (0, 1):
        sb = synthetic.sparse_scan_bins(seed=seed)
        site_all = np.concatenate(sb.sites)
        order = np.argsort(site_all, kind="stable")
        uniq, counts = np.unique(site_all[order], return_counts=True)
        perm = torch.from_numpy(order)
        x = dict(cu=torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int64, device=dev),
                 sidx=torch.from_numpy(uniq.astype(np.int32)).to(dev), n=int(uniq.size), scale=float(sb.scale),
                 state0=sb.state0.to(dev).contiguous())
        for nm, xs in (("q", sb.q), ("k", sb.k), ("v", sb.v), ("g", sb.g)):
            x[nm] = torch.cat(xs)[perm].to(dev).contiguous()
        x["state"] = x["state0"].clone()
        x["o"] = torch.empty_like(x["v"])
        sets.append(x)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream

    def call(x):
        T, H, K = x["q"].shape
        V = x["v"].shape[-1]
        st = lib.ssla_gla_recurrent_fwd(x["q"].data_ptr(), x["k"].data_ptr(), x["v"].data_ptr(), x["g"].data_ptr(),
                                        _lib.SSLA_F32, x["cu"].data_ptr(), x["n"], T, H, K, V, x["scale"],
                                        x["state"].data_ptr(), x["o"].data_ptr(), x["state"].data_ptr(),
                                        x["sidx"].data_ptr(), int(x["state"].shape[0]), None, _lib.SSLA_F32, None,
                                        0, sh)
        _lib.check(st, "ssla_gla_recurrent_fwd")

    for x in sets:
        call(x)
    torch.cuda.synchronize()
    ms_tot = 0.0
    for i in range(reps):
        x = sets[i % 2]
        x["state"].copy_(x["state0"])
        _flush_mall(torch, dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        call(x)
        e1.record(stream)
        torch.cuda.synchronize()
        ms_tot += e0.elapsed_time(e1)
    ms = ms_tot / reps
    T, H, K = sets[0]["q"].shape
    V = sets[0]["v"].shape[-1]
    alg = T * 4 * (3 * H * K + 2 * H * V) + sets[0]["n"] * 2 * H * K * V * 4
    gbs = alg / (ms * 1e-3) / 1e9
    return {"workload": "sparse scan config 3, 64 bins in one call (per-site histories, state once per site)",
            "metric": "sparse scan site-steps/s", "value": T / (ms * 1e-3), "unit": "site-steps/s",
            "ms_per_pass": ms, "site_steps_per_pass": T, "active_sites": sets[0]["n"],
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "algorithmic_bytes": alg,
                         "note": "q, k, g, v in and o out per step; the state of each active site in and out "
                                 "once; Infinity Cache flushed before every call"}}


def cpu_pool(src, index, n_out):
    """CPU leg of config 4: Tensor.scatter_reduce_('amax', include_self=False)
    plus the first-index argmax pass (torch_scatter is not installed)."""
    import torch
    from oracle import torch_ref
    torch.set_num_threads(_cpu_threads())
    torch_ref.scatter_max(src[:10000], index[:10000], n_out)   # warm-up
    med, ts = _median_time(lambda: torch_ref.scatter_max(src, index, n_out), 5)
    return {"value": src.shape[0] / med, "unit": "events/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"the whole config-4 call ({src.shape[0]} events x {src.shape[1]} channels, same index "
                      f"order), torch fp32 scatter_reduce_ amax + first-index argmax; median of {len(ts)} runs "
                      f"{[round(t, 3) for t in ts]} s", **_cpu_info()}


def bench_pool(torch, lib, reps, dev, sorted_index=False, cpu=True):
    """Config 4: scatter_max of 1e6 clustered events (C=64) into 152x120
    cells; with sorted_index the events are first ordered by cell (the
    non-decreasing segment ids SparsePool hands over), outside the timing.
    Two input sets (2 x 264 MB) alternate."""
    from ssla_amd import _lib, synthetic
    sets = []
    cpu_in = None
    for seed in (0, 1):
        src, index, n_out = synthetic.pooling_events(seed=seed)
        if sorted_index:
            index, order = torch.sort(index, stable=True)
            src = src[order]
        if cpu_in is None:
            cpu_in = (src, index, n_out)
        sets.append(dict(src=src.to(dev), idx=index.to(dev)))
    E, C = sets[0]["src"].shape
    ws_bytes = lib.ssla_scatter_workspace_size(E, C, n_out)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    out = torch.empty(n_out, C, device=dev)
    arg = torch.empty(n_out, C, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream

    def call(x):
        st = lib.ssla_scatter_max(x["src"].data_ptr(), x["idx"].data_ptr(), E, C, n_out, int(sorted_index),
                                  out.data_ptr(), arg.data_ptr(), ws.data_ptr(), ws_bytes, sh)
        _lib.check(st, "ssla_scatter_max")

    for i in range(3):
        call(sets[i % 2])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        call(sets[i % 2])
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    alg = E * (4 * C + 4) + n_out * C * (4 + 8)
    gbs = alg / (ms * 1e-3) / 1e9
    order = "sorted by cell" if sorted_index else "shuffled"
    return {"workload": f"scatter_max config 4: 1e6 {order} events, C=64, 18240 cells",
            "metric": "pooling events/s", "value": E / (ms * 1e-3), "unit": "events/s",
            "ms_per_call": ms,
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "algorithmic_bytes": alg,
                         "note": "whole call (bucketing + reduce), not one kernel"},
            **({"cpu_baseline": cpu_pool(*cpu_in)} if cpu else {})}


def bench_event_stage(torch, lib, reps, dev):
    """First stage of the reference's MOS_S backbone (configs/model/MOS_S.yaml
    layers 1-4, built as model_mos.py:32-122 builds them, run as
    model_mos.py:157-209) over a C5-like batch of 8 Gen1 windows (~50k events
    each): the .dat records are decoded and padded on the device (ingest,
    PCIe copy of the records included), then preprocess ->
    MosAttention(2 -> 12, k1) -> MosAttention(12, k3) -> SparseMaxPool(k2) ->
    TemporalDropout(4), forward only.  Each step is timed with HIP events on
    the current stream (host syncs inside a layer count)."""
    import numpy as np
    from ssla_amd import events as E, io, layers, synthetic
    frame = (240, 304)
    ev, ln = synthetic.event_windows()
    recs = []
    for b in range(ev.shape[0]):
        x = ev[b, :int(ln[b])].numpy()
        r = np.empty(x.shape[0], dtype=io.EV_TYPE)
        r["t"] = x[:, 2].astype(np.uint32)
        r["_"] = (x[:, 0].astype(np.int32) + (x[:, 1].astype(np.int32) << 14)
                  + (((x[:, 3] + 1) // 2).astype(np.int32) << 28))
        recs.append(r)
    torch.manual_seed(0)
    m1 = layers.MosAttention(2, 12, frame, (1, 1)).to(dev)
    m2 = layers.MosAttention(12, 12, frame, (3, 3)).to(dev)
    pool = layers.SparseMaxPool(frame, kernel_size=(2, 2)).to(dev)
    drop = layers.TemporalDropout(4, pool.frame_output_size).to(dev)
    stream = torch.cuda.current_stream(dev)
    names = ["ingest", "preprocess", "mos_k1_h12", "mos_k3_h12", "maxpool_k2", "tdrop_w4"]

    def run(ev_marks):
        x = io.pad_events(recs, dev)
        ev_marks[1].record(stream)
        x = E.preprocess_inputs(x[0], x[1].to(dev), frame, 50)
        ev_marks[2].record(stream)
        for i, m in enumerate((m1, m2, pool, drop)):
            x = m(x)
            ev_marks[3 + i].record(stream)
        return x

    marks = [torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
    with torch.no_grad():
        for _ in range(2):
            marks[0].record(stream)
            out = run(marks)
        torch.cuda.synchronize()
        tot = [0.0] * len(names)
        for _ in range(reps):
            marks[0].record(stream)
            out = run(marks)
            torch.cuda.synchronize()
            for i in range(len(names)):
                tot[i] += marks[i].elapsed_time(marks[i + 1])
    per = {n: t / reps for n, t in zip(names, tot)}
    ms = sum(per.values())
    n_ev = int(ln.sum())
    # the k3 layer's fused call alone (outside the stage timing): its patch
    # rows precomputed, ssla_mos_attention_fwd timed with HIP events
    from ssla_amd import _lib
    with torch.no_grad():
        x = E.preprocess_inputs(*[t.to(dev) for t in io.pad_events(recs, dev)], frame, 50)
        x = m1(x)
        src, _t, pos, _fi, f_len, _n = E._rf_scatter(x, frame, m2.patch2pixel_lut)
        rows, px = int(src.numel()), int(x["time"].numel())
        evx = x["events"].contiguous()
        A = 9
        ws = torch.empty(max(lib.ssla_mos_attention_workspace_size(px, 12, 12, A, rows, f_len.numel()), 1),
                         dtype=torch.uint8, device=dev)
        yk = torch.empty(px, 12, device=dev)
        w = [t.detach().contiguous() for t in (m2.scatter_conv_weights, m2.q_proj.weight, m2.v_proj.weight,
                                               m2.g_proj.weight, m2.o_proj.weight, m2.gather_conv_weights,
                                               m2.norm.weight, m2.norm.bias)]

        def fused_call():
            _lib.check(lib.ssla_mos_attention_fwd(
                evx.data_ptr(), px, 12, src.data_ptr(), pos.data_ptr(), rows, f_len.data_ptr(), f_len.numel(), A,
                w[0].data_ptr(), 1, w[1].data_ptr(), w[2].data_ptr(), w[3].data_ptr(), w[4].data_ptr(),
                w[5].data_ptr(), 1, None, w[6].data_ptr(), w[7].data_ptr(), float(m2.norm.eps), 12, yk.data_ptr(),
                ws.data_ptr(), ws.numel(), stream.cuda_stream), "ssla_mos_attention_fwd")

        fused_call()
        torch.cuda.synchronize()
        f0, f1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        f0.record(stream)
        for _ in range(10):
            fused_call()
        f1.record(stream)
        torch.cuda.synchronize()
        fused_ms = f0.elapsed_time(f1) / 10
    flop_exec = 2 * rows * (3 * 12 * 12 + 12 * 12)   # folded matrices: q, v, g, then output
    return {"workload": "MOS_S stage 1 forward on 8 Gen1 windows (C5-like, synthetic): ingest + preprocess + "
                        "MosAttention k1/k3 (hidden 12) + SparseMaxPool k2 + TemporalDropout 4",
            "metric": "stage-1 events/s", "value": n_ev / (ms * 1e-3), "unit": "events/s", "ms_per_call": ms,
            "events_in": n_ev, "events_out": int(out["lengths"].sum()), "ms_per_step": per,
            "mos_k3": {"pixel_events": px, "patch_rows": rows,
                       "fp32_flop_reference": 2 * rows * (12 * 12 + 3 * 12 * 12 + 12 * 12 + 12 * 12),
                       "fp32_flop_executed": flop_exec, "fused_call_ms": fused_ms,
                       "note": "scatter proj, q/v/g, o_proj, gather proj per patch row (folded: 576 FMAs)"},
            "roofline": {"bound": "valu", "achieved": flop_exec / (fused_ms * 1e-3) / 1e12, "peak": FP32_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": flop_exec / (fused_ms * 1e-3) / 1e12 / FP32_PEAK_TFLOPS,
                         "kernel": "ssla_mos_attention_fwd of the k3 layer (fold + patch + event kernels, one call)",
                         "note": "fp32 FMAs of the patch rows; the per-row weight choice keeps it off MFMA"}}


def cpu_baseline(x):
    """CPU leg of config 2: the fp32 PyTorch restatement of
    naive_gla_recurrent (ops/gla/naive.py:50-111, per time step [H, K, V]
    tensor ops) on this host's cores, over the 8 whole 4096-token sequences
    of the same C2 batch, timed one sequence per run (the sequences are
    independent, so the batch rate is the per-sequence rate): the median of
    the 8 runs, after a warm-up on 64 tokens."""
    import torch
    from oracle import torch_ref
    torch.set_num_threads(_cpu_threads())
    q, k, v, g = (x[nm].float().cpu() for nm in ("q", "k", "v", "g"))
    h0 = x["initial_state"].cpu()
    cu = x["cu_seqlens"].cpu()
    scale = float(x["scale"])
    H = q.shape[1]
    torch_ref.naive_gla_recurrent(q[:64], k[:64], v[:64], g[:64], torch.tensor([0, 64]), scale, h0[:1], True)
    runs = []
    for n in range(len(cu) - 1):
        s, e = int(cu[n]), int(cu[n + 1])
        t0 = time.perf_counter()
        torch_ref.naive_gla_recurrent(q[s:e], k[s:e], v[s:e], g[s:e], torch.tensor([0, e - s]), scale,
                                      h0[n:n + 1], True)
        runs.append((time.perf_counter() - t0, e - s))
    runs.sort()
    t_med, tok = runs[len(runs) // 2]
    return {"value": tok / t_med / 1e6, "unit": "Mtok/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"the {len(runs)} sequences of the C2 batch ({tok} tokens x {H} heads each), one run per "
                      f"sequence, torch fp32 naive_gla_recurrent restatement; median {t_med:.2f} s of "
                      f"{[round(r[0], 2) for r in runs]} s", **_cpu_info()}


def bench_c1(torch, lib, reps, dev):
    """Config 1 (plumbing): naive recurrent GLA forward, N=1, H=4, T=256,
    K=V=32, fp32, q pre-scaled by 32^-1/2 and scale 1.0, zero initial state
    (seed 0).  The reference runs this on the CPU: its wall time with the
    host's threads is the baseline; the value is the same call through
    naive_gla_recurrent on the GPU (HIP events, launch included)."""
    import torch.nn.functional as F
    from oracle import torch_ref
    from ssla_amd.gla import naive_gla_recurrent
    gen = torch.Generator().manual_seed(0)
    q = torch.randn(256, 4, 32, generator=gen) * 32 ** -0.5
    k, v = torch.randn(256, 4, 32, generator=gen), torch.randn(256, 4, 32, generator=gen)
    g = F.logsigmoid(torch.randn(256, 4, 32, generator=gen) / 16)
    cu = torch.tensor([0, 256])
    dq, dk, dv, dg, dcu = (t.to(dev) for t in (q, k, v, g, cu))
    stream = torch.cuda.current_stream(dev)
    with torch.no_grad():
        for _ in range(3):
            naive_gla_recurrent(dq, dk, dv, dg, dcu, 1.0, None, True)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            naive_gla_recurrent(dq, dk, dv, dg, dcu, 1.0, None, True)
        e1.record(stream)
        torch.cuda.synchronize()
    gpu_ms = e0.elapsed_time(e1) / reps
    torch.set_num_threads(_cpu_threads())
    torch_ref.naive_gla_recurrent(q[:16], k[:16], v[:16], g[:16], torch.tensor([0, 16]), 1.0, None, True)
    med, ts = _median_time(lambda: torch_ref.naive_gla_recurrent(q, k, v, g, cu, 1.0, None, True), 5)
    return {"workload": "naive_gla_recurrent config 1 (C1): N=1, H=4, T=256, K=V=32, fp32, scale 1.0",
            "metric": "C1 recurrent GLA forward wall time", "value": gpu_ms, "unit": "ms",
            "higher_is_better": False, "roofline": None,
            "note": "plumbing configuration: 256 serial steps of a 4x32x32 state, no roofline binds; the GPU "
                    "time is the wrapper call (device-to-device, one launch)",
            "cpu_baseline": {"value": med * 1e3, "unit": "ms", "cores": torch.get_num_threads(), "kind": "port",
                             "sample": f"the whole C1 call, torch fp32 naive_gla_recurrent restatement; median of "
                                       f"{len(ts)} runs {[round(t * 1e3, 2) for t in ts]} ms", **_cpu_info()}}


def cpu_async_step(model, window, n_events):
    """CPU leg of config 5: the fp64 restatement of one window of the step
    (oracle.backbone: numpy event glue, C recurrence, numpy projections and
    head) on this host's cores, one window, one run (it takes seconds)."""
    import numpy as np
    import torch
    from oracle import backbone as ob
    torch.set_num_threads(_cpu_threads())
    params = {k: v.detach().float().cpu().numpy() for k, v in model.state_dict().items()}
    states = [np.zeros((Hg * Wg, model.heads, model.head_dim, model.head_dim), np.float32)
              for Hg, Wg in model.grid_sizes]
    ev = window.cpu().numpy()
    t0 = time.perf_counter()
    ob.async_step(params, ev, np.array([n_events]), states)
    dt = time.perf_counter() - t0
    return {"value": 1.0 / dt, "unit": "windows/s", "events_per_s": n_events / dt, "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"one {n_events}-event window of the step in the CPU restatement "
                                      f"(oracle.backbone.async_step, fp64), {dt:.1f} s", **_cpu_info()}


def _async_scan_times(torch, model, window, lengths, states, stream, reps=20):
    """Per stage: the per-site scan (sparse_gla_scan, the call inside
    ssla_site_gla_block) on the stage's inputs of one window, one event pair
    per call around each of reps calls on a copy of the states, the Infinity
    Cache flushed before each (so the states come from HBM); and its algorithmic
    bytes (bf16 q / k / v / o and fp32 g per event, each active site's fp32
    state read and written)."""
    import torch.nn.functional as F
    from ssla_amd.scan import sparse_gla_scan
    ms, nbytes = [], []
    hd = model.heads * model.head_dim
    with torch.no_grad():
        x = model.stem(window, lengths)
        for i, blk in enumerate(model.blocks):
            xe = x["events"].to(torch.float32)
            q, k, v, g = blk.project(xe)
            cu = F.pad(torch.cumsum(x["lengths"], 0), (1, 0))
            sites = blk.sites(x, model.grid_sizes[i])
            st = states[i].clone()
            o = sparse_gla_scan(q, k, v, g, cu, sites, st, scale=blk.head_dim ** -0.5, check=False)
            tot = 0.0
            for _ in range(reps):
                _flush_mall(torch, window.device)   # the states and inputs come from HBM, as in the step
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                sparse_gla_scan(q, k, v, g, cu, sites, st, scale=blk.head_dim ** -0.5, check=False)
                e1.record(stream)
                torch.cuda.synchronize()
                tot += e0.elapsed_time(e1)
            ms.append(tot / reps)
            n_ev, n_site = int(xe.shape[0]), int(x["lengths"].numel())
            nbytes.append(n_ev * (3 * hd * 2 + hd * 4 + hd * 2) + n_site * 2 * hd * model.head_dim * 4)
            out = dict(x)
            out["events"] = blk.finish(o, xe)
            if i < len(model.pools):
                x = model.pools[i](out)
    return ms, nbytes


def bench_async_step(torch, lib, dev, n_windows=20, n_events=50_000, cpu=True):
    """Config 5: the asynchronous forward step (ssla_amd.backbone) over
    n_windows consecutive windows of n_events events, per-stage states
    carried from window to window; raw <x, y, t, p> windows resident on the
    device before the timing.  value = windows/s over the whole timed run
    (host wall clock, synchronised) of AsyncSparseGLA.run, which plans each
    window while the previous one's stages run; the same windows through
    forward() one at a time are timed too (ms_per_window_forward_loop).  A
    second, instrumented pass over the
    same windows (fresh states) times each piece with HIP events (those
    intervals include the GPU's idle time while the host prepares a piece).
    The per-site scan of every stage is priced against HBM from its own
    timing: the stage's scan call on the last window's inputs, an event pair
    around each call, the Infinity Cache flushed before each (kernel time,
    no host gaps, states from HBM)."""
    from ssla_amd import synthetic
    from ssla_amd.backbone import AsyncSparseGLA
    torch.manual_seed(0)
    model = AsyncSparseGLA().to(dev).eval()
    wins = [w.to(dev) for w in synthetic.async_windows(n_windows, n_events, seed=0)]
    ln = torch.tensor([n_events], device=dev)
    stream = torch.cuda.current_stream(dev)
    with torch.no_grad():
        lns = [ln] * len(wins)
        warm = model.init_states(1, dev)
        model.run(wins, lns, warm)   # a whole pass: pinned count buffers and allocator pools warm
        for w in wins[:2]:
            model(w, ln, warm)
        states = model.init_states(1, dev)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for w in wins:
            model(w, ln, states)
        torch.cuda.synchronize()
        wall_loop = time.perf_counter() - t0
        states = model.init_states(1, dev)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        model.run(wins, lns, states)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        # instrumented pass: per-piece HIP events
        states = model.init_states(1, dev)
        piece_ms = {}
        for w in wins:
            marks = [("start", torch.cuda.Event(enable_timing=True))]
            marks[0][1].record(stream)

            def mark(name):
                e = torch.cuda.Event(enable_timing=True)
                e.record(stream)
                marks.append((name, e))

            model(w, ln, states, mark=mark)
            torch.cuda.synchronize()
            interval = {nm: a.elapsed_time(b) for (_, a), (nm, b) in zip(marks[:-1], marks[1:])}
            for nm, ms in interval.items():
                piece_ms[nm] = piece_ms.get(nm, 0.0) + ms / n_windows
        scan_ms, scan_bytes = _async_scan_times(torch, model, wins[-1], ln, states, stream)
    per_window_ms = wall * 1e3 / n_windows
    scans = []
    for i in range(4):
        gbs = scan_bytes[i] / (scan_ms[i] * 1e-3) / 1e9
        scans.append({"stage": i + 1, "ms_per_call": scan_ms[i], "algorithmic_bytes": scan_bytes[i],
                      "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS})
    line = {"workload": f"async forward step (config 5): {n_windows} windows x {n_events} events, 4 stages "
                        "32/64/128/256 ch at stride 4/8/16/32, H=4, D=32, per-site fp32 states carried, "
                        "bf16 projections and head",
            "metric": "async step windows/s", "value": n_windows / wall, "unit": "windows/s",
            "events_per_s": n_windows * n_events / wall, "ms_per_window": per_window_ms,
            "ms_per_window_forward_loop": wall_loop * 1e3 / n_windows,
            "ms_per_piece": piece_ms, "scan_kernels": scans,
            "roofline": {"bound": "hbm", "kernel": "ssla_gla_recurrent_fwd with state_idx (per-site scan), "
                                                   "stage 1", **{k: scans[0][k] for k in
                                                                 ("achieved", "peak", "unit", "frac")},
                         "note": "per stage: bf16 q/k/v, fp32 g, bf16 o per event plus each active site's "
                                 "fp32 state in and out, over the scan call's own time (one window's "
                                 "inputs, Infinity Cache flushed before each call); stage 1 (4,560 sites, "
                                 "~11 events each) is the "
                                 "widest, stages 2-4 walk long per-site histories"}}
    if cpu:
        line["cpu_baseline"] = cpu_async_step(model, wins[0], n_events)
    return line


def calibrate_copy(torch, dev, mib=256, reps=3):
    """Plain device-to-device copies of a known size.  Profiled with
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, the counter value per copy
    dispatch divided by mib MiB is the factor that turns those counters into
    bytes for the kernels of this path."""
    n = mib * 2**20 // 4
    src = torch.randn(n, device=dev)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": n * 4, "reps": reps}), flush=True)


def bench_chunk_bwd(torch, lib, reps, dev):
    """Backward of config 2 (ssla_gla_chunk_bwd): gradients of o and ht for
    the C2 batch, three input sets in rotation (369 MB each with their
    gradients: a call's data was last touched two calls before, more than
    the 256 MB Infinity Cache holds)."""
    from ssla_amd import _lib, synthetic
    Tt, H, D = C2["B"] * C2["T"], C2["H"], C2["D"]
    sets = []
    for seed in (0, 1, 2):
        x = synthetic.chunk_gla_inputs(seed=seed, device=dev)
        gen = torch.Generator(device=dev).manual_seed(100 + seed)
        x["do"] = torch.randn(x["v"].shape, generator=gen, device=dev).to(torch.bfloat16)
        x["dht"] = torch.randn(x["initial_state"].shape, generator=gen, device=dev) * 0.1
        for name, like in (("dq", "q"), ("dk", "k"), ("dv", "v"), ("dg", "g"), ("dh0", "initial_state")):
            x[name] = torch.empty_like(x[like])
        sets.append(x)
    ws_bytes = lib.ssla_gla_chunk_bwd_workspace_size(C2["B"], Tt, H, D, D)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream

    def launch(x):
        st = lib.ssla_gla_chunk_bwd(
            x["q"].data_ptr(), x["k"].data_ptr(), x["v"].data_ptr(), x["g"].data_ptr(), _lib.SSLA_F32,
            x["cu_seqlens"].data_ptr(), C2["B"], Tt, H, D, D, float(x["scale"]), x["initial_state"].data_ptr(),
            x["do"].data_ptr(), x["dht"].data_ptr(), x["dq"].data_ptr(), x["dk"].data_ptr(), x["dv"].data_ptr(),
            x["dg"].data_ptr(), x["dh0"].data_ptr(), _lib.SSLA_BF16, ws.data_ptr(), ws_bytes, sh)
        _lib.check(st, "ssla_gla_chunk_bwd")

    for i in range(3):
        launch(sets[i % len(sets)])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        launch(sets[i % len(sets)])
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    n16, n32, st_b = Tt * H * D * 2, Tt * H * D * 4, C2["B"] * H * D * D * 4
    alg = 4 * n16 + n32 + 2 * st_b + 3 * n16 + n32 + st_b   # q k v do g h0 dht in; dq dk dv dg dh0 out
    gbs = alg / (ms * 1e-3) / 1e9
    return {"workload": "chunk_gla backward (config 2): dq, dk, dv, dg, dh0 of o and ht; bf16, fp32 g",
            "metric": "GLA chunk bwd Mtok/s", "value": Tt / (ms * 1e-3) / 1e6, "unit": "Mtok/s",
            "ms_per_call": ms,
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "algorithmic_bytes": alg,
                         "note": "whole call (state passes + chunk kernel)"}}


def bench_mos_backbone(torch, lib, reps, dev):
    """The reference's MOS_S backbone forward (configs/model/MOS_S.yaml
    layers, built as model_mos.py:32-122 builds them, run as
    model_mos.py:157-209), random-init weights, over a C5-like batch of 8
    Gen1 windows (~50k events each): preprocess, then four stages of two
    MosAttention layers (hidden 12 / 24 / 48 / 96; the first of stages 2-4
    with an input projection) with SparseMaxPool k2 + TemporalDropout 4
    between them.  Every layer is timed with HIP events on the current stream
    (host syncs inside a layer count).  For the hidden 48 / 96 layers (the
    matrix-core path) the same layer through the composed forward is timed
    too, on the same input."""
    from ssla_amd import events as E, layers, synthetic
    frame = (240, 304)
    ev, ln = synthetic.event_windows()
    ev, ln = ev.to(dev), ln.to(dev)
    torch.manual_seed(0)
    mods, names = [], []
    size, cin = frame, 2
    for st, hid in enumerate((12, 24, 48, 96)):
        for j in range(2):
            k = 1 if (st == 0 and j == 0) else 3
            mods.append(layers.MosAttention(cin, hid, size, (k, k)).to(dev))
            names.append(f"s{st + 1}_mos{j + 1}_k{k}_{cin}to{hid}")
            cin = hid
        if st < 3:
            pool = layers.SparseMaxPool(size, kernel_size=(2, 2)).to(dev)
            mods += [pool, layers.TemporalDropout(4, pool.frame_output_size).to(dev)]
            names += [f"s{st + 1}_maxpool", f"s{st + 1}_tdrop"]
            size = pool.frame_output_size
    stream = torch.cuda.current_stream(dev)
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(len(mods) + 2)]

    def run(fused=None):
        marks[0].record(stream)
        x = E.preprocess_inputs(ev, ln, frame, 50)
        marks[1].record(stream)
        ins = []
        for i, m in enumerate(mods):
            ins.append(x)
            x = m(x, fused=fused) if isinstance(m, layers.MosAttention) else m(x)
            marks[2 + i].record(stream)
        return x, ins

    with torch.no_grad():
        for _ in range(2):
            out, ins = run()
        torch.cuda.synchronize()
        tot = [0.0] * (len(mods) + 1)
        for _ in range(reps):
            out, ins = run()
            torch.cuda.synchronize()
            for i in range(len(mods) + 1):
                tot[i] += marks[i].elapsed_time(marks[i + 1])
        per = {n: t / reps for n, t in zip(["preprocess"] + names, tot)}
        ms = sum(per.values())
        # hidden 48 / 96: fused (matrix-core) vs composed on each layer's own input
        big = {}
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for i, (m, n) in enumerate(zip(mods, names)):
            if not isinstance(m, layers.MosAttention) or m.hidden_size < 48:
                continue
            rows = {}
            for mode in (True, False):
                m(ins[i], fused=mode)
                torch.cuda.synchronize()
                a.record(stream)
                for _ in range(reps):
                    m(ins[i], fused=mode)
                b.record(stream)
                torch.cuda.synchronize()
                rows["fused_ms" if mode else "composed_ms"] = a.elapsed_time(b) / reps
            rows["pixel_events"] = int(ins[i]["time"].numel())
            rows["speedup"] = rows["composed_ms"] / rows["fused_ms"]
            big[n] = rows
    n_ev = int(ln.sum())
    return {"workload": "MOS_S backbone forward on 8 Gen1 windows (C5-like, synthetic): preprocess + 8 MosAttention "
                        "(hidden 12/24/48/96) + 3 x (SparseMaxPool k2 + TemporalDropout 4)",
            "metric": "MOS_S backbone events/s", "value": n_ev / (ms * 1e-3), "unit": "events/s", "ms_per_call": ms,
            "events_in": n_ev, "events_out": int(out["lengths"].sum()), "ms_per_step": per,
            "hidden_48_96_fused_vs_composed": big}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--only", choices=["chunk", "c1", "sparse", "sparse_batched", "pool", "pool_sorted", "chunk_bwd",
                                       "event_stage", "async_step", "mos_s"], default=None,
                    help="run one workload and print its line (profiling runs; --no-cpu-baseline skips "
                         "the CPU legs where a line has one)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run 256 MiB device copies (counter calibration) and exit")
    args = ap.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only; the hot path is not sharded "
              "across GPUs here. Run with --gpus 1.", file=sys.stderr)
        return 2
    import torch
    from ssla_amd import _lib
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        calibrate_copy(torch, dev)
        return 0
    lib = _lib.load()
    if args.only == "c1":
        print(json.dumps(bench_c1(torch, lib, args.steps, dev)), flush=True)
        return 0
    if args.only == "async_step":
        print(json.dumps(bench_async_step(torch, lib, dev, cpu=not args.no_cpu_baseline)), flush=True)
        return 0
    if args.only == "sparse":
        print(json.dumps(bench_sparse(torch, lib, args.steps, dev, cpu=not args.no_cpu_baseline)), flush=True)
        return 0
    if args.only == "chunk_bwd":
        print(json.dumps(bench_chunk_bwd(torch, lib, args.steps, dev)), flush=True)
        return 0
    if args.only == "sparse_batched":
        print(json.dumps(bench_sparse_batched(torch, lib, args.steps, dev)), flush=True)
        return 0
    if args.only == "mos_s":
        print(json.dumps(bench_mos_backbone(torch, lib, args.steps, dev)), flush=True)
        return 0
    if args.only == "event_stage":
        print(json.dumps(bench_event_stage(torch, lib, args.steps, dev)), flush=True)
        return 0
    if args.only in ("pool", "pool_sorted"):
        print(json.dumps(bench_pool(torch, lib, args.steps, dev, args.only == "pool_sorted",
                                    cpu=not args.no_cpu_baseline)), flush=True)
        return 0
    r = bench_chunk(torch, lib, args.steps, args.warmup, dev)
    ms_step = r["wall_s"] * 1e3 / args.steps
    value = r["tokens"] / (r["wall_s"] / args.steps) / 1e6
    kern_s = r["kernel_avg_ms"] * 1e-3
    alg_bytes = c2_bytes()
    achieved = alg_bytes / kern_s / 1e9
    traffic, traffic_note = _traffic_from_profile("gla_chunk_fwd_c2_pmc.txt", "ssla_amd/csrc/gla_chunk.hip")
    tflops = c2_flops() / kern_s / 1e12
    line = {
        "metric": "GLA chunk fwd Mtok/s (%bf16 MFMA peak); sparse scan site-steps/s (%HBM BW)",
        "value": value, "unit": "Mtok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "chunk_gla_fwd (config 2, C2): B=8, H=8, T=4096, K=V=64, chunk 64; "
                               "bf16 q/k/v/o, fp32 g/h0/ht; 3 input sets rotating (each call's inputs last touched 406 MB earlier, > MALL)",
                   "global_batch": C2["B"], "seq_len": C2["T"], "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic, "traffic_source": traffic_note,
                     "kernel": "ssla_gla_chunk_fwd (state + segment kernels, one call)",
                     "kernel_avg_us": r["kernel_avg_ms"] * 1e3,
                     "timing": "HIP events on the launch stream around the K timed calls, / K (gaps between "
                               "calls included)",
                     "algorithmic_bytes": alg_bytes},
        "mfma": {"achieved": tflops, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                 "frac": tflops / BF16_PEAK_TFLOPS, "flops_per_launch": c2_flops(),
                 "note": "causal-useful flops; the shape is HBM-bound (31.8 flop/B < 312 ridge)"},
    }
    if not args.no_secondary and args.only is None:
        line["secondary"] = [bench_c1(torch, lib, 20, dev), bench_sparse(torch, lib, 10, dev),
                             bench_sparse_batched(torch, lib, 10, dev), bench_pool(torch, lib, 20, dev),
                             bench_pool(torch, lib, 20, dev, sorted_index=True),
                             bench_async_step(torch, lib, dev, cpu=not args.no_cpu_baseline),
                             bench_chunk_bwd(torch, lib, 10, dev), bench_event_stage(torch, lib, 5, dev),
                             bench_mos_backbone(torch, lib, 5, dev)]
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(r["sample"])
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
