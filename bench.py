#!/usr/bin/env python3
"""Benchmark of the SSLA hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Headline workload (config 2, C2): chunked GLA forward, B=8 sequences x
T=4096 tokens, H=8, K=V=64, chunk 64, bf16 q/k/v/o, fp32 g/h0/ht.  One
"step" = one call of ssla_gla_chunk_fwd over the whole batch with inputs
already resident in HBM.  Two input sets (2 x 203 MB, more than the 256 MB
Infinity Cache) alternate so that the timed loop streams from HBM.

Secondary lines (same JSON object): the per-site sparse GLA scan (config 3,
64 bins per step), the scatter-max pooling (config 4, 1e6 events, in
shuffled order and sorted by cell), the chunk GLA backward at config 2, and
the first stage of the MOS_S backbone (ingest, preprocess, two MosAttention
layers, SparseMaxPool, TemporalDropout) on 8 synthetic Gen1 windows.

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


def _traffic_from_profile(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by the copy-kernel calibration), read from the
    committed summary profiles/<name>; None if absent."""
    p = ROOT / "profiles" / name
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return float(line.split(":", 1)[1].strip().split()[0])
            except ValueError:
                return None
    return None


def bench_chunk(torch, lib, steps, warmup, dev):
    from ssla_amd import _lib, synthetic
    sets = []
    for seed in (0, 1):
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
        launch(sets[i % 2])
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        ev[i][0].record(stream)
        launch(sets[i % 2])
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kern_ms = sorted(a.elapsed_time(b) for a, b in ev)
    avg_ms = sum(kern_ms) / len(kern_ms)
    return dict(wall_s=wall, kernel_avg_ms=avg_ms, kernel_median_ms=kern_ms[len(kern_ms) // 2],
                tokens=Tt, sample=sets[0])


def bench_sparse(torch, lib, reps, dev):
    """Config 3: 64 bins of per-site GLA updates, bin by bin."""
    from ssla_amd import _lib, synthetic
    sb = synthetic.sparse_scan_bins()
    state = sb.state0.to(dev).contiguous()
    bins = []
    for b in range(len(sb.sites)):
        bins.append(dict(s=torch.from_numpy(sb.sites[b]).to(dev), q=sb.q[b].to(dev), k=sb.k[b].to(dev),
                         v=sb.v[b].to(dev), g=sb.g[b].to(dev),
                         o=torch.empty(sb.sites[b].size, 4, 32, device=dev)))
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream

    def one_pass():
        for x in bins:
            st = lib.ssla_sparse_gla_step(x["s"].data_ptr(), x["s"].numel(), x["q"].data_ptr(),
                                          x["k"].data_ptr(), x["v"].data_ptr(), x["g"].data_ptr(),
                                          state.data_ptr(), sb.n_sites, 4, 32, 32, float(sb.scale),
                                          x["o"].data_ptr(), None, sh)
            _lib.check(st, "ssla_sparse_gla_step")

    one_pass()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        one_pass()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    # the same pass captured once as a HIP graph and replayed (no launch gaps)
    side = torch.cuda.Stream(dev)
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        sh = side.cuda_stream
        one_pass()
    stream.wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sh = torch.cuda.current_stream(dev).cuda_stream
        one_pass()
    sh = stream.cuda_stream
    graph.replay()
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(reps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    ms_graph = e0.elapsed_time(e1) / reps
    steps = sb.site_steps
    per_step_bytes = 4 * (2 * 4 * 32 * 32 + 3 * 4 * 32 + 2 * 4 * 32) + 4
    gbs = steps * per_step_bytes / (ms * 1e-3) / 1e9
    gbs_graph = steps * per_step_bytes / (ms_graph * 1e-3) / 1e9
    return {"workload": "sparse_gla_step config 3: 76x60 sites, 64 bins, H=4, K=V=32, fp32",
            "metric": "sparse scan site-steps/s", "value": steps / (ms * 1e-3), "unit": "site-steps/s",
            "ms_per_pass": ms, "site_steps_per_pass": steps, "launches_per_pass": len(bins),
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "bytes_per_site_step": per_step_bytes,
                         "note": "per-pass average over 64 launches, launch gaps included"},
            "graph": {"value": steps / (ms_graph * 1e-3), "ms_per_pass": ms_graph, "achieved": gbs_graph,
                      "frac": gbs_graph / HBM_PEAK_GBS,
                      "note": "the 64 launches captured once as a HIP graph and replayed"}}


def bench_sparse_batched(torch, lib, reps, dev):
    """Config 3 with all 64 bins in one call (sparse_gla_scan ->
    ssla_gla_recurrent_fwd with state_idx): the same site-steps regrouped
    site-major, stable in time (outside the timing), so each active site's
    state is read and written once per pass instead of once per step.  The
    state is restored between passes by a device copy outside the events."""
    import numpy as np
    from ssla_amd import _lib, synthetic
    sb = synthetic.sparse_scan_bins()
    site_all = np.concatenate(sb.sites)
    order = np.argsort(site_all, kind="stable")
    uniq, counts = np.unique(site_all[order], return_counts=True)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int64, device=dev)
    sidx = torch.from_numpy(uniq.astype(np.int32)).to(dev)
    perm = torch.from_numpy(order)
    q, k, v, g = (torch.cat(xs)[perm].to(dev).contiguous() for xs in (sb.q, sb.k, sb.v, sb.g))
    T, H, K = q.shape
    V = v.shape[-1]
    state0 = sb.state0.to(dev).contiguous()
    state = state0.clone()
    o = torch.empty(T, H, V, device=dev)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream

    def call():
        st = lib.ssla_gla_recurrent_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), _lib.SSLA_F32,
                                        cu.data_ptr(), int(uniq.size), T, H, K, V, float(sb.scale), state.data_ptr(),
                                        o.data_ptr(), state.data_ptr(), sidx.data_ptr(), int(state.shape[0]),
                                        None, _lib.SSLA_F32, sh)
        _lib.check(st, "ssla_gla_recurrent_fwd")

    call()
    torch.cuda.synchronize()
    ms_tot = 0.0
    for _ in range(reps):
        state.copy_(state0)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        call()
        e1.record(stream)
        torch.cuda.synchronize()
        ms_tot += e0.elapsed_time(e1)
    ms = ms_tot / reps
    steps = T
    alg = steps * 4 * (3 * H * K + 2 * H * V) + int(uniq.size) * 2 * H * K * V * 4
    gbs = alg / (ms * 1e-3) / 1e9
    return {"workload": "sparse scan config 3, 64 bins in one call (per-site histories, state once per site)",
            "metric": "sparse scan site-steps/s", "value": steps / (ms * 1e-3), "unit": "site-steps/s",
            "ms_per_pass": ms, "site_steps_per_pass": steps, "active_sites": int(uniq.size),
            "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs / HBM_PEAK_GBS, "algorithmic_bytes": alg,
                         "note": "q, k, g, v in and o out per step; the state of each active site in and out once"}}


def bench_pool(torch, lib, reps, dev, sorted_index=False):
    """Config 4: scatter_max of 1e6 clustered events (C=64) into 152x120
    cells; with sorted_index the events are first ordered by cell (the
    non-decreasing segment ids SparsePool hands over), outside the timing."""
    from ssla_amd import _lib, synthetic
    sets = []
    for seed in (0, 1):
        src, index, n_out = synthetic.pooling_events(seed=seed)
        if sorted_index:
            index, order = torch.sort(index, stable=True)
            src = src[order]
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
                         "note": "whole call (bucketing + reduce), not one kernel"}}


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


def cpu_baseline(x, min_s=10.0):
    """The fp64 C restatement of naive_gla_recurrent (oracle/) on this host,
    run over the sequences of the same C2 batch, cycling through the batch
    until at least min_s seconds of CPU work are done (one pass over the 8
    sequences takes well under a second)."""
    import numpy as np
    import oracle
    q = x["q"].float().cpu().numpy()
    k = x["k"].float().cpu().numpy()
    v = x["v"].float().cpu().numpy()
    g = x["g"].cpu().numpy()
    h0 = x["initial_state"].cpu().numpy()
    cu = x["cu_seqlens"].cpu().numpy()
    n_seq = len(cu) - 1
    H = q.shape[1]
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    oracle.load()
    done_tok, t_used, runs = 0, 0.0, 0
    while t_used < min_s:
        n = runs % n_seq
        s, e = int(cu[n]), int(cu[n + 1])
        t0 = time.perf_counter()
        oracle.gla_recurrent(q[s:e], k[s:e], v[s:e], g[s:e], np.array([0, e - s]), float(x["scale"]),
                             h0[n:n + 1], True)
        t_used += time.perf_counter() - t0
        done_tok += e - s
        runs += 1
    rate = done_tok / t_used / 1e6
    return {"value": rate, "unit": "Mtok/s", "cores": min(threads, H, os.cpu_count() or 1),
            "kind": "port",
            "sample": f"{runs} sequence runs ({runs / n_seq:.1f} passes over the 8 x 4096-token batch, "
                      f"{done_tok} tokens x {H} heads) of naive_gla_recurrent's fp64 C restatement, "
                      f"OpenMP over heads, {t_used:.1f} s",
            "host_cpus": os.cpu_count()}


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
    the C2 batch, two input sets alternating."""
    from ssla_amd import _lib, synthetic
    Tt, H, D = C2["B"] * C2["T"], C2["H"], C2["D"]
    sets = []
    for seed in (0, 1):
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
        launch(sets[i % 2])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        launch(sets[i % 2])
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


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--only", choices=["chunk", "sparse", "sparse_batched", "pool", "pool_sorted", "chunk_bwd", "event_stage"], default=None,
                    help="run one workload and print its line (profiling runs)")
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
    if args.only == "sparse":
        print(json.dumps(bench_sparse(torch, lib, args.steps, dev)), flush=True)
        return 0
    if args.only == "chunk_bwd":
        print(json.dumps(bench_chunk_bwd(torch, lib, args.steps, dev)), flush=True)
        return 0
    if args.only == "sparse_batched":
        print(json.dumps(bench_sparse_batched(torch, lib, args.steps, dev)), flush=True)
        return 0
    if args.only == "event_stage":
        print(json.dumps(bench_event_stage(torch, lib, args.steps, dev)), flush=True)
        return 0
    if args.only in ("pool", "pool_sorted"):
        print(json.dumps(bench_pool(torch, lib, args.steps, dev, args.only == "pool_sorted")), flush=True)
        return 0
    r = bench_chunk(torch, lib, args.steps, args.warmup, dev)
    ms_step = r["wall_s"] * 1e3 / args.steps
    value = r["tokens"] / (r["wall_s"] / args.steps) / 1e6
    kern_s = r["kernel_avg_ms"] * 1e-3
    alg_bytes = c2_bytes()
    achieved = alg_bytes / kern_s / 1e9
    traffic = _traffic_from_profile("gla_chunk_fwd_c2_pmc.txt")
    tflops = c2_flops() / kern_s / 1e12
    line = {
        "metric": "GLA chunk fwd Mtok/s (%bf16 MFMA peak); sparse scan site-steps/s (%HBM BW)",
        "value": value, "unit": "Mtok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "chunk_gla_fwd (config 2, C2): B=8, H=8, T=4096, K=V=64, chunk 64; "
                               "bf16 q/k/v/o, fp32 g/h0/ht; 2 input sets alternating (> MALL)",
                   "global_batch": C2["B"], "seq_len": C2["T"], "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "kernel": "ssla_gla_chunk_fwd (state + segment kernels, one call)",
                     "kernel_avg_us": r["kernel_avg_ms"] * 1e3,
                     "algorithmic_bytes": alg_bytes},
        "mfma": {"achieved": tflops, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                 "frac": tflops / BF16_PEAK_TFLOPS, "flops_per_launch": c2_flops(),
                 "note": "causal-useful flops; the shape is HBM-bound (31.8 flop/B < 312 ridge)"},
    }
    if not args.no_secondary and args.only is None:
        line["secondary"] = [bench_sparse(torch, lib, 10, dev), bench_sparse_batched(torch, lib, 10, dev),
                             bench_pool(torch, lib, 20, dev),
                             bench_pool(torch, lib, 20, dev, sorted_index=True), bench_chunk_bwd(torch, lib, 10, dev),
                             bench_event_stage(torch, lib, 5, dev)]
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(r["sample"])
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
