"""GPU parity of the asynchronous forward step (ssla_amd.backbone, the fifth
benchmark configuration) against its CPU restatement (oracle.backbone).

Every piece is checked on the GPU's own input to that piece, so a
difference is pinned to the piece that made it:
* preprocessing and pooling keys (times, lengths, sites) bit for bit; pooled
  features bit for bit when the pooled rows are the GPU's own (the max
  selects, it does not round);
* bf16 projections within bf16 rounding: RMS error ratio <= 2e-3 and every
  element within 2 bf16 ulps (2^-7 relative) plus 2e-3 of the RMS;
* the per-site recurrence on the GPU's q, k, v, g: o (rounded to bf16)
  within twice its measured error (RMS ratio 3.3e-3 against the north
  star's 2e-2, every element within 0.12 of the RMS), the fp32 states of the
  active sites at 1e-4, the states of every inactive site unchanged bit
  for bit;
* LayerNorm outputs and the bf16 detection head within twice their
  measured errors (RMS ratios 5e-5 and 3.5e-3).
The whole ``forward`` equals the piecewise run bit for bit (the kernels are
deterministic)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle import backbone as ob
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu


def _params(module):
    return {k: v.detach().float().cpu().numpy() for k, v in module.state_dict().items()}


def _np(x):
    return x.detach().float().cpu().numpy()


def _np_dict(d):
    """A grouped-events dict on the host: fp32 features, int64 keys."""
    out = {}
    for key, val in d.items():
        if torch.is_tensor(val):
            out[key] = _np(val) if key == "events" else val.cpu().numpy().astype(np.int64)
        else:
            out[key] = val
    return out


def _int_keys_equal(gpu, ref, what):
    for key in ("lengths", "time", "h", "w", "batch_id"):
        a, b = _np(gpu[key]).astype(np.int64), np.asarray(ref[key], np.int64)
        assert a.shape == b.shape and np.array_equal(a, b), f"{what}: {key} differs"


def _close_bf16(a, b, name):
    """bf16 GEMM results: 2 ulps elementwise plus 2e-3 of the RMS."""
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    rms = float(np.sqrt(np.mean(b * b))) if b.size else 0.0
    err = np.abs(a - b)
    bad = err > 2.0 ** -7 * np.abs(b) + 2e-3 * rms
    assert not bad.any(), f"{name}: {int(bad.sum())}/{bad.size} beyond 2 bf16 ulps; max err {err.max():.3g}"
    ratio = float(np.sqrt(np.mean(err * err)) / (rms + 1e-30)) if b.size else 0.0
    assert ratio <= 2e-3, f"{name}: RMS ratio {ratio:.3g}"


def _window_piecewise(model, ev, ln, states, params, dev, check_oracle=True, tag=""):
    from ssla_amd.scan import sparse_gla_scan
    frame = model.frame_size
    with torch.no_grad():
        x = model.stem(ev.to(dev), ln.to(dev))
    if check_oracle:
        rx = ob.stem(params, ev.numpy(), ln.numpy(), frame, model.stages[0][1])
        _int_keys_equal(x, rx, f"stem{tag}")
        _close_bf16(_np(x["events"]), rx["events"], f"stem events{tag}")
    feats = []
    for i, blk in enumerate(model.blocks):
        p = {k[len(f"blocks.{i}."):]: v for k, v in params.items() if k.startswith(f"blocks.{i}.")}
        grid = model.grid_sizes[i]
        before = states[i].clone()
        xe = x["events"].to(torch.float32)
        with torch.no_grad():
            q, k, v, g = blk.project(xe)
            cu = torch.nn.functional.pad(torch.cumsum(x["lengths"], 0), (1, 0))
            sites = blk.sites(x, grid)
            o = sparse_gla_scan(q, k, v, g, cu, sites, states[i], scale=blk.head_dim ** -0.5)
            y = blk.finish(o, xe)
        out = dict(x)
        out["events"] = y
        if check_oracle:
            xn = _np(xe)
            rq, rk, rv, rg = ob.block_project(p, xn, blk.heads, blk.head_dim)
            for nm, a, b in (("q", q, rq), ("k", k, rk), ("v", v, rv), ("g", g, rg)):
                _close_bf16(_np(a), b, f"stage {i} {nm}{tag}")
            ref_state = before.cpu().numpy()
            ro = ob.block_scan(_np(q), _np(k), _np(v), _np(g), _np(x["lengths"]).astype(np.int64),
                               _np(sites).astype(np.int64), ref_state, blk.head_dim ** -0.5)
            assert_close(_np(o), ro, 0.0, f"stage {i} o{tag}", band=0.12, ratio_max=3.3e-3)
            act = np.unique(_np(sites).astype(np.int64))
            inact = torch.from_numpy(np.setdiff1d(np.arange(states[i].shape[0]), act)).to(dev)
            assert torch.equal(states[i][inact], before[inact]), f"stage {i}: inactive states changed{tag}"
            assert_close(states[i].cpu().numpy()[act], ref_state[act], 1e-4, f"stage {i} states{tag}")
            ry = ob.block_finish(p, _np(o).astype(np.float64), xn)
            assert_close(_np(y), ry, 0.0, f"stage {i} out{tag}", band=0.033, ratio_max=5e-5)
        feats.append(out)
        if i < len(model.pools):
            with torch.no_grad():
                x = model.pools[i](out)
            if check_oracle:
                rp = ob.max_pool(_np_dict(out), grid, model.stages[i + 1][1] // model.stages[i][1])
                _int_keys_equal(x, rp, f"pool {i}{tag}")
                assert np.array_equal(_np(x["events"]), rp["events"]), f"pool {i} events{tag}"
    from ssla_amd import events as E
    with torch.no_grad():
        grids = [E.events_to_grid(feats[i], model.grid_sizes[i], model.stages[i][0]) for i in model.head_levels]
        out = model.head([gg.to(torch.bfloat16) for gg in grids])
    if check_oracle:
        for lvl, i in enumerate(model.head_levels):
            rg = oracle.events.event_to_grid(_np_dict(feats[i]), model.grid_sizes[i], model.stages[i][0])
            assert np.array_equal(_np(grids[lvl]), rg), f"grid {lvl}{tag}"
        hp = {k[5:]: v for k, v in params.items() if k.startswith("head.")}
        rh = ob.head(hp, [_np(gg) for gg in grids], [model.stages[i][1] for i in model.head_levels])
        assert_close(_np(out), rh, 0.0, f"head{tag}", band=0.024, ratio_max=3.5e-3)
    return out, feats


def test_async_step_windows_vs_oracle(dev):
    """Three consecutive windows of 5k events: every piece against the
    oracle, states carried from window to window (so later windows start
    from non-zero states), and forward() == the piecewise run."""
    import oracle.events  # noqa: F401
    from ssla_amd import synthetic
    from ssla_amd.backbone import AsyncSparseGLA
    torch.manual_seed(0)
    model = AsyncSparseGLA().to(dev)
    params = _params(model)
    states = model.init_states(1, dev)
    for w, ev in enumerate(synthetic.async_windows(3, 5000, seed=1)):
        ln = torch.tensor([ev.shape[1]])
        print(f"async step window {w}: {ev.shape[1]} events", flush=True)
        states_fwd = [s.clone() for s in states]
        out, _ = _window_piecewise(model, ev, ln, states, params, dev, tag=f" w{w}")
        with torch.no_grad():
            out_f, _ = model(ev.to(dev), ln.to(dev), states_fwd)
        assert torch.equal(out_f, out), f"forward() differs from the piecewise run in window {w}"
        for i in range(4):
            assert torch.equal(states_fwd[i], states[i]), f"forward() states differ (stage {i}, window {w})"


def test_async_step_full_window_vs_oracle(dev):
    """Config 5 at full size: two consecutive 50k-event windows, every piece
    against the oracle on the GPU's own input to it (the same checks as the
    5k-event windows), states carried, and forward() == the piecewise run."""
    import oracle.events  # noqa: F401
    from ssla_amd import synthetic
    from ssla_amd.backbone import AsyncSparseGLA
    torch.manual_seed(3)
    model = AsyncSparseGLA().to(dev)
    params = _params(model)
    states = model.init_states(1, dev)
    for w, ev in enumerate(synthetic.async_windows(2, 50_000, seed=4)):
        ln = torch.tensor([ev.shape[1]])
        print(f"async step full window {w}: {ev.shape[1]} events", flush=True)
        states_fwd = [s.clone() for s in states]
        out, _ = _window_piecewise(model, ev, ln, states, params, dev, tag=f" full w{w}")
        with torch.no_grad():
            out_f, _ = model(ev.to(dev), ln.to(dev), states_fwd)
        assert torch.equal(out_f, out), f"forward() differs from the piecewise run in full window {w}"
        for i in range(4):
            assert torch.equal(states_fwd[i], states[i]), f"forward() states differ (stage {i}, full window {w})"


def test_async_step_full_size_properties(dev):
    """Four windows of 50k events at full size: head output [1, 1505, 7]
    and finite, every state row either unchanged (inactive site) or
    changed, stage outputs unit-scale (LayerNorm), and a rerun from the same
    states is bit-identical."""
    from ssla_amd import synthetic
    from ssla_amd.backbone import AsyncSparseGLA
    torch.manual_seed(1)
    model = AsyncSparseGLA().to(dev)
    states = model.init_states(1, dev)
    for w, ev in enumerate(synthetic.async_windows(4, 50_000, seed=2)):
        ln = torch.tensor([ev.shape[1]], device=dev)
        print(f"async step full size window {w}", flush=True)
        prev = [s.clone() for s in states]
        with torch.no_grad():
            out, feats = model(ev.to(dev), ln, states)
            again = [p.clone() for p in prev]
            out2, feats2 = model(ev.to(dev), ln, again)
        assert out.shape == (1, 30 * 38 + 15 * 19 + 8 * 10, 7) and torch.isfinite(out.float()).all()
        for i in range(4):
            assert torch.equal(feats[i]["events"], feats2[i]["events"]), f"stage {i} output differs on a rerun"
            assert torch.equal(again[i], states[i]), f"stage {i} states differ on a rerun"
        assert torch.equal(out, out2), "head output differs on a rerun"
        for i, f in enumerate(feats):
            sites = ((f["batch_id"] * model.grid_sizes[i][0] + f["h"]) * model.grid_sizes[i][1] + f["w"]).long()
            assert bool((sites[1:] > sites[:-1]).all()), f"stage {i}: site list not strictly increasing"
            changed = (states[i] != prev[i]).flatten(1).any(1)
            mask = torch.zeros_like(changed)
            mask[sites] = True
            assert not bool((changed & ~mask).any()), f"stage {i}: an inactive state changed"
            assert bool(changed[sites].all()), f"stage {i}: an active state did not change"
            y = f["events"]
            assert torch.isfinite(y).all()
            assert abs(float(y.mean())) < 0.1 and 0.8 < float(y.std()) < 1.2


def test_async_plan_then_forward_matches(dev):
    """plan() of every window first, then forward(plan=...) window by
    window: outputs, pooled structure and carried states equal forward()
    that plans each window itself, bit for bit, over three 50k-event
    windows."""
    from ssla_amd import synthetic
    from ssla_amd.backbone import AsyncSparseGLA
    torch.manual_seed(5)
    model = AsyncSparseGLA().to(dev).eval()
    wins = [w.to(dev) for w in synthetic.async_windows(3, 50_000, seed=6)]
    ln = torch.tensor([50_000], device=dev)
    print("async plan then forward", flush=True)
    with torch.no_grad():
        s_seq = model.init_states(1, dev)
        seq = [model(w, ln, s_seq) for w in wins]
        plans = [model.plan(w, ln) for w in wins]
        s_pl = model.init_states(1, dev)
        got = [model(w, ln, s_pl, plan=p) for w, p in zip(wins, plans)]
    for w, ((o1, f1), (o2, f2)) in enumerate(zip(seq, got)):
        assert torch.equal(o1, o2), f"window {w}: head output differs"
        for i in range(4):
            assert torch.equal(f1[i]["events"], f2[i]["events"]), f"window {w} stage {i}: events differ"
            for key in ("time", "lengths", "batch_id", "h", "w"):
                assert torch.equal(f1[i][key], f2[i][key]), f"window {w} stage {i}: {key} differs"
    for i in range(4):
        assert torch.equal(s_seq[i], s_pl[i]), f"stage {i}: carried states differ"


def test_async_run_matches_forward(dev):
    """run() over four 50k-event windows (each window planned step by step
    while the previous one's stages run, counts copied back without
    draining the stream) equals forward() window by window, bit for bit:
    head outputs, every stage's events and structure, the carried states;
    a second run() on the same states continues them the same way."""
    from ssla_amd import synthetic
    from ssla_amd.backbone import AsyncSparseGLA
    torch.manual_seed(7)
    model = AsyncSparseGLA().to(dev).eval()
    wins = [w.to(dev) for w in synthetic.async_windows(6, 50_000, seed=8)]
    lns = [torch.tensor([50_000], device=dev)] * len(wins)
    print("async run vs forward", flush=True)
    with torch.no_grad():
        s_seq = model.init_states(1, dev)
        seq = [model(w, ln, s_seq) for w, ln in zip(wins, lns)]
        s_run = model.init_states(1, dev)
        got = model.run(wins[:4], lns[:4], s_run) + model.run(wins[4:], lns[4:], s_run)
        assert model.run([], [], s_run) == []
    assert len(got) == len(seq)
    for w, ((o1, f1), (o2, f2)) in enumerate(zip(seq, got)):
        assert torch.equal(o1, o2), f"window {w}: head output differs"
        for i in range(4):
            for key in ("events", "time", "lengths", "batch_id", "h", "w"):
                assert torch.equal(f1[i][key], f2[i][key]), f"window {w} stage {i}: {key} differs"
    for i in range(4):
        assert torch.equal(s_seq[i], s_run[i]), f"stage {i}: carried states differ"


def test_async_run_batched_ragged(dev):
    """run() on windows of two samples with different lengths (the padded
    [B, N, 4] batch the reference collates, padding rows never read) equals
    forward() window by window, bit for bit, states included."""
    from ssla_amd import synthetic
    from ssla_amd.backbone import AsyncSparseGLA
    torch.manual_seed(9)
    model = AsyncSparseGLA().to(dev).eval()
    a = synthetic.async_windows(3, 30_000, seed=10)
    b = synthetic.async_windows(3, 30_000, seed=11)
    wins, lns = [], []
    for i, (wa, wb) in enumerate(zip(a, b)):
        na, nb = 30_000 - 4_000 * i, 21_000 + 3_000 * i
        w = torch.full((2, 30_000, 4), -7.0)   # padding rows hold junk
        w[0, :na], w[1, :nb] = wa[0, :na], wb[0, :nb]
        wins.append(w.to(dev))
        lns.append(torch.tensor([na, nb], device=dev))
    print("async run batched ragged", flush=True)
    with torch.no_grad():
        s_seq = model.init_states(2, dev)
        seq = [model(w, ln, s_seq) for w, ln in zip(wins, lns)]
        s_run = model.init_states(2, dev)
        got = model.run(wins, lns, s_run)
    for w, ((o1, f1), (o2, f2)) in enumerate(zip(seq, got)):
        assert torch.equal(o1, o2), f"window {w}: head output differs"
        for i in range(4):
            for key in ("events", "time", "lengths", "batch_id", "h", "w"):
                assert torch.equal(f1[i][key], f2[i][key]), f"window {w} stage {i}: {key} differs"
    for i in range(4):
        assert torch.equal(s_seq[i], s_run[i]), f"stage {i}: carried states differ"


def test_pool_plan_halves_match_plan(dev):
    """ssla_sparse_pool_plan_enqueue + an asynchronous copy of the counts +
    ssla_sparse_pool_plan_finish give the plan, structure and pooled values
    of ssla_sparse_pool_plan, for runs sorted by time (the counting fill)
    and for runs that are not (the sort fill inside the finish), and report
    out-of-range coordinates the same way."""
    from ssla_amd import events as E
    from ssla_amd.layers import SparseMaxPool
    torch.manual_seed(3)
    frame = (24, 30)
    pool = SparseMaxPool(frame, kernel_size=(3, 3), stride=(2, 2)).to(dev)
    print("pool plan halves", flush=True)
    for sort_times in (True, False):
        G, B = 200, 2
        cells = torch.randperm(frame[0] * frame[1] * B)[:G].sort().values
        lengths = torch.randint(1, 6, (G,))
        E_in = int(lengths.sum())
        times = torch.randint(0, 40, (E_in,))
        if sort_times:   # every pixel run sorted by time
            starts = torch.cumsum(lengths, 0) - lengths
            times = torch.cat([times[s:s + n].sort().values for s, n in zip(starts.tolist(), lengths.tolist())])
        inputs = {"batch_id": (cells // (frame[0] * frame[1])).to(dev),
                  "h": ((cells % (frame[0] * frame[1])) // frame[1]).to(dev),
                  "w": (cells % frame[1]).to(dev), "lengths": lengths.to(dev), "time": times.to(dev),
                  "batch_size": B}
        ev = torch.randn(E_in, 16, device=dev)
        with torch.no_grad():
            ref = pool.plan(dict(inputs))
            ref_out = pool.apply_plan(ref, ev)
            got = pool.plan_finish(pool.plan_enqueue(dict(inputs)))
            got_out = pool.apply_plan(got, ev)
        assert (ref.n_act, ref.n_seg, ref.E_out) == (got.n_act, got.n_seg, got.E_out)
        for key in ("events", "time", "lengths", "batch_id", "h", "w"):
            assert torch.equal(ref_out[key], got_out[key]), f"sorted={sort_times}: {key} differs"
    bad = dict(inputs, h=inputs["h"] + frame[0])
    with torch.no_grad(), pytest.raises(ValueError):
        pool.plan_finish(pool.plan_enqueue(bad))


def test_head_kernel_matches_module(dev):
    """ssla_detect_head (all levels in one kernel, fp32 between its two bf16
    GEMMs) against the module's bf16 ops run one by one and against the fp64
    oracle, on random maps: closer to the oracle than the module is (it
    rounds after every op), and within the module's own rounding of it; a
    weight updated in place is seen by the next call."""
    from ssla_amd.backbone import AsyncSparseGLA
    torch.manual_seed(4)
    model = AsyncSparseGLA().to(dev)
    head = model.head
    shapes = [(1, model.stages[i][0], *model.grid_sizes[i]) for i in model.head_levels]
    strides = [model.stages[i][1] for i in model.head_levels]
    gen = torch.Generator(device=dev).manual_seed(9)
    for rep in range(3):
        if rep == 2:
            with torch.no_grad():
                head.cls_preds[0].bias.add_(0.5)   # in place: the folded parameters are rebuilt
        xin = [torch.randn(s, device=dev, generator=gen) for s in shapes]
        print(f"head kernel check {rep}", flush=True)
        with torch.no_grad():
            got = head(xin)
            eager = head(xin, fused=False)
        hp = {k: v.detach().float().cpu().numpy() for k, v in head.state_dict().items()}
        ref = ob.head(hp, [_np(x) for x in xin], strides)
        e_got = np.sqrt(np.mean((_np(got) - ref) ** 2))
        e_eager = np.sqrt(np.mean((_np(eager) - ref) ** 2))
        assert e_got <= e_eager * 1.05, f"rep {rep}: kernel rms error {e_got:.3g} vs module {e_eager:.3g}"
        assert_close(_np(got), ref, 0.0, f"head kernel rep {rep}", band=0.024, ratio_max=3.5e-3)
        assert_close(_np(got), _np(eager), 0.0, f"head kernel vs module rep {rep}", band=0.05, ratio_max=7e-3)


def test_head_outside_kernel_sizes_runs_module(dev):
    """A head the kernel does not take (80 classes: 85 outputs) runs the
    module's ops instead of raising, with the oracle's decode."""
    from ssla_amd.backbone import DetectionHead
    torch.manual_seed(5)
    head = DetectionHead(80, (8, 16), (64, 128), 64).to(dev).to(torch.bfloat16).eval()
    gen = torch.Generator(device=dev).manual_seed(2)
    xin = [torch.randn(1, 64, 6, 8, device=dev, generator=gen), torch.randn(1, 128, 3, 4, device=dev, generator=gen)]
    print("head with 80 classes", flush=True)
    with torch.no_grad():
        got = head(xin)
        eager = head(xin, fused=False)
    assert got.shape == (1, 6 * 8 + 3 * 4, 85)
    assert torch.equal(got, eager)
    hp = {k: v.detach().float().cpu().numpy() for k, v in head.state_dict().items()}
    ref = ob.head(hp, [_np(x) for x in xin], (8, 16))
    assert_close(_np(got), ref, 2 ** -7, "80-class head vs oracle", band=0.05, ratio_max=1e-2)


def test_site_block_kernels_match_torch(dev):
    """ssla_site_project / ssla_site_finish against the same block run as
    torch's bf16 F.linear calls (the rounding points the kernels follow) for
    every stage shape of the step: the bf16 outputs within one bf16 unit of
    rounding (fp32 sums in another order can move a rounding), the gates and
    the LayerNorm outputs within 1e-3 of their RMS."""
    from ssla_amd.backbone import AsyncSparseGLA
    torch.manual_seed(5)
    model = AsyncSparseGLA().to(dev)
    gen = torch.Generator(device=dev).manual_seed(6)
    for i, blk in enumerate(model.blocks):
        n = 3001 + 17 * i
        x = torch.randn(n, blk.in_channels, device=dev, generator=gen)
        print(f"site block kernels stage {i}: {blk.in_channels} -> {blk.out_channels}", flush=True)
        with torch.no_grad():
            q, k, v, g = blk.project(x)
            o = (torch.randn(n, blk.heads * blk.head_dim, device=dev, generator=gen) * 0.3).to(torch.bfloat16)
            y = blk.finish(o.view(n, blk.heads, blk.head_dim), x)
            xb = x.to(torch.bfloat16)
            w = {nm: getattr(blk, f"{nm}_proj").weight.to(torch.bfloat16) for nm in ("q", "k", "v", "g", "o")}
            ref = [F.linear(xb, w[nm]).view(q.shape) for nm in ("q", "k", "v")]
            rg = (F.logsigmoid(F.linear(xb, w["g"]).float()) / blk.gate_normalizer).view(g.shape)
            ry = F.linear(o, w["o"]).float()
            ry = ry + (F.linear(xb, blk.res_proj.weight.to(torch.bfloat16)).float() if blk.res_proj is not None else x)
            ry = blk.norm(ry)
        for nm, a, b in zip("qkv", (q, k, v), ref):
            a, b = _np(a), _np(b)
            assert np.all(np.abs(a - b) <= 2.0 ** -8 * np.abs(b) + 1e-30), f"stage {i} {nm}: beyond one bf16 unit"
        assert_close(_np(g), _np(rg), 0.0, f"stage {i} g", band=1e-3, ratio_max=1e-3)
        assert_close(_np(y), _np(ry), 0.0, f"stage {i} y", band=1e-3, ratio_max=1e-3)


def test_site_block_one_call_checks(dev):
    """ssla_site_gla_block: equal to the composed block bit for bit (y and the
    states); with check=True a site list that is not strictly increasing
    raises ValueError after the call and leaves those sequences' states
    untouched; a state of the wrong shape is refused before any launch."""
    from ssla_amd.backbone import AsyncSparseGLA
    torch.manual_seed(7)
    model = AsyncSparseGLA().to(dev)
    blk, grid = model.blocks[1], model.grid_sizes[1]
    gen = torch.Generator(device=dev).manual_seed(3)
    G = 200
    cells = torch.randperm(grid[0] * grid[1], generator=gen, device=dev)[:G].sort().values
    lengths = torch.randint(1, 9, (G,), generator=gen, device=dev)
    n = int(lengths.sum())
    x = {"events": torch.randn(n, blk.in_channels, device=dev, generator=gen), "lengths": lengths,
         "batch_id": torch.zeros(G, dtype=torch.int64, device=dev), "h": cells // grid[1], "w": cells % grid[1],
         "time": torch.zeros(n, dtype=torch.int64, device=dev), "batch_size": 1}
    st0 = torch.randn(grid[0] * grid[1], blk.heads, blk.head_dim, blk.head_dim, device=dev, generator=gen) * 0.1
    s1, s2 = st0.clone(), st0.clone()
    with torch.no_grad():
        one = blk(x, s1, grid, check=True)
        comp = blk(x, s2, grid, check=True, mark=lambda name: None)   # the composed path
    assert torch.equal(one["events"], comp["events"]) and torch.equal(s1, s2)
    bad = dict(x)
    bad["w"] = x["w"].clone()
    bad["h"] = x["h"].clone()
    bad["h"][5], bad["w"][5] = bad["h"][4], bad["w"][4]   # a repeated site
    s3 = st0.clone()
    with torch.no_grad(), pytest.raises(ValueError):
        blk(bad, s3, grid, check=True)
    # the bad sequence (index 5) is skipped: the cell it originally named is
    # untouched, its repeated cell holds sequence 4's update only, and every
    # other row is what the good call wrote
    c5 = int(cells[5])
    assert torch.equal(s3[c5], st0[c5]), "the skipped sequence's original cell changed"
    keep = torch.ones(st0.shape[0], dtype=torch.bool, device=dev)
    keep[c5] = False
    assert torch.equal(s3[keep], s1[keep]), "rows of the valid sequences differ from the good call"
    with torch.no_grad(), pytest.raises(ValueError):
        blk(x, st0[:, :, :16].contiguous(), grid)
