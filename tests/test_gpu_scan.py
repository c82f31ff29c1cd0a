"""GPU parity: varlen diagonal scan (reference ops/common/scan.py:20-43) and
the per-site sparse GLA step / batched sparse scan, vs the CPU oracle.
fp32 throughout: rtol 1e-4 (north star); inactive sites bit-exact."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("C", [1, 3, 12, 24, 48, 64, 96, 200, 256])
def test_scan_matches_oracle(dev, C):
    from ssla_amd.scan import scan
    gen = torch.Generator().manual_seed(C)
    lens = [5, 0, 1, 33, 8, 120, 2]
    # leading and trailing rows outside every sequence must come back zero
    cu = torch.tensor(np.concatenate([[3], 3 + np.cumsum(lens)]), dtype=torch.int64)
    T = int(cu[-1]) + 4
    u = torch.randn(T, C, generator=gen)
    g = torch.sigmoid(torch.randn(T, C, generator=gen))
    with torch.no_grad():
        h = scan(u.to(dev), g.to(dev), cu.to(dev)).cpu().numpy()
    ref = oracle.diag_scan(u.numpy(), g.numpy(), cu.numpy())
    assert_close(h, ref, 1e-5, f"scan C={C}")
    assert (h[:3] == 0).all() and (h[-4:] == 0).all()


@pytest.mark.parametrize("C", [1, 3, 24, 64, 100, 256])
def test_scan_backward_matches_oracle(dev, C):
    """SequentialScan.backward (reference ops/common/scan.py:55-86, 116-137)
    through torch autograd: du, dg vs the fp64 oracle; rows in no sequence
    get zero gradients."""
    from ssla_amd.scan import scan
    gen = torch.Generator().manual_seed(100 + C)
    lens = [5, 0, 1, 33, 8, 1200, 2, 17]
    cu = torch.tensor(np.concatenate([[3], 3 + np.cumsum(lens)]), dtype=torch.int64)
    T = int(cu[-1]) + 4
    u = torch.randn(T, C, generator=gen)
    g = torch.sigmoid(torch.randn(T, C, generator=gen) + 2)
    w = torch.randn(T, C, generator=gen)
    ud, gd = u.to(dev).requires_grad_(), g.to(dev).requires_grad_()
    h = scan(ud, gd, cu.to(dev))
    (h * w.to(dev)).sum().backward()
    rdu, rdg = oracle.diag_scan_bwd(u.numpy(), g.numpy(), w.numpy(), cu.numpy())
    du, dg = ud.grad.cpu().numpy(), gd.grad.cpu().numpy()
    assert_close(du, rdu, 1e-5, f"du C={C}")
    assert_close(dg, rdg, 1e-5, f"dg C={C}")
    assert (du[:3] == 0).all() and (dg[-4:] == 0).all()


def test_scan_backward_layer_shapes(dev):
    """Many short sequences (one per active patch), C = 48."""
    from ssla_amd.scan import scan
    rng = np.random.default_rng(1)
    lens = rng.integers(1, 40, size=3000)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64)
    T = int(cu[-1])
    u = torch.from_numpy(rng.standard_normal((T, 48)).astype(np.float32))
    g = torch.sigmoid(torch.from_numpy(rng.standard_normal((T, 48)).astype(np.float32)))
    w = torch.from_numpy(rng.standard_normal((T, 48)).astype(np.float32))
    ud, gd = u.to(dev).requires_grad_(), g.to(dev).requires_grad_()
    (scan(ud, gd, cu.to(dev)) * w.to(dev)).sum().backward()
    rdu, rdg = oracle.diag_scan_bwd(u.numpy(), g.numpy(), w.numpy(), cu.numpy())
    assert_close(ud.grad.cpu().numpy(), rdu, 1e-5, "du")
    assert_close(gd.grad.cpu().numpy(), rdg, 1e-5, "dg")


def test_scan_layer_shapes(dev):
    """Many short sequences, as MosAttention produces (one per active patch)."""
    from ssla_amd.scan import scan
    rng = np.random.default_rng(0)
    lens = rng.integers(1, 40, size=3000)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64)
    T = int(cu[-1])
    u = torch.from_numpy(rng.standard_normal((T, 48)).astype(np.float32))
    g = torch.sigmoid(torch.from_numpy(rng.standard_normal((T, 48)).astype(np.float32)))
    with torch.no_grad():
        h = scan(u.to(dev), g.to(dev), cu.to(dev)).cpu().numpy()
    assert_close(h, oracle.diag_scan(u.numpy(), g.numpy(), cu.numpy()), 1e-5, "scan")


def test_sparse_step_c3_bins(dev):
    """Config 3 (C3: 76x60 sites, H=4, D=32) at full size, all 64 bins: o
    checked after every bin against the oracle, inactive states
    bit-identical in every bin, all states against the oracle at the end."""
    from ssla_amd import synthetic
    from ssla_amd.scan import sparse_gla_step
    sb = synthetic.sparse_scan_bins()
    assert len(sb.sites) == 64
    st_gpu = sb.state0.clone().to(dev)
    st_ref = sb.state0.numpy().copy()
    print("C3 per-bin steps, 64 bins", flush=True)
    for b in range(64):
        sites = sb.sites[b]
        prev = st_gpu.clone()
        with torch.no_grad():
            o = sparse_gla_step(torch.from_numpy(sites).to(dev), sb.q[b].to(dev), sb.k[b].to(dev),
                                sb.v[b].to(dev), sb.g[b].to(dev), st_gpu, scale=sb.scale)
        ro = oracle.sparse_gla_step(sites, sb.q[b].numpy(), sb.k[b].numpy(), sb.v[b].numpy(),
                                    sb.g[b].numpy(), st_ref, sb.scale)
        assert_close(o.cpu().numpy(), ro, 1e-4, f"o bin {b}")
        inactive = np.setdiff1d(np.arange(sb.n_sites), sites)
        inact = torch.from_numpy(inactive).to(dev)
        assert torch.equal(st_gpu[inact], prev[inact]), f"inactive states changed in bin {b}"
    assert_close(st_gpu.cpu().numpy(), st_ref, 1e-4, "states")


def test_sparse_scan_c3_full_vs_oracle(dev):
    """Config 3 at full size through the one-call path (all 64 bins as one
    ssla_gla_recurrent_fwd with state_idx, the bench's batched line): the
    rows regrouped by site (stable in time), o and the updated states
    against the oracle recurrence from each site's stored state, and every
    state row of a site that was never active bit-identical."""
    from ssla_amd import synthetic
    from ssla_amd.scan import sparse_gla_scan
    sb = synthetic.sparse_scan_bins()
    site_all = np.concatenate(sb.sites)
    order = np.argsort(site_all, kind="stable")
    uniq, counts = np.unique(site_all[order], return_counts=True)
    cu = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    cat = lambda xs: torch.cat(xs)[torch.from_numpy(order)]   # noqa: E731
    q, k, v, g = cat(sb.q), cat(sb.k), cat(sb.v), cat(sb.g)
    st = sb.state0.clone().to(dev)
    print(f"C3 one call: {len(uniq)} sites, {int(cu[-1])} site-steps", flush=True)
    with torch.no_grad():
        o = sparse_gla_scan(q.to(dev), k.to(dev), v.to(dev), g.to(dev), torch.from_numpy(cu).to(dev),
                            torch.from_numpy(uniq.astype(np.int32)).to(dev), st, scale=sb.scale, check=True)
    ro, rht = oracle.gla_recurrent(q.numpy(), k.numpy(), v.numpy(), g.numpy(), cu, sb.scale,
                                   sb.state0.numpy()[uniq], True)
    assert_close(o.cpu().numpy(), ro, 1e-4, "o (one call, 64 bins)")
    st = st.cpu()
    assert_close(st.numpy()[uniq], rht, 1e-4, "states of the active sites")
    never = np.setdiff1d(np.arange(sb.n_sites), uniq)
    assert torch.equal(st[torch.from_numpy(never)], sb.state0[torch.from_numpy(never)]), \
        "states of sites never active changed"


def test_sparse_scan_matches_steps(dev):
    """Batched multi-bin form == bin-by-bin steps (same site histories)."""
    from ssla_amd import synthetic
    from ssla_amd.scan import sparse_gla_scan, sparse_gla_step
    sb = synthetic.sparse_scan_bins(n_bins=12, seed=3)
    st_a = sb.state0.clone().to(dev)
    outs = []
    with torch.no_grad():
        for b in range(12):
            outs.append(sparse_gla_step(torch.from_numpy(sb.sites[b]).to(dev), sb.q[b].to(dev),
                                        sb.k[b].to(dev), sb.v[b].to(dev), sb.g[b].to(dev), st_a,
                                        scale=sb.scale))
    # regroup rows by site (stable in time) for the batched call
    site_all = np.concatenate(sb.sites)
    order = np.argsort(site_all, kind="stable")
    uniq, counts = np.unique(site_all[order], return_counts=True)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int64)
    cat = lambda xs: torch.cat(xs)[torch.from_numpy(order)]
    st_b = sb.state0.clone().to(dev)
    with torch.no_grad():
        o_b = sparse_gla_scan(cat(sb.q).to(dev), cat(sb.k).to(dev), cat(sb.v).to(dev),
                              cat(sb.g).to(dev), cu.to(dev), torch.from_numpy(uniq).to(dev), st_b,
                              scale=sb.scale)
    o_a = torch.cat(outs)[torch.from_numpy(order).to(dev)]
    assert_close(o_b.cpu().numpy(), o_a.cpu().numpy(), 1e-4, "o")
    assert_close(st_b.cpu().numpy(), st_a.cpu().numpy(), 1e-4, "state")


def test_sparse_step_graph_replay(dev):
    """The per-bin pass (one ssla_sparse_gla_step launch per bin) captured as
    one HIP graph: every replay, with eager work and synchronisations between
    replays, reproduces the eager pass bit for bit (states and outputs)."""
    from ssla_amd import _lib, synthetic
    lib = _lib.load()
    sb = synthetic.sparse_scan_bins(n_bins=12, seed=4)
    bins = [dict(s=torch.from_numpy(sb.sites[b]).to(dev), q=sb.q[b].to(dev), k=sb.k[b].to(dev),
                 v=sb.v[b].to(dev), g=sb.g[b].to(dev), o=torch.empty(sb.sites[b].size, 4, 32, device=dev))
            for b in range(12)]
    state0 = sb.state0.to(dev).contiguous()
    state = state0.clone()

    def one_pass(sh):
        for x in bins:
            _lib.check(lib.ssla_sparse_gla_step(x["s"].data_ptr(), x["s"].numel(), x["q"].data_ptr(),
                                                x["k"].data_ptr(), x["v"].data_ptr(), x["g"].data_ptr(),
                                                state.data_ptr(), sb.n_sites, 4, 32, 32, float(sb.scale),
                                                x["o"].data_ptr(), None, sh), "sparse_gla_step")

    one_pass(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    st_e, o_e = state.clone(), [x["o"].clone() for x in bins]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        state.copy_(state0)
        one_pass(side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        one_pass(torch.cuda.current_stream().cuda_stream)
    for rep in range(3):
        state.copy_(state0)
        for x in bins:
            x["o"].fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"graph replay {rep}", flush=True)
        assert torch.equal(state, st_e), f"state differs on replay {rep}"
        for b, x in enumerate(bins):
            assert torch.equal(x["o"], o_e[b]), f"o of bin {b} differs on replay {rep}"


def test_sparse_step_rejects_bad_site_lists(dev):
    """An out-of-range site and a duplicate are reported (ValueError from
    the wrapper, SSLA_ERR_ARG in the status word through the C-ABI); their o
    rows are zero, no state they name changes, and the valid entries are
    updated as usual."""
    from ssla_amd import _lib
    from ssla_amd.scan import sparse_gla_step
    gen = torch.Generator().manual_seed(31)
    n_sites, H, K, V = 50, 2, 32, 32
    state0 = torch.randn(n_sites, H, K, V, generator=gen) * 0.1
    sites = np.array([3, 7, 7, 12, 60], dtype=np.int32)   # duplicate 7, out-of-range 60
    n = sites.size
    q, k, v = (torch.randn(n, H, D, generator=gen) for D in (K, K, V))
    g = F.logsigmoid(torch.randn(n, H, K, generator=gen))
    st = state0.clone().to(dev)
    print("sparse step: bad site list through the wrapper", flush=True)
    with torch.no_grad(), pytest.raises(ValueError, match="strictly increasing"):
        sparse_gla_step(torch.from_numpy(sites).to(dev), q.to(dev), k.to(dev), v.to(dev), g.to(dev), st, check=True)
    # the same call through the C-ABI: status word, zero rows, state effects
    lib = _lib.load()
    st = state0.clone().to(dev)
    o = torch.full((n, H, V), float("nan"), device=dev)
    status = _lib.new_status(dev)
    qd, kd, vd, gd = (t.to(dev).contiguous() for t in (q, k, v, g))
    sd = torch.from_numpy(sites).to(dev)
    _lib.check(lib.ssla_sparse_gla_step(sd.data_ptr(), n, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                        gd.data_ptr(), st.data_ptr(), n_sites, H, K, V, K ** -0.5,
                                        o.data_ptr(), status.data_ptr(), _lib.stream_of(qd)), "step")
    assert _lib.read_status(status) == _lib.SSLA_ERR_ARG
    o = o.cpu()
    assert torch.equal(o[2], torch.zeros(H, V)) and torch.equal(o[4], torch.zeros(H, V))
    ref_state = state0.numpy().copy()
    good = [0, 1, 3]
    ro = oracle.sparse_gla_step(sites[good], q.numpy()[good], k.numpy()[good], v.numpy()[good],
                                g.numpy()[good], ref_state, K ** -0.5)
    assert_close(o.numpy()[good], ro, 1e-4, "o of the valid entries")
    assert_close(st.cpu().numpy(), ref_state, 1e-4, "states (site 7 updated once)")


def test_sparse_scan_rejects_bad_site_lists(dev):
    """sparse_gla_scan (ssla_gla_recurrent_fwd with state_idx): a repeated
    site is reported and its sequence skipped (zero o rows)."""
    from ssla_amd import _lib
    from ssla_amd.gla import _recurrent
    from ssla_amd.scan import sparse_gla_scan
    gen = torch.Generator().manual_seed(32)
    H, K, V, n_sites = 2, 32, 32, 20
    lens = [3, 2, 4]
    T = sum(lens)
    q, k, v = (torch.randn(T, H, D, generator=gen).to(dev) for D in (K, K, V))
    g = F.logsigmoid(torch.randn(T, H, K, generator=gen)).to(dev)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64, device=dev)
    state0 = (torch.randn(n_sites, H, K, V, generator=gen) * 0.1).to(dev)
    print("sparse scan: repeated site", flush=True)
    with torch.no_grad(), pytest.raises(ValueError, match="strictly increasing"):
        sparse_gla_scan(q, k, v, g, cu, torch.tensor([4, 9, 9], device=dev), state0.clone(), check=True)
    st = state0.clone()
    o = torch.full((T, H, V), float("nan"), device=dev)
    status = _lib.new_status(dev)
    with torch.no_grad():
        _recurrent(q, k, v, g, cu, K ** -0.5, st, o, st, torch.tensor([4, 9, 9], device=dev, dtype=torch.int32),
                   n_sites, status)
    assert _lib.read_status(status) == _lib.SSLA_ERR_ARG
    assert torch.equal(o[5:].cpu(), torch.zeros(4, H, V))
    assert torch.isfinite(o[:5]).all()
    untouched = [i for i in range(n_sites) if i not in (4, 9)]
    assert torch.equal(st[untouched], state0[untouched])


@pytest.mark.parametrize("bad", ["repeat", "range"])
def test_sparse_scan_rejects_bad_site_lists_segmented(dev, bad):
    """The segmented schedule (long histories: the workspace query is
    non-zero) with a repeated or out-of-range site: SSLA_ERR_ARG in the
    status word, every o row of the bad sequence's segments zero, the states
    of the bad entry untouched, and the valid sequences against the
    oracle."""
    from ssla_amd import _lib
    from ssla_amd.gla import _recurrent
    gen = torch.Generator().manual_seed(33)
    H, K, V, n_sites = 2, 32, 32, 12
    lens = [700, 300, 1000]
    sites = [2, 5, 5] if bad == "repeat" else [2, 5, 40]
    T = sum(lens)
    assert _lib.load().ssla_gla_recurrent_workspace_size(len(lens), T, H, K, V) > 0
    q, k, v = (torch.randn(T, H, D, generator=gen) for D in (K, K, V))
    g = F.logsigmoid(torch.randn(T, H, K, generator=gen) / 4)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64)
    state0 = torch.randn(n_sites, H, K, V, generator=gen) * 0.1
    st = state0.clone().to(dev)
    o = torch.full((T, H, V), float("nan"), device=dev)
    status = _lib.new_status(dev)
    print(f"sparse scan segmented, bad site list ({bad})", flush=True)
    with torch.no_grad():
        _recurrent(q.to(dev), k.to(dev), v.to(dev), g.to(dev), cu.to(dev), K ** -0.5, st, o, st,
                   torch.tensor(sites, device=dev, dtype=torch.int32), n_sites, status)
    assert _lib.read_status(status) == _lib.SSLA_ERR_ARG
    o = o.cpu()
    assert torch.equal(o[1000:], torch.zeros(1000, H, V)), "o rows of the bad sequence must be zero"
    ro, rht = oracle.gla_recurrent(q.numpy()[:1000], k.numpy()[:1000], v.numpy()[:1000], g.numpy()[:1000],
                                   np.array([0, 700, 1000]), K ** -0.5, state0.numpy()[[2, 5]], True)
    assert_close(o.numpy()[:1000], ro, 1e-4, "o of the valid sequences")
    st = st.cpu()
    assert_close(st.numpy()[[2, 5]], rht, 1e-4, "states of the valid sequences")
    others = [i for i in range(n_sites) if i not in (2, 5)]
    assert torch.equal(st[others], state0[others]), "rows outside the valid sequences changed"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sparse_scan_long_sequences_in_place(dev, dtype):
    """Long and ragged per-site histories (the segmented schedule: 128-step
    segments folded into each other, and an in-place state table that the
    last segment overwrites while the first reads it from the copy): o and
    the updated states against the oracle, other rows untouched bit for
    bit."""
    from ssla_amd import _lib
    from ssla_amd.scan import sparse_gla_scan
    gen = torch.Generator().manual_seed(40)
    lens = [700, 5, 300, 129, 0, 1000, 128]
    sites = [2, 3, 7, 8, 11, 15, 19]
    H, K, V, n_sites = 4, 32, 32, 24
    T = sum(lens)
    assert _lib.load().ssla_gla_recurrent_workspace_size(len(lens), T, H, K, V) > 0
    q, k, v = (torch.randn(T, H, D, generator=gen).to(dtype) for D in (K, K, V))
    g = F.logsigmoid(torch.randn(T, H, K, generator=gen) / 4)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64)
    state0 = torch.randn(n_sites, H, K, V, generator=gen) * 0.1
    st = state0.clone().to(dev)
    print(f"sparse scan long sequences {dtype}", flush=True)
    with torch.no_grad():
        o = sparse_gla_scan(q.to(dev), k.to(dev), v.to(dev), g.to(dev), cu.to(dev),
                            torch.tensor(sites, dtype=torch.int32, device=dev), st, scale=K ** -0.5)
    ro, rht = oracle.gla_recurrent(q.float().numpy(), k.float().numpy(), v.float().numpy(), g.numpy(), cu.numpy(),
                                   K ** -0.5, state0.numpy()[sites], True)
    if dtype == torch.float32:
        assert_close(o.cpu().numpy(), ro, 1e-4, "o")
    else:   # o rounded to bf16: within a bf16 rounding (2^-8 relative, fp32 sums on both sides) of each element
        assert_close(o.float().cpu().numpy(), ro, 2 ** -8, "o", band=1e-4, ratio_max=3e-3)
    assert_close(st.cpu().numpy()[sites], rht, 1e-4, "states")
    others = [i for i in range(n_sites) if i not in sites]
    assert torch.equal(st[others].cpu(), state0[others])
    # the same call again from the same states: the same bits
    st2 = state0.clone().to(dev)
    with torch.no_grad():
        o2 = sparse_gla_scan(q.to(dev), k.to(dev), v.to(dev), g.to(dev), cu.to(dev),
                             torch.tensor(sites, dtype=torch.int32, device=dev), st2, scale=K ** -0.5)
    assert torch.equal(o2, o) and torch.equal(st2, st), "segmented scan not repeatable"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_scan_returns_input_dtype(dev, dtype):
    """scan returns h in u's dtype (reference ops/common/scan.py:101,
    ``zeros_like(u)``): the fp32 running state rounded once per stored row,
    so the result equals the fp32 scan of the same inputs rounded to u's
    dtype, bit for bit; the gradients come back in the inputs' dtypes."""
    from ssla_amd.scan import scan
    gen = torch.Generator().manual_seed(71)
    lens = [5, 0, 40, 7]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64, device=dev)
    T, C = sum(lens), 24
    u = torch.randn(T, C, generator=gen).to(dtype).to(dev)
    g = torch.sigmoid(torch.randn(T, C, generator=gen)).to(dtype).to(dev)
    with torch.no_grad():
        h = scan(u, g, cu)
        h32 = scan(u.float(), g.float(), cu)
    assert h.dtype == dtype
    assert torch.equal(h, h32.to(dtype))
    ud, gd = u.clone().requires_grad_(), g.clone().requires_grad_()
    scan(ud, gd, cu).float().sum().backward()
    assert ud.grad.dtype == dtype and gd.grad.dtype == dtype
