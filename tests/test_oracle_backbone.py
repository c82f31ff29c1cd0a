"""CPU pins of the async-step oracle (oracle.backbone).

* block_scan (per-site recurrence with stored states) is pinned by
  split-and-carry: running each site's events in two pieces with the state
  stored in between equals one pass, and state rows of sites without events
  are left untouched; a planted mistake (starting each site from zero
  instead of its stored state) breaks the equality.
* head is pinned against the DetectionHead module run in fp64 on the CPU
  with the same bf16-rounded weights and inputs.
* max_pool's site list is strictly increasing (the order the GPU step
  relies on for its state rows).
"""
import numpy as np
import torch

from oracle import backbone as ob


def _site_inputs(seed=0, n_sites=30, H=2, D=8):
    rng = np.random.default_rng(seed)
    sites = np.sort(rng.choice(n_sites, size=12, replace=False))
    lens = rng.integers(1, 9, size=sites.size)
    T = int(lens.sum())
    q, k, v = (rng.standard_normal((T, H, D)).astype(np.float32) for _ in range(3))
    g = np.log(1 / (1 + np.exp(-rng.standard_normal((T, H, D))))).astype(np.float32)
    state = (0.1 * rng.standard_normal((n_sites, H, D, D))).astype(np.float32)
    return sites, lens, q, k, v, g, state


def test_block_scan_split_and_carry():
    sites, lens, q, k, v, g, state = _site_inputs()
    one = state.copy()
    o1 = ob.block_scan(q, k, v, g, lens, sites, one, 0.5)
    # first part of every site's rows, then the rest, state carried
    starts = np.concatenate([[0], np.cumsum(lens)])
    cut = lens // 2
    two = state.copy()
    rows_a = np.concatenate([np.arange(starts[i], starts[i] + cut[i]) for i in range(sites.size)])
    rows_b = np.concatenate([np.arange(starts[i] + cut[i], starts[i + 1]) for i in range(sites.size)])
    has_a = cut > 0
    oa = ob.block_scan(q[rows_a], k[rows_a], v[rows_a], g[rows_a], cut[has_a], sites[has_a], two, 0.5)
    ob_ = ob.block_scan(q[rows_b], k[rows_b], v[rows_b], g[rows_b], lens - cut, sites, two, 0.5)
    o2 = np.empty_like(o1)
    o2[rows_a], o2[rows_b] = oa, ob_
    assert np.allclose(o1, o2, rtol=1e-6, atol=1e-7)
    assert np.allclose(one, two, rtol=1e-6, atol=1e-7)
    others = np.setdiff1d(np.arange(state.shape[0]), sites)
    assert np.array_equal(one[others], state[others])
    # planted mistake: each site from zero instead of its stored state
    bad = state.copy()
    bad[sites] = 0.0
    o_bad = ob.block_scan(q, k, v, g, lens, sites, bad, 0.5)
    assert not np.allclose(o_bad, o1, rtol=1e-3, atol=1e-4)


def test_head_matches_module_in_fp64():
    from ssla_amd.backbone import DetectionHead
    torch.manual_seed(3)
    head = DetectionHead(2, (8, 16), (6, 10), 12)
    for m in head.modules():
        if isinstance(m, torch.nn.BatchNorm2d):
            m.running_mean.uniform_(-0.5, 0.5)
            m.running_var.uniform_(0.5, 2.0)
    head.eval()
    params = {k: v.detach().float().numpy() for k, v in head.state_dict().items()}
    grids = [torch.randn(1, 6, 5, 7), torch.randn(1, 10, 3, 4)]
    ref = ob.head(params, [g.numpy() for g in grids], (8, 16))
    h64 = DetectionHead(2, (8, 16), (6, 10), 12).double().eval()
    with torch.no_grad():
        for name, t in h64.state_dict().items():
            src = head.state_dict()[name]
            t.copy_(src.bfloat16().double() if src.is_floating_point() else src)
        out = h64([g.bfloat16().double() for g in grids]).numpy()
    assert out.shape == (1, 5 * 7 + 3 * 4, 7)
    assert np.allclose(out, ref, rtol=1e-9, atol=1e-9)


def test_max_pool_sites_strictly_increasing():
    rng = np.random.default_rng(5)
    n = 400
    gr = {"events": rng.standard_normal((n, 3)).astype(np.float32), "time": np.sort(rng.integers(0, 50, n)),
          "batch_id": np.zeros(n, np.int64)}
    # one event per pixel group on a 20 x 24 frame
    pix = np.sort(rng.choice(20 * 24, size=n, replace=False))
    gr.update({"h": pix // 24, "w": pix % 24, "lengths": np.ones(n, np.int64), "batch_size": 1,
               "time": rng.integers(0, 50, n)})
    out = ob.max_pool(gr, (20, 24), 2)
    sites = ob.sites_of(out, (10, 12))
    assert sites.size > 0 and np.all(np.diff(sites) > 0)
    assert out["events"].shape[0] == int(out["lengths"].sum())
