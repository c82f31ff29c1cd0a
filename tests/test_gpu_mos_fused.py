"""GPU parity of the fused MosAttention forward (ssla_mos_attention_fwd)
against the composed forward (the same layer through the patch scatter,
per-position GEMMs, scan and ordered index-add, itself pinned to the
reference layer's outputs in test_gpu_layers.py) on full-size and edge
inputs.  Both are fp32; they differ in summation order only, so the bar is
rtol = atol = 1e-4 on the LayerNorm outputs (unit scale)."""
import numpy as np
import pytest
import torch

from tests.conftest import assert_close

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _grouped(B=8, n_mean=50_000, seed=0, C=None):
    from ssla_amd import events as E, synthetic
    ev, ln = synthetic.event_windows(B=B, n_mean=n_mean, seed=seed)
    gr = E.preprocess_inputs(ev.cuda(), ln.cuda(), (240, 304), 50)
    if C is not None:
        gen = torch.Generator(device="cuda").manual_seed(seed)
        gr["events"] = torch.randn(gr["time"].shape[0], C, device="cuda", generator=gen)
    return gr


def _both(layer, gr):
    with torch.no_grad():
        a = layer(gr, fused=True)["events"]
        b = layer(gr, fused=False)["events"]
    return a.cpu().numpy(), b.cpu().numpy()


@pytest.mark.parametrize("cin,hid,k", [(2, 12, 1), (12, 12, 3), (12, 24, 3), (24, 24, 3), (16, 32, 2), (24, 32, 1)])
def test_fused_matches_composed_stage_sizes(cin, hid, k):
    """MOS_S layer shapes on a C5-like batch of 8 Gen1 windows."""
    from ssla_amd.layers import MosAttention
    torch.manual_seed(cin * 100 + hid)
    gr = _grouped(C=None if cin == 2 else cin)
    layer = MosAttention(cin, hid, (240, 304), (k, k)).cuda()
    print(f"mos fused full: E={gr['time'].shape[0]} cin={cin} hid={hid} k={k}", flush=True)
    a, b = _both(layer, gr)
    assert a.shape == (gr["time"].shape[0], hid)
    assert_close(a, b, TOL, f"fused vs composed cin={cin} hid={hid} k={k}")


@pytest.mark.parametrize("cin,hid,k", [(24, 48, 3), (48, 48, 3), (48, 96, 3), (96, 96, 3), (16, 32, 3)])
def test_fused_matrix_core_sizes(cin, hid, k):
    """MOS_S stages 3-4 (hidden 48 / 96, with and without the input
    projection) and hidden 32 whose 9 per-position matrices exceed the small
    kernels' LDS: the matrix-core path against the composed forward on a
    C5-like batch of 8 Gen1 windows."""
    from ssla_amd.layers import MosAttention
    torch.manual_seed(cin * 100 + hid)
    gr = _grouped(C=cin)
    layer = MosAttention(cin, hid, (240, 304), (k, k)).cuda()
    print(f"mos fused matrix-core: E={gr['time'].shape[0]} cin={cin} hid={hid} k={k}", flush=True)
    with torch.no_grad():
        assert layer._fused_ok(gr["events"])
    a, b = _both(layer, gr)
    assert a.shape == (gr["time"].shape[0], hid)
    assert_close(a, b, TOL, f"matrix-core vs composed cin={cin} hid={hid} k={k}")


def test_fused_matrix_core_edges():
    """The matrix-core path on one pixel holding 1500 events beside isolated
    ones (patch rows spanning many 64-row tiles of one position), a single
    event, and every combination of shared / per-position projections."""
    from ssla_amd import events as E
    from ssla_amd.layers import MosAttention
    H, W = 20, 30
    rng = np.random.default_rng(4)
    n_hot, n_rest = 1500, 400
    x = np.concatenate([np.full(n_hot, 7), rng.integers(0, W, n_rest)])
    y = np.concatenate([np.full(n_hot, 5), rng.integers(0, H, n_rest)])
    t = np.sort(rng.integers(0, 100_000, n_hot + n_rest))
    order = rng.permutation(n_hot + n_rest)
    ev = torch.zeros(1, n_hot + n_rest, 4)
    ev[0, :, 0] = torch.from_numpy(x[order]).float()
    ev[0, :, 1] = torch.from_numpy(y[order]).float()
    ev[0, :, 2] = torch.from_numpy(t).float()
    ev[0, :, 3] = 1.0
    gr = E.group_events((ev.cuda(), torch.tensor([n_hot + n_rest]).cuda()), (H, W), max_events_per_px=4096)
    gr["events"] = torch.randn(gr["time"].shape[0], 48, device="cuda")
    for sp, gp in ((True, True), (False, True), (True, False), (False, False)):
        torch.manual_seed(5)
        layer = MosAttention(48, 48, (H, W), (3, 3), scatter_proj=sp, gather_proj=gp).cuda()
        print(f"mos matrix-core long patch sp={sp} gp={gp}", flush=True)
        a, b = _both(layer, gr)
        assert_close(a, b, TOL, f"matrix-core long patch sp={sp} gp={gp}")
    one = E.group_events((torch.tensor([[[3.0, 2.0, 10.0, 1.0]]]).cuda(), torch.tensor([1]).cuda()), (8, 8))
    one["events"] = torch.randn(1, 24, device="cuda")
    torch.manual_seed(6)
    layer = MosAttention(24, 48, (8, 8), (3, 3)).cuda()
    print("mos matrix-core single event", flush=True)
    a, b = _both(layer, one)
    assert_close(a, b, TOL, "matrix-core single event")


def test_fused_long_patch_and_singletons():
    """One pixel holding 1500 events (its patches span many 64-row windows
    and several wavefront windows) beside isolated single events."""
    from ssla_amd import events as E
    from ssla_amd.layers import MosAttention
    H, W = 20, 30
    rng = np.random.default_rng(3)
    n_hot, n_rest = 1500, 400
    x = np.concatenate([np.full(n_hot, 7), rng.integers(0, W, n_rest)])
    y = np.concatenate([np.full(n_hot, 5), rng.integers(0, H, n_rest)])
    t = np.sort(rng.integers(0, 100_000, n_hot + n_rest))
    order = rng.permutation(n_hot + n_rest)
    ev = torch.zeros(1, n_hot + n_rest, 4)
    ev[0, :, 0] = torch.from_numpy(x[order]).float()
    ev[0, :, 1] = torch.from_numpy(y[order]).float()
    ev[0, :, 2] = torch.from_numpy(t).float()
    ev[0, :, 3] = 1.0
    gr = E.group_events((ev.cuda(), torch.tensor([n_hot + n_rest]).cuda()), (H, W), max_events_per_px=4096)
    gr["events"] = torch.randn(gr["time"].shape[0], 12, device="cuda")
    torch.manual_seed(1)
    layer = MosAttention(12, 12, (H, W), (3, 3)).cuda()
    print(f"mos fused long patch: E={gr['time'].shape[0]} max len={int(gr['lengths'].max())}", flush=True)
    a, b = _both(layer, gr)
    assert_close(a, b, TOL, "long patch")


def test_fused_single_event_and_disabled_projections():
    from ssla_amd import events as E
    from ssla_amd.layers import MosAttention
    ev = torch.tensor([[[3.0, 2.0, 10.0, 1.0]]])
    gr = E.group_events((ev.cuda(), torch.tensor([1]).cuda()), (8, 8))
    gr["events"] = torch.randn(1, 12, device="cuda")
    for sp, gp in ((True, True), (False, True), (True, False), (False, False)):
        torch.manual_seed(2)
        layer = MosAttention(12, 12, (8, 8), (3, 3), scatter_proj=sp, gather_proj=gp).cuda()
        print(f"mos fused single event sp={sp} gp={gp}", flush=True)
        a, b = _both(layer, gr)
        assert_close(a, b, TOL, f"single event sp={sp} gp={gp}")


@pytest.mark.parametrize("cin,hid,k", [(6, 48, 3), (48, 132, 1), (2, 12, 8)])
def test_fused_unsupported_sizes(cin, hid, k):
    """Hidden > 32 with an input size that is not a multiple of 4, hidden >
    128, or more than 49 kernel positions (8 x 8, whose small weights would
    fit LDS): fused=True raises, the default runs the composed path."""
    from ssla_amd import _lib
    from ssla_amd.layers import MosAttention
    gr = _grouped(B=1, n_mean=2000, C=cin)
    layer = MosAttention(cin, hid, (240, 304), (k, k)).cuda()
    with torch.no_grad():
        with pytest.raises(_lib.SslaError):
            layer(gr, fused=True)
        out = layer(gr)["events"]
    assert out.shape == (gr["time"].shape[0], hid) and torch.isfinite(out).all()


def test_fused_not_used_under_autograd():
    from ssla_amd.layers import MosAttention
    gr = _grouped(B=1, n_mean=2000, C=12)
    layer = MosAttention(12, 12, (240, 304), (3, 3)).cuda()
    assert not layer._fused_ok(gr["events"])   # parameters require grad
    out = layer(gr)["events"]
    assert out.requires_grad
