"""SparsePool as two library calls (ssla_sparse_pool_plan / _emit, the path
SparsePool.forward takes when no gradient is recorded) against the composed
path (receptive-field gather, pool_segments, scatter_max / scatter_mean on a
sorted index -- the path a recorded gradient takes) and the CPU oracle.
Max is bit-exact; mean sums in fp64 in both paths and the oracle."""
import numpy as np
import pytest
import torch

from oracle import events as OE

pytestmark = pytest.mark.gpu


def _groups(seed, B, H, W, n_px, max_len, t_levels, C, sorted_runs=True):
    """Pixel groups in (batch, row, column) order, runs of 1..max_len events
    with times drawn from t_levels values (few levels: many equal times)."""
    rng = np.random.default_rng(seed)
    gb, gh, gw, gl, tim = [], [], [], [], []
    for b in range(B):
        for p in np.sort(rng.choice(H * W, size=min(n_px, H * W), replace=False)):
            n = int(rng.integers(1, max_len + 1))
            t = rng.integers(0, t_levels, size=n)
            tim.append(np.sort(t) if sorted_runs else t)
            gb.append(b), gh.append(p // W), gw.append(p % W), gl.append(n)
    tim = np.concatenate(tim).astype(np.int64) if tim else np.zeros(0, np.int64)
    ev = rng.standard_normal((tim.size, C)).astype(np.float32)
    return {"events": ev, "time": tim, "batch_id": np.array(gb, np.int64), "h": np.array(gh, np.int64),
            "w": np.array(gw, np.int64), "lengths": np.array(gl, np.int64), "batch_size": B}


def _dev(gr):
    d = {k: torch.from_numpy(np.ascontiguousarray(gr[k])).cuda()
         for k in ("events", "time", "batch_id", "h", "w", "lengths")}
    d["batch_size"] = gr["batch_size"]
    return d


def _both(layer, d):
    """(one-call result, composed result) of the same layer on d."""
    with torch.no_grad():
        one = layer(d)
    dg = dict(d)
    dg["events"] = d["events"].clone().requires_grad_(True)
    with torch.enable_grad():
        comp = layer(dg)
    comp = {k: (v.detach() if torch.is_tensor(v) else v) for k, v in comp.items()}
    return one, comp


KEYS = ("events", "time", "lengths", "batch_id", "h", "w")


@pytest.mark.parametrize("kind", ["max", "mean"])
@pytest.mark.parametrize("k,s", [((2, 2), None), ((4, 4), None), ((3, 3), (2, 2)), ((2, 3), (1, 2))])
@pytest.mark.parametrize("t_levels,sorted_runs", [(1000000, True), (7, True), (7, False)],
                         ids=["distinct", "ties", "unsorted"])
def test_pool_one_call_vs_composed_and_oracle(kind, k, s, t_levels, sorted_runs):
    from ssla_amd.layers import SparseAvgPool, SparseMaxPool
    frame = (13, 17)
    gr = _groups(3, 2, *frame, n_px=60, max_len=6, t_levels=t_levels, C=24, sorted_runs=sorted_runs)
    layer = (SparseMaxPool if kind == "max" else SparseAvgPool)(frame, kernel_size=k, stride=s).cuda()
    print(f"pool one-call {kind} k={k} s={s} t_levels={t_levels} sorted={sorted_runs}", flush=True)
    one, comp = _both(layer, _dev(gr))
    for key in KEYS:
        a, b = one[key].cpu().numpy(), comp[key].cpu().numpy()
        assert a.dtype == b.dtype and a.shape == b.shape, key
        if key == "events" and kind == "mean":
            np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7)
        else:
            np.testing.assert_array_equal(a, b, err_msg=key)
    lut, outc = OE.rf2pixels(frame, k, s or k)
    rf = OE.gather_receptive_fields(gr, frame, lut, outc)
    want = OE.sparse_pool(rf, kind)
    got = one["events"].cpu().numpy()
    if kind == "max":
        np.testing.assert_array_equal(got, want["events"])
    else:
        np.testing.assert_allclose(got, want["events"], rtol=1e-6, atol=1e-7)
    np.testing.assert_array_equal(one["time"].cpu().numpy(), want["time"])
    np.testing.assert_array_equal(one["lengths"].cpu().numpy(), want["lengths"])
    np.testing.assert_array_equal(one["h"].cpu().numpy(), rf["h"])
    np.testing.assert_array_equal(one["w"].cpu().numpy(), rf["w"])
    np.testing.assert_array_equal(one["batch_id"].cpu().numpy(), rf["batch_id"])


@pytest.mark.parametrize("kind", ["max", "mean"])
def test_pool_one_call_large_vs_oracle(kind):
    """The one-call pooling at 20,000 pixel groups and about 40,000 events
    on the 304 x 240 sensor (4 x 4 fields): its group-start and
    segment-head prefix sums run as multi-tile look-back scans.  Against the
    oracle and the composed path."""
    from ssla_amd.layers import SparseAvgPool, SparseMaxPool
    frame = (240, 304)
    gr = _groups(41, 1, *frame, n_px=20_000, max_len=3, t_levels=50, C=8)
    layer = (SparseMaxPool if kind == "max" else SparseAvgPool)(frame, kernel_size=(4, 4)).cuda()
    print(f"pool one-call large {kind}", flush=True)
    one, comp = _both(layer, _dev(gr))
    for key in KEYS:
        a, b = one[key].cpu().numpy(), comp[key].cpu().numpy()
        if key == "events" and kind == "mean":
            np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7)
        else:
            np.testing.assert_array_equal(a, b, err_msg=key)
    lut, outc = OE.rf2pixels(frame, (4, 4), (4, 4))
    want = OE.sparse_pool(OE.gather_receptive_fields(gr, frame, lut, outc), kind)
    assert want["time"].size > 8192
    if kind == "max":
        np.testing.assert_array_equal(one["events"].cpu().numpy(), want["events"])
    else:
        np.testing.assert_allclose(one["events"].cpu().numpy(), want["events"], rtol=1e-6, atol=1e-7)
    np.testing.assert_array_equal(one["time"].cpu().numpy(), want["time"])
    np.testing.assert_array_equal(one["lengths"].cpu().numpy(), want["lengths"])


@pytest.mark.parametrize("C", [16, 6])
def test_pool_one_call_special_values(C):
    """NaN never wins, equal maxima keep the first row (+0 / -0 bits), -inf
    is a value: the same bits as scatter_max on the composed path (four
    channels per thread, and one for a width that is not a multiple of 4)."""
    from ssla_amd.layers import SparseMaxPool
    frame = (9, 11)
    gr = _groups(5, 1, *frame, n_px=40, max_len=5, t_levels=3, C=C)
    ev = gr["events"]
    rng = np.random.default_rng(9)
    pick = rng.random(ev.shape)
    ev[pick < 0.15] = np.nan
    ev[(pick >= 0.15) & (pick < 0.3)] = 0.0
    ev[(pick >= 0.3) & (pick < 0.45)] = -0.0
    ev[(pick >= 0.45) & (pick < 0.5)] = -np.inf
    ev[:, 3] = np.nan   # a channel with no winner anywhere: 0
    layer = SparseMaxPool(frame, kernel_size=(3, 3)).cuda()
    one, comp = _both(layer, _dev(gr))
    a = one["events"].cpu().numpy().view(np.int32)
    b = comp["events"].cpu().numpy().view(np.int32)
    np.testing.assert_array_equal(a, b)
    assert np.all(one["events"].cpu().numpy()[:, 3] == 0)


def test_pool_one_call_empty_and_bad():
    from ssla_amd.layers import SparseMaxPool
    frame = (8, 8)
    layer = SparseMaxPool(frame, kernel_size=(2, 2)).cuda()
    gr = _groups(1, 2, *frame, n_px=0, max_len=1, t_levels=5, C=8)
    with torch.no_grad():
        r = layer(_dev(gr))
    assert r["events"].shape == (0, 8) and r["time"].numel() == 0 and r["lengths"].numel() == 0
    gr = _groups(2, 1, *frame, n_px=5, max_len=3, t_levels=5, C=8)
    gr["h"][2] = frame[0] + 3   # a pixel outside the frame
    with torch.no_grad(), pytest.raises(ValueError):
        layer(_dev(gr))


def test_pool_one_call_row_capacity():
    """A row capacity below the rows the fields hold is an error, not a
    write past the workspace: 3 x 3 fields at stride 1 put a pixel in up to
    9 fields, promised as 1."""
    from ssla_amd import events as E
    frame = (10, 12)
    gr = _groups(6, 1, *frame, n_px=50, max_len=4, t_levels=100, C=8)
    lut, outc = E.compute_rf2pixels(frame, (3, 3), (1, 1), device="cuda")
    with torch.no_grad():
        ok = E.sparse_pool(_dev(gr), frame, lut, outc, fields_per_pixel=9)
        with pytest.raises(ValueError, match="capacity"):
            E.sparse_pool(_dev(gr), frame, lut, outc, fields_per_pixel=1)
    rf = OE.gather_receptive_fields(gr, frame, lut.cpu().numpy(), outc.cpu().numpy())
    np.testing.assert_array_equal(ok["events"].cpu().numpy(), OE.sparse_pool(rf, "max")["events"])


@pytest.mark.parametrize("kind", ["max", "mean"])
@pytest.mark.parametrize("t_levels", [1000000, 7], ids=["distinct", "ties"])
def test_pool_values_linear_equals_linear_then_pool(kind, t_levels):
    """SparsePool.apply_plan_linear (the bf16 linear map of two inputs folded
    into the value pass, ssla_sparse_pool_emit_linear) equals
    F.linear(x.bfloat16(), w).float() followed by apply_plan, bit for bit:
    inputs that need rounding to bf16, repeated rows (ties in the max) and
    a 4 x 4 field as in the backbone's stem."""
    import torch.nn.functional as F
    from ssla_amd.layers import SparseAvgPool, SparseMaxPool
    frame = (24, 28)
    gr = _groups(21, 2, *frame, 250, 5, t_levels, 2)
    rng = np.random.default_rng(22)
    x = rng.standard_normal((gr["time"].size, 2)).astype(np.float32) * np.float32(3.3)
    rep = np.arange(0, x.shape[0] - 1, 5)
    x[rep + 1] = x[rep]   # repeated inputs: equal mapped rows
    gr["events"] = x
    d = _dev(gr)
    layer = (SparseMaxPool if kind == "max" else SparseAvgPool)(frame, kernel_size=(4, 4))
    w = (torch.randn(32, 2, device="cuda") * 0.7).to(torch.bfloat16)
    print(f"pool values linear {kind} t_levels={t_levels}", flush=True)
    with torch.no_grad():
        plan = layer.plan(d)
        fused = layer.apply_plan_linear(plan, d["events"], w)
        ref = layer.apply_plan(plan, F.linear(d["events"].to(torch.bfloat16), w).float())
    for key in KEYS:
        assert torch.equal(fused[key], ref[key]), key
    with pytest.raises(ValueError):
        layer.apply_plan_linear(plan, d["events"][:-1], w)
