"""Layers on the GPU (ssla_amd.layers) against the reference's own layer
outputs (tests/golden/layer_fixtures.npz, event_fixtures.npz) and the CPU
oracle.  The state dicts of the reference's layers load unchanged."""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import events as OE
from oracle import layers as OL

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"
MOS_CASES = {
    "mos_a": (6, (3, 3), (1, 1), True, True),
    "mos_b": (8, (2, 2), (2, 2), True, True),
    "mos_c": (6, (3, 3), (1, 1), False, False),
}
LIN_CASES = {"lin_a": 6, "lin_b": 8}
# fp32 GEMMs + fp32 scan + LayerNorm against fp32 CPU reference outputs
TOL = dict(rtol=2e-4, atol=2e-4)


@pytest.fixture(scope="module")
def lfx():
    return np.load(GOLD / "layer_fixtures.npz", allow_pickle=False)


@pytest.fixture(scope="module")
def efx():
    return np.load(GOLD / "event_fixtures.npz", allow_pickle=False)


def dev_inputs(fx, C):
    d = {k: torch.from_numpy(fx[f"in_{k}"]).cuda() for k in ("time", "batch_id", "h", "w", "lengths")}
    d["batch_size"] = int(fx["in_batch_size"])
    d["events"] = torch.from_numpy(fx[f"in_events_c{C}"]).cuda()
    return d


def state(fx, tag):
    pre = f"{tag}_sd_"
    return {k[len(pre):]: torch.from_numpy(fx[k]) for k in fx.files if k.startswith(pre)}


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "composed"])
@pytest.mark.parametrize("tag", sorted(MOS_CASES))
def test_mos_attention_matches_reference(lfx, tag, fused):
    from ssla_amd.layers import MosAttention
    C, k, s, sp, gp = MOS_CASES[tag]
    frame = tuple(int(v) for v in lfx["in_frame"])
    layer = MosAttention(C, 8, frame, k, s, scatter_proj=sp, gather_proj=gp)
    layer.load_state_dict(state(lfx, tag), strict=True)
    layer = layer.cuda()
    print(f"mos {tag}: E={lfx['in_time'].shape[0]} C={C} k={k} s={s} fused={fused}", flush=True)
    with torch.no_grad():
        r = layer(dev_inputs(lfx, C), fused=fused)
    np.testing.assert_allclose(r["events"].cpu().numpy(), lfx[f"{tag}_out"], **TOL)
    # the device-built table equals the reference's registered buffer
    np.testing.assert_array_equal(layer.patch2pixel_lut.cpu().numpy(), lfx[f"{tag}_sd_patch2pixel_lut"])
    for key in ("time", "lengths", "batch_id", "h", "w"):
        np.testing.assert_array_equal(r[key].cpu().numpy(), lfx[f"in_{key}"])


@pytest.mark.parametrize("tag", sorted(LIN_CASES))
def test_linear_attention_matches_reference(lfx, tag):
    from ssla_amd.layers import LinearAttention
    C = LIN_CASES[tag]
    frame = tuple(int(v) for v in lfx["in_frame"])
    layer = LinearAttention(C, 8, frame)
    layer.load_state_dict(state(lfx, tag), strict=True)
    layer = layer.cuda()
    print(f"lin {tag}: C={C}", flush=True)
    with torch.no_grad():
        r = layer(dev_inputs(lfx, C))
    np.testing.assert_allclose(r["events"].cpu().numpy(), lfx[f"{tag}_out"], **TOL)


@pytest.mark.parametrize("cin,hid", [(16, 24), (24, 48), (48, 96)])
@pytest.mark.parametrize("fused", [True, False], ids=["fused", "composed"])
def test_mos_attention_larger_vs_oracle(fused, cin, hid):
    """A bigger random case (hot pixels, many patches) against the fp64
    oracle; hidden 24 runs the small fused kernels, 48 and 96 the
    matrix-core path."""
    from ssla_amd.layers import MosAttention
    from ssla_amd import events as E
    torch.manual_seed(7)
    B, N, H, W = 2, 3000, 24, 32
    ev, lengths = _random_events(B, N, H, W, seed=7)
    gr = E.group_events((ev.cuda(), lengths.cuda()), (H, W))
    gr["events"] = torch.randn(gr["time"].shape[0], cin, device="cuda")
    layer = MosAttention(cin, hid, (H, W), (3, 3), (1, 1)).cuda()
    print(f"mos oracle: E={gr['time'].shape[0]} cin={cin} hid={hid} fused={fused}", flush=True)
    with torch.no_grad():
        r = layer(gr, fused=fused)
    p = {k: v.detach().cpu().numpy() for k, v in layer.state_dict().items()}
    grn = {k: (v.cpu().numpy() if torch.is_tensor(v) else v) for k, v in gr.items()}
    want = OL.mos_attention(p, grn, (H, W), (3, 3), (1, 1))
    np.testing.assert_allclose(r["events"].cpu().numpy(), want, rtol=1e-3, atol=1e-3)


def _random_events(B, N, H, W, seed):
    g = torch.Generator().manual_seed(seed)
    ev = torch.zeros(B, N, 5)
    lengths = torch.randint(N // 2, N + 1, (B,), generator=g)
    for b in range(B):
        n = int(lengths[b])
        ev[b, :n, 0] = torch.randint(0, W, (n,), generator=g).float()
        ev[b, :n, 1] = torch.randint(0, H, (n,), generator=g).float()
        t = torch.sort(torch.randint(0, n // 2, (n,), generator=g) * 5).values.float()
        ev[b, :n, 2] = t
        ev[b, :n, 3] = t
        ev[b, :n, 4] = torch.where(torch.rand(n, generator=g) < 0.5, -1.0, 1.0)
    return ev, lengths


def _grouped_dev(efx):
    gr = OE.group_events(efx["ge_events"], efx["ge_lengths"], tuple(efx["ge_frame"]), 512)
    d = {k: torch.from_numpy(np.ascontiguousarray(gr[k])).cuda() for k in ("time", "batch_id", "h", "w", "lengths")}
    d["batch_size"] = int(gr["batch_size"])
    d["events"] = torch.from_numpy(efx["sp_pix_events"]).cuda()
    return d, gr


@pytest.mark.parametrize("kind", ["max", "mean"])
@pytest.mark.parametrize("k,s", [((2, 2), None), ((3, 3), (2, 2))])
def test_sparse_pool_vs_oracle(efx, kind, k, s):
    from ssla_amd.layers import SparseMaxPool, SparseAvgPool
    frame = tuple(int(v) for v in efx["ge_frame"])
    cls = SparseMaxPool if kind == "max" else SparseAvgPool
    layer = cls(frame, kernel_size=k, stride=s).cuda()
    d, gr = _grouped_dev(efx)
    gr["events"] = efx["sp_pix_events"]
    print(f"pool {kind} k={k} s={s}", flush=True)
    with torch.no_grad():
        r = layer(d)
    s_ = s or k
    lut, outc = OE.rf2pixels(frame, k, s_)
    rf = OE.gather_receptive_fields(gr, frame, lut, outc)
    want = OE.sparse_pool(rf, kind)
    got = r["events"].cpu().numpy()
    if kind == "max":
        np.testing.assert_array_equal(got, want["events"])
    else:
        np.testing.assert_allclose(got, want["events"], rtol=1e-6, atol=1e-6)
    np.testing.assert_array_equal(r["time"].cpu().numpy(), want["time"])
    np.testing.assert_array_equal(r["lengths"].cpu().numpy(), want["lengths"])
    np.testing.assert_array_equal(r["h"].cpu().numpy(), rf["h"])
    np.testing.assert_array_equal(r["w"].cpu().numpy(), rf["w"])
    np.testing.assert_array_equal(r["batch_id"].cpu().numpy(), rf["batch_id"])
    assert layer.frame_output_size == (int(outc[:, 1].max()) + 1, int(outc[:, 0].max()) + 1)


def test_adaptive_pool_kernel():
    from ssla_amd.layers import SparseAdaptiveMaxPool, SparseAdaptiveAvgPool
    a = SparseAdaptiveMaxPool((16, 20), (4, 6))
    assert list(a.kernel_size) == [4, 4] and list(a.stride) == [4, 4]
    b = SparseAdaptiveAvgPool((16, 20), (5, 5))
    assert list(b.kernel_size) == [4, 4]
    with pytest.raises(ValueError):
        SparseAdaptiveMaxPool((16, 20), (17, 5))


@pytest.mark.parametrize("wsz", [1, 3, 4])
def test_temporal_dropout_matches_reference(efx, wsz):
    from ssla_amd.layers import TemporalDropout
    frame = tuple(int(v) for v in efx["ge_frame"])
    layer = TemporalDropout(wsz, frame).cuda()
    d, _ = _grouped_dev(efx)
    print(f"temporal dropout w={wsz}", flush=True)
    with torch.no_grad():
        r = layer(d)
    np.testing.assert_array_equal(r["events"].cpu().numpy(), efx[f"td_w{wsz}_events"])
    np.testing.assert_array_equal(r["time"].cpu().numpy(), efx[f"td_w{wsz}_time"])
    np.testing.assert_array_equal(r["lengths"].cpu().numpy(), efx[f"td_w{wsz}_lengths"])


def test_pool_from_ungrouped_events(efx):
    """grouped_events=False groups the padded events first."""
    from ssla_amd.layers import SparseMaxPool
    frame = tuple(int(v) for v in efx["ge_frame"])
    layer = SparseMaxPool(frame, kernel_size=(2, 2)).cuda()
    ev = torch.from_numpy(efx["ge_events"]).cuda()
    ln = torch.from_numpy(efx["ge_lengths"]).cuda()
    with torch.no_grad():
        r = layer((ev, ln), grouped_events=False)
    gr = OE.group_events(efx["ge_events"], efx["ge_lengths"], frame, 512)
    lut, outc = OE.rf2pixels(frame, (2, 2), (2, 2))
    want = OE.sparse_pool(OE.gather_receptive_fields(gr, frame, lut, outc), "max")
    np.testing.assert_array_equal(r["events"].cpu().numpy(), want["events"])
    np.testing.assert_array_equal(r["time"].cpu().numpy(), want["time"])


@pytest.mark.parametrize("kind", ["max", "mean"])
@pytest.mark.parametrize("k,s", [((2, 2), None), ((3, 3), (2, 2))])
def test_sparse_pool_compute_flops(efx, kind, k, s):
    """SparseMaxPool / SparseAvgPool.compute_flops (reference
    layers/sparse_pooling.py:53-87): the receptive-field events that join an
    earlier event of the same field and time, times the channels, times 1
    (max) or 2 (mean); the count is taken from the oracle's field gather."""
    from ssla_amd.layers import SparseMaxPool, SparseAvgPool
    frame = tuple(int(v) for v in efx["ge_frame"])
    cls = SparseMaxPool if kind == "max" else SparseAvgPool
    layer = cls(frame, kernel_size=k, stride=s).cuda()
    d, gr = _grouped_dev(efx)
    gr["events"] = efx["sp_pix_events"]
    lut, outc = OE.rf2pixels(frame, k, s or k)
    rf = OE.gather_receptive_fields(gr, frame, lut, outc)
    field = np.repeat(np.arange(len(rf["lengths"])), rf["lengths"])
    t = np.asarray(rf["time"])
    joins = int(np.sum((field[1:] == field[:-1]) & (t[1:] == t[:-1])))
    C = efx["sp_pix_events"].shape[1]
    print(f"pool compute_flops {kind} k={k}", flush=True)
    assert layer.compute_flops(d) == joins * C * (1 if kind == "max" else 2)
