"""Pins of the layer oracle (oracle/layers.py) against golden vectors that
the reference's own MosAttention / LinearAttention wrote
(tests/golden/make_layer_fixtures.py), plus planted-mistake checks that the
pin is sharp.  CPU only."""
from pathlib import Path

import numpy as np
import pytest

from oracle import layers as OL

FIX = Path(__file__).resolve().parent / "golden" / "layer_fixtures.npz"
MOS_CASES = {
    "mos_a": (6, (3, 3), (1, 1), True, True),
    "mos_b": (8, (2, 2), (2, 2), True, True),
    "mos_c": (6, (3, 3), (1, 1), False, False),
}
LIN_CASES = {"lin_a": 6, "lin_b": 8}
TOL = dict(rtol=1e-4, atol=1e-4)   # fixtures are fp32 reference outputs


@pytest.fixture(scope="module")
def fx():
    return np.load(FIX, allow_pickle=False)


def grouped_inputs(fx, C):
    gr = {k: fx[f"in_{k}"] for k in ("time", "batch_id", "h", "w", "lengths")}
    gr["batch_size"] = int(fx["in_batch_size"])
    gr["events"] = fx[f"in_events_c{C}"]
    return gr


def params(fx, tag):
    pre = f"{tag}_sd_"
    return {k[len(pre):]: fx[k] for k in fx.files if k.startswith(pre)}


@pytest.mark.parametrize("tag", sorted(MOS_CASES))
def test_mos_attention(fx, tag):
    C, k, s, sp, gp = MOS_CASES[tag]
    out = OL.mos_attention(params(fx, tag), grouped_inputs(fx, C), tuple(fx["in_frame"]), k, s, sp, gp)
    np.testing.assert_allclose(out, fx[f"{tag}_out"], **TOL)


@pytest.mark.parametrize("tag", sorted(LIN_CASES))
def test_linear_attention(fx, tag):
    out = OL.linear_attention(params(fx, tag), grouped_inputs(fx, LIN_CASES[tag]))
    np.testing.assert_allclose(out, fx[f"{tag}_out"], **TOL)


def test_planted_mistakes_fail(fx):
    """Swapping the per-position weights, dropping the gate, or ordering
    LinearAttention by time only must each break the pin."""
    C, k, s, sp, gp = MOS_CASES["mos_a"]
    p = params(fx, "mos_a")
    gr = grouped_inputs(fx, C)
    want = fx["mos_a_out"]
    q = dict(p)
    q["scatter_conv_weights"] = p["scatter_conv_weights"][::-1].copy()
    assert not np.allclose(OL.mos_attention(q, gr, tuple(fx["in_frame"]), k, s, sp, gp), want, **TOL)
    q = dict(p)
    q["gather_conv_weights"] = p["gather_conv_weights"][:, ::-1].copy()
    assert not np.allclose(OL.mos_attention(q, gr, tuple(fx["in_frame"]), k, s, sp, gp), want, **TOL)
    # all-open gate (g -> 1 everywhere): the scan degenerates to a prefix sum
    q = dict(p)
    q["g_proj.weight"] = np.zeros_like(p["g_proj.weight"])
    assert not np.allclose(OL.mos_attention(q, gr, tuple(fx["in_frame"]), k, s, sp, gp), want, **TOL)
    # LinearAttention: dropping the batch key merges samples into one sequence
    pl = params(fx, "lin_a")
    grl = grouped_inputs(fx, 6)
    grl = dict(grl)
    grl["batch_id"] = np.zeros_like(grl["batch_id"])
    grl["batch_size"] = 1
    assert not np.allclose(OL.linear_attention(pl, grl), fx["lin_a_out"], **TOL)


def test_layer_norm_closed_form():
    x = np.array([[1.0, 2.0, 3.0, 6.0]])
    y = OL._layer_norm(x, np.ones(4), np.zeros(4), eps=0.0)
    np.testing.assert_allclose(y.mean(), 0.0, atol=1e-12)
    np.testing.assert_allclose((y ** 2).mean(), 1.0, rtol=1e-12)
