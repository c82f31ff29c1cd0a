"""Host-side checks of ssla_amd.layers that need no GPU: constructor
arguments, parameter / buffer names and shapes match the reference's layers
(their state dicts, written by tests/golden/make_layer_fixtures.py), and the
output frame sizes of the pooling modules."""
from pathlib import Path

import numpy as np
import pytest

from oracle import events as OE

GOLD = Path(__file__).resolve().parent / "golden" / "layer_fixtures.npz"


@pytest.fixture(scope="module")
def fx():
    return np.load(GOLD, allow_pickle=False)


def _ref_shapes(fx, tag):
    pre = f"{tag}_sd_"
    return {k[len(pre):]: fx[k].shape for k in fx.files if k.startswith(pre)}


@pytest.mark.parametrize("tag,args", [
    ("mos_a", (6, 8, (3, 3), (1, 1), True, True)),
    ("mos_b", (8, 8, (2, 2), (2, 2), True, True)),
    ("mos_c", (6, 8, (3, 3), (1, 1), False, False)),
])
def test_mos_attention_state_dict(fx, tag, args):
    from ssla_amd.layers import MosAttention
    ci, ch, k, s, sp, gp = args
    layer = MosAttention(ci, ch, tuple(fx["in_frame"]), k, s, scatter_proj=sp, gather_proj=gp)
    got = {k_: tuple(v.shape) for k_, v in layer.state_dict().items()}
    assert got == _ref_shapes(fx, tag)
    assert layer.frame_output_size == tuple(fx["in_frame"])


@pytest.mark.parametrize("tag,ci", [("lin_a", 6), ("lin_b", 8)])
def test_linear_attention_state_dict(fx, tag, ci):
    from ssla_amd.layers import LinearAttention
    layer = LinearAttention(ci, 8, tuple(fx["in_frame"]))
    got = {k_: tuple(v.shape) for k_, v in layer.state_dict().items()}
    assert got == _ref_shapes(fx, tag)


@pytest.mark.parametrize("frame,k,s", [((16, 20), (2, 2), None), ((7, 10), (3, 3), (2, 2)),
                                       ((9, 5), (2, 2), (2, 2)), ((6, 8), (5, 5), (3, 3)),
                                       ((16, 20), (1, 1), None)])
def test_pool_output_frame(frame, k, s):
    from ssla_amd.layers import SparseMaxPool
    layer = SparseMaxPool(frame, kernel_size=k, stride=s)
    _, outc = OE.rf2pixels(frame, k, s or k)
    assert layer.frame_output_size == (int(outc[:, 1].max()) + 1, int(outc[:, 0].max()) + 1)
    names = dict(layer.named_buffers())
    assert set(names) == {"max_events_per_rf", "rf2pixel_lut", "rf_outcoord"}
    assert tuple(names["rf2pixel_lut"].shape) == (outc.shape[0], k[0] * k[1])


def test_temporal_dropout_rejects_bad_window():
    from ssla_amd.layers import TemporalDropout
    with pytest.raises(ValueError):
        TemporalDropout(0, (8, 8))


def test_layers_refuse_cpu_tensors(fx):
    """No CPU fallback: the product path raises on host tensors."""
    import torch
    from ssla_amd.layers import LinearAttention
    layer = LinearAttention(6, 8, tuple(fx["in_frame"]))
    inp = {k: torch.from_numpy(fx[f"in_{k}"]) for k in ("time", "batch_id", "h", "w", "lengths")}
    inp["batch_size"] = int(fx["in_batch_size"])
    inp["events"] = torch.from_numpy(fx["in_events_c6"])
    with pytest.raises(Exception, match="(?i)cuda|device|gpu"):
        with torch.no_grad():
            layer(inp)


@pytest.mark.parametrize("ins,hs,k", [(2, 12, (3, 3)), (12, 12, (1, 1)), (24, 48, (3, 3)), (48, 48, (5, 3))])
def test_mos_attention_compute_flops(ins, hs, k):
    """MosAttention.compute_flops (reference layers/mos_attention.py:169-199)
    against the count collected per event: each of the n * kh * kw patch
    copies costs hs (2 ins + 10 hs + 2) flops, each pixel event hs (9) + 1
    more, plus hs (2 ins - 1) for the input projection when ins != hs."""
    import torch
    from ssla_amd.layers import MosAttention
    layer = MosAttention(ins, hs, (16, 20), k)
    n = 137
    x = {"events": torch.zeros(n, ins)}
    want = n * k[0] * k[1] * hs * (2 * ins + 10 * hs + 2) + n * (9 * hs + 1)
    if ins != hs:
        want += n * hs * (2 * ins - 1)
    assert layer.compute_flops(x) == want


@pytest.mark.parametrize("ins,hs", [(2, 12), (24, 24)])
def test_linear_attention_compute_flops(ins, hs):
    """LinearAttention.compute_flops (terms of reference
    layers/linear_attention.py:105-124, one scan row per event), collected
    per event: hs (8 hs + 3) for q, v, g, the gates, the scan, q * h and the
    output projection, hs for the residual and 8 hs + 1 for the norm, plus
    2 hs (2 ins - 1) for the input and residual projections when ins != hs."""
    import torch
    from ssla_amd.layers import LinearAttention
    layer = LinearAttention(ins, hs, (16, 20))
    n = 53
    want = n * (hs * (8 * hs + 3) + hs + 8 * hs + 1)
    if ins != hs:
        want += 2 * n * hs * (2 * ins - 1)
    assert layer.compute_flops({"events": torch.zeros(n, ins)}) == want


def test_async_module_compute_flops_fallback():
    """TemporalDropout and other modules without a cost of their own count 0
    (reference layers/async_sparse_module.py:44-46)."""
    from ssla_amd.layers import TemporalDropout
    assert TemporalDropout(4, (16, 20)).compute_flops({}) == 0
