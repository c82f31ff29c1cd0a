"""GPU gradients: the row gather / index-add pair and LinearAttention's
backward (through the scan backward), against plain torch on the CPU in
float64 (autograd of the same operations).  fp32 device arithmetic: rtol
1e-5 for the pure data movement, 1e-4 for the layer."""
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import layers as OL
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


def test_gather_rows_backward_sums_repeats(dev):
    from ssla_amd.events import gather_rows
    gen = torch.Generator().manual_seed(0)
    src = torch.randn(500, 24, generator=gen)
    idx = torch.randint(0, 500, (3000,), generator=gen)   # repeats: gradients add up
    w = torch.randn(3000, 24, generator=gen)
    s = src.to(dev).requires_grad_()
    (gather_rows(s, idx.to(dev)) * w.to(dev)).sum().backward()
    s64 = src.double().requires_grad_()
    (s64[idx] * w.double()).sum().backward()
    assert_close(s.grad.cpu().numpy(), s64.grad.numpy(), 1e-5, "d src")


def test_index_add_rows_backward_gathers(dev):
    from ssla_amd.events import gather_patch_events_to_group
    gen = torch.Generator().manual_seed(1)
    pe = torch.randn(2000, 16, generator=gen)
    idx = torch.randint(0, 300, (2000,), generator=gen)
    w = torch.randn(300, 16, generator=gen)
    p = pe.to(dev).requires_grad_()
    (gather_patch_events_to_group(p, idx.to(dev), 300) * w.to(dev)).sum().backward()
    p64 = pe.double().requires_grad_()
    (torch.zeros(300, 16, dtype=torch.float64).index_add(0, idx, p64) * w.double()).sum().backward()
    assert_close(p.grad.cpu().numpy(), p64.grad.numpy(), 1e-5, "d patch events")


def _linear_attention_t64(params, ev, gr):
    """LinearAttention.forward (reference layers/linear_attention.py:39-102)
    in torch float64 on the CPU; the scan is a plain loop."""
    x = ev @ params["input_proj.weight"].T if "input_proj.weight" in params else ev
    lens = np.asarray(gr["lengths"], np.int64)
    ev_b = np.repeat(np.asarray(gr["batch_id"], np.int64), lens)
    t = np.asarray(gr["time"], np.int64)
    order = np.lexsort((np.arange(t.size), t, ev_b))
    counts = np.bincount(ev_b, minlength=int(gr["batch_size"]))
    cu = np.concatenate([[0], np.cumsum(counts[counts > 0])])
    xs = x[torch.from_numpy(order)]
    q, v = xs @ params["q_proj.weight"].T, xs @ params["v_proj.weight"].T
    g = torch.sigmoid(xs @ params["g_proj.weight"].T)
    rows = []
    for s, e in zip(cu[:-1], cu[1:]):
        h = torch.zeros(v.shape[1], dtype=torch.float64)
        for i in range(int(s), int(e)):
            h = h * g[i] + v[i]
            rows.append(h)
    o = (q * torch.stack(rows)) @ params["o_proj.weight"].T
    out = torch.zeros_like(o).index_copy(0, torch.from_numpy(order), o)
    res = ev @ params["residual_proj.weight"].T if "residual_proj.weight" in params else ev
    return F.layer_norm(out + res, (o.shape[1],), params["norm.weight"], params["norm.bias"], eps=1e-5)


@pytest.mark.parametrize("tag,C", [("lin_a", 6), ("lin_b", 8)])
def test_linear_attention_backward(dev, tag, C):
    from ssla_amd.layers import LinearAttention
    fx = np.load(GOLD / "layer_fixtures.npz", allow_pickle=False)
    sd = {k[len(tag) + 4:]: torch.from_numpy(fx[k]) for k in fx.files if k.startswith(f"{tag}_sd_")}
    gr = {k: fx[f"in_{k}"] for k in ("time", "batch_id", "h", "w", "lengths")}
    gr["batch_size"] = int(fx["in_batch_size"])
    ev = torch.from_numpy(fx[f"in_events_c{C}"])
    # the float64 restatement agrees with the oracle's forward (whose scan
    # rounds its inputs to fp32) and with the reference layer's own output
    p64 = {k: v.double().requires_grad_() for k, v in sd.items()}
    e64 = ev.double().requires_grad_()
    y64 = _linear_attention_t64(p64, e64, gr)
    assert np.allclose(y64.detach().numpy(), OL.linear_attention(fx_params(sd), {**gr, "events": ev.numpy()}),
                       rtol=1e-6, atol=1e-6)
    assert np.allclose(y64.detach().numpy(), fx[f"{tag}_out"], rtol=1e-5, atol=1e-5)
    w = torch.randn(y64.shape, generator=torch.Generator().manual_seed(5), dtype=torch.float64)
    (y64 * w).sum().backward()

    layer = LinearAttention(C, 8, tuple(int(v) for v in fx["in_frame"]))
    layer.load_state_dict(sd, strict=True)
    layer = layer.to(dev)
    inp = {k: torch.from_numpy(v).to(dev) for k, v in gr.items() if k != "batch_size"}
    inp["batch_size"] = gr["batch_size"]
    inp["events"] = ev.to(dev).requires_grad_()
    y = layer(inp)["events"]
    (y * w.float().to(dev)).sum().backward()
    assert_close(inp["events"].grad.cpu().numpy(), e64.grad.numpy(), 1e-4, "d events")
    for name, prm in layer.named_parameters():
        assert_close(prm.grad.cpu().numpy(), p64[name].grad.numpy(), 1e-4, f"d {name}")


def fx_params(sd):
    return {k: v.numpy() for k, v in sd.items()}
