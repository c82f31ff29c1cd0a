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


def _random_grouped(dev, n=600, H=12, W=16, C=8, seed=11):
    """A grouped-events dict of one sample: n events on an H x W frame,
    random fp32 features of C channels."""
    from ssla_amd import events as E
    g = torch.Generator().manual_seed(seed)
    ev = torch.zeros(1, n, 4)
    ev[0, :, 0] = torch.randint(0, W, (n,), generator=g).float()
    ev[0, :, 1] = torch.randint(0, H, (n,), generator=g).float()
    ev[0, :, 2] = torch.sort(torch.randint(0, n // 3, (n,), generator=g) * 7).values.float()
    ev[0, :, 3] = 1.0
    gr = E.group_events((ev.to(dev), torch.tensor([n], device=dev)), (H, W))
    gr["events"] = torch.randn(gr["time"].shape[0], C, generator=g).to(dev)
    return gr


@pytest.mark.parametrize("kind", ["max", "mean"])
def test_scatter_backward_matches_torch(dev, kind):
    """scatter_max / scatter_mean gradients against torch's scatter_reduce
    ('amax' / 'mean', include_self=False) autograd in float64 on the CPU
    (random values: no ties, so amax's tie rule does not matter); rows of
    the output without events give no gradient."""
    from ssla_amd.scatter import scatter_max, scatter_mean
    g = torch.Generator().manual_seed(3)
    E_, C, n_out = 5000, 24, 700
    src = torch.randn(E_, C, generator=g)
    idx = torch.randint(0, n_out - 20, (E_,), generator=g)   # the last 20 rows stay empty
    w = torch.randn(n_out, C, generator=g, dtype=torch.float64)
    s64 = src.double().requires_grad_()
    ref = torch.zeros(n_out, C, dtype=torch.float64).scatter_reduce(
        0, idx.view(-1, 1).expand(E_, C), s64, "amax" if kind == "max" else "mean", include_self=False)
    (ref * w).sum().backward()
    sd = src.to(dev).requires_grad_()
    out = (scatter_max if kind == "max" else scatter_mean)(sd, idx.to(dev), dim=0, dim_size=n_out)
    out = out[0] if kind == "max" else out
    assert_close(out.detach().cpu().numpy(), ref.detach().numpy(), 1e-6, f"scatter_{kind} forward")
    (out * w.float().to(dev)).sum().backward()
    assert_close(sd.grad.cpu().numpy(), s64.grad.numpy(), 1e-6, f"scatter_{kind} d src")


def test_sparse_max_pool_backward(dev):
    """SparseMaxPool k=2 end to end (receptive-field gather, pooled
    segments, scatter_max): the gradient of the pixel events against float64
    CPU autograd of the same gather and scatter_reduce('amax'), with the
    receptive-field rows read back from the layer itself (events carrying
    their own index)."""
    from ssla_amd import events as E
    from ssla_amd.layers import SparseMaxPool
    gr = _random_grouped(dev)
    pool = SparseMaxPool((12, 16), kernel_size=(2, 2)).to(dev)
    with torch.no_grad():
        probe = dict(gr)
        probe["events"] = torch.arange(gr["events"].shape[0], device=dev, dtype=torch.float32)[:, None]
        rf = pool.prepare_inputs(probe, True)
        ridx = rf["events"][:, 0].long().cpu()
        seg, seg_time, _ = E.pool_segments(rf["time"], rf["lengths"])
        seg, n_seg = seg.cpu(), int(seg_time.numel())
    ev = gr["events"].detach().requires_grad_()
    out = pool({**gr, "events": ev})["events"]
    assert out.shape[0] == n_seg
    w = torch.randn(out.shape, generator=torch.Generator().manual_seed(8), dtype=torch.float64)
    (out * w.float().to(dev)).sum().backward()
    e64 = gr["events"].detach().cpu().double().requires_grad_()
    rows = e64[ridx]
    ref = torch.zeros(n_seg, rows.shape[1], dtype=torch.float64).scatter_reduce(
        0, seg.view(-1, 1).expand_as(rows), rows, "amax", include_self=False)
    assert_close(out.detach().cpu().numpy(), ref.detach().numpy(), 1e-6, "max pool forward")
    (ref * w).sum().backward()
    assert_close(ev.grad.cpu().numpy(), e64.grad.numpy(), 1e-6, "max pool d events")


def _mos_t64(p, ev, src, pos, f_len, H, sp, gp):
    """MosAttention.forward (reference layers/mos_attention.py:75-146) in
    torch float64 on the CPU, on given patch rows (src: pixel event, pos:
    kernel position; rows of each patch consecutive in time order)."""
    Cin = ev.shape[1]
    Ws = p["scatter_conv_weights"].reshape(-1, H, Cin)
    Wgp = p["gather_conv_weights"].reshape(-1, H, H)
    xe = ev[src]
    x = torch.einsum("rhc,rc->rh", Ws[pos] if sp else Ws[torch.zeros_like(pos)], xe)
    q, v = x @ p["q_proj.weight"].T, x @ p["v_proj.weight"].T
    a = torch.sigmoid(x @ p["g_proj.weight"].T)
    hs, r0 = [], 0
    for n in f_len.tolist():
        h = torch.zeros(H, dtype=torch.float64)
        for r in range(r0, r0 + n):
            h = a[r] * h + v[r]
            hs.append(h)
        r0 += n
    o = (q * torch.stack(hs)) @ p["o_proj.weight"].T
    z = torch.einsum("rhk,rk->rh", Wgp[pos] if gp else Wgp[torch.zeros_like(pos)], o)
    y = torch.zeros(ev.shape[0], H, dtype=torch.float64).index_add(0, src, z)
    res = ev @ p["input_proj.weight"].T if "input_proj.weight" in p else ev
    return F.layer_norm(y + res, (H,), p["norm.weight"], p["norm.bias"], eps=1e-5)


@pytest.mark.parametrize("cin,hid,sp,gp", [(8, 12, True, True), (12, 12, False, True), (8, 16, True, False)])
def test_mos_attention_backward(dev, cin, hid, sp, gp):
    """The composed MosAttention forward trains: gradients of the pixel
    events and of every parameter against float64 CPU autograd of the same
    layer on the same patch rows (read from the layer's own scatter)."""
    from ssla_amd import events as E
    from ssla_amd.layers import MosAttention
    torch.manual_seed(cin * 10 + hid)
    gr = _random_grouped(dev, C=cin, seed=cin + hid)
    layer = MosAttention(cin, hid, (12, 16), (3, 3), scatter_proj=sp, gather_proj=gp).to(dev)
    with torch.no_grad():
        layer(gr, fused=False)   # builds the lookup table
        src, _t, pos, _fi, f_len, _n = E._rf_scatter(gr, layer.frame_size, layer.patch2pixel_lut)
        src, pos, f_len = src.cpu(), pos.cpu(), f_len.cpu()
    ev = gr["events"].detach().requires_grad_()
    y = layer({**gr, "events": ev}, fused=False)["events"]
    w = torch.randn(y.shape, generator=torch.Generator().manual_seed(2), dtype=torch.float64)
    (y * w.float().to(dev)).sum().backward()
    p64 = {k: v.detach().cpu().double().requires_grad_() for k, v in layer.named_parameters()}
    e64 = gr["events"].detach().cpu().double().requires_grad_()
    y64 = _mos_t64(p64, e64, src, pos, f_len, hid, sp, gp)
    assert_close(y.detach().cpu().numpy(), y64.detach().numpy(), 1e-4, "mos forward")
    (y64 * w).sum().backward()
    assert_close(ev.grad.cpu().numpy(), e64.grad.numpy(), 1e-4, "mos d events")
    for name, prm in layer.named_parameters():
        assert_close(prm.grad.cpu().numpy(), p64[name].grad.numpy(), 1e-4, f"mos d {name}")
