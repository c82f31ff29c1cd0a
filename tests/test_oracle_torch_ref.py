"""CPU pins of oracle.torch_ref (the fp32 PyTorch restatements bench.py
times as the CPU baseline) against the fp64 oracle: the GLA recurrence at
the config-1 shape and on ragged sequences with initial states, the per-bin
sparse scan against the per-site step, and the scatter reductions (max
values and first-index argmax bit for bit, including empty rows and ties)."""
import numpy as np
import torch
import torch.nn.functional as F

import oracle
from oracle import torch_ref


def test_naive_recurrent_matches_oracle():
    gen = torch.Generator().manual_seed(0)
    # config 1: N=1, H=4, T=256, K=V=32, q pre-scaled, scale=1.0, zero state
    q = torch.randn(256, 4, 32, generator=gen) * 32 ** -0.5
    k, v = torch.randn(256, 4, 32, generator=gen), torch.randn(256, 4, 32, generator=gen)
    g = F.logsigmoid(torch.randn(256, 4, 32, generator=gen) / 16)
    cu = torch.tensor([0, 256])
    o, ht = torch_ref.naive_gla_recurrent(q, k, v, g, cu, 1.0, None, True)
    ro, rht = oracle.gla_recurrent(q.numpy(), k.numpy(), v.numpy(), g.numpy(), cu.numpy(), 1.0, None, True)
    assert np.allclose(o.numpy(), ro, rtol=1e-4, atol=1e-5) and np.allclose(ht.numpy(), rht, rtol=1e-4, atol=1e-5)
    # ragged, with initial states
    lens = [0, 5, 70]
    T = sum(lens)
    q, k, v = (torch.randn(T, 2, 16, generator=gen) for _ in range(3))
    g = torch.randn(T, 2, 16, generator=gen) - 1.0
    h0 = torch.randn(3, 2, 16, 16, generator=gen) * 0.1
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]))
    o, ht = torch_ref.naive_gla_recurrent(q, k, v, g, cu, 0.25, h0, True)
    ro, rht = oracle.gla_recurrent(q.numpy(), k.numpy(), v.numpy(), g.numpy(), cu.numpy(), 0.25, h0.numpy(), True)
    assert np.allclose(o.numpy(), ro, rtol=1e-4, atol=1e-5) and np.allclose(ht.numpy(), rht, rtol=1e-4, atol=1e-5)


def test_sparse_scan_bins_matches_steps():
    from ssla_amd import synthetic
    sb = synthetic.sparse_scan_bins(n_bins=6, W=20, Hg=15, seed=2)
    st = sb.state0.clone()
    ref = sb.state0.numpy().copy()
    outs = torch_ref.sparse_scan_bins(st, [torch.from_numpy(s).long() for s in sb.sites], sb.q, sb.k, sb.v, sb.g,
                                      sb.scale)
    for b in range(6):
        ro = oracle.sparse_gla_step(sb.sites[b], sb.q[b].numpy(), sb.k[b].numpy(), sb.v[b].numpy(),
                                    sb.g[b].numpy(), ref, sb.scale)
        assert np.allclose(outs[b].numpy(), ro, rtol=1e-4, atol=1e-5)
    assert np.allclose(st.numpy(), ref, rtol=1e-5, atol=1e-6)


def test_scatter_reductions_match_oracle():
    gen = torch.Generator().manual_seed(4)
    E, C, n_out = 3000, 8, 700          # some rows empty
    src = torch.randint(-4, 5, (E, C), generator=gen).float()   # many ties
    idx = torch.randint(0, n_out, (E,), generator=gen)
    out, arg = torch_ref.scatter_max(src, idx, n_out)
    ro, ra = oracle.scatter_max(src.numpy(), idx.numpy(), n_out)
    assert np.array_equal(out.numpy(), ro) and np.array_equal(arg.numpy(), ra)
    m = torch_ref.scatter_mean(src, idx, n_out)
    assert np.allclose(m.numpy(), oracle.scatter_mean(src.numpy(), idx.numpy(), n_out), rtol=1e-6, atol=1e-6)
