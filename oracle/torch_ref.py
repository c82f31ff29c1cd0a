"""PyTorch fp32 CPU restatements of the reference's CPU-capable paths -- the
CPU BASELINE of bench.py and TEST INFRASTRUCTURE ONLY.

These are written the way the reference's own PyTorch code runs on a CPU
(tensor ops per time step / per bin, library scatter reductions), so that
bench.py can time "the reference's CPU path" on the GPU box's host cores
next to the GPU kernels.  Only ``tests/`` and ``bench.py``'s
``cpu_baseline`` legs use this module.  Each function is pinned against the
fp64 oracle in tests/test_oracle_torch_ref.py.

* naive_gla_recurrent -- ops/gla/naive.py:50-111 (configs 1 and 2).
* sparse_scan_bins    -- the per-bin gather / update / scatter loop of the
  per-site GLA state (config 3): naive_gla_recurrent on length-1 sequences
  whose initial states are the stored site states.
* scatter_max / scatter_mean -- torch_scatter's semantics through
  ``Tensor.scatter_reduce_`` ('amax' / 'mean', include_self=False) plus a
  first-index argmax pass (config 4; torch_scatter itself is not installed).
"""
from __future__ import annotations

import torch


def naive_gla_recurrent(q, k, v, g, cu_seqlens, scale=None, initial_state=None, output_final_state=False):
    """S_t = exp(g_t)[:, :, None] * S_{t-1} + k_t[:, :, None] v_t[:, None, :],
    o_t = einsum('hk,hkv->hv', q_t * scale, S_t), per sequence, in fp32."""
    T, H, K = q.shape
    V = v.shape[-1]
    if scale is None:
        scale = K ** -0.5
    outs, finals = [], []
    cu = [int(x) for x in cu_seqlens.tolist()]
    for n in range(len(cu) - 1):
        s, e = cu[n], cu[n + 1]
        qn, kn, vn, gn = (x[s:e].float() for x in (q, k, v, g))
        S = initial_state[n].float().clone() if initial_state is not None else torch.zeros(H, K, V)
        on = []
        for t in range(e - s):
            S = torch.exp(gn[t])[:, :, None] * S + kn[t][:, :, None] * vn[t][:, None, :]
            on.append(torch.einsum("hk,hkv->hv", qn[t] * scale, S).to(q.dtype))
        outs.append(torch.stack(on, 0) if on else torch.zeros(0, H, V, dtype=q.dtype))
        finals.append(S)
    o = torch.cat(outs, 0)
    return o, (torch.stack(finals, 0) if output_final_state else None)


def sparse_scan_bins(state, sites, q, k, v, g, scale):
    """One pass over the bins: for bin b, gather the states of sites[b],
    update them with the bin's rows, write them back; returns the o of every
    bin.  `state` [n_sites, H, K, V] is updated in place."""
    outs = []
    for b in range(len(sites)):
        idx = sites[b]
        S = state.index_select(0, idx)
        S = torch.exp(g[b])[..., None] * S + k[b][..., None] * v[b][..., None, :]
        outs.append(torch.einsum("nhk,nhkv->nhv", q[b] * scale, S))
        state.index_copy_(0, idx, S)
    return outs


def scatter_max(src, index, n_out):
    """(out, argmax): max over the rows of each output row; argmax the
    smallest event index attaining it; empty rows give 0 and argmax E."""
    E, C = src.shape
    idx = index.view(-1, 1).expand(E, C)
    out = torch.zeros(n_out, C, dtype=src.dtype).scatter_reduce_(0, idx, src, "amax", include_self=False)
    hit = src == out.index_select(0, index)
    cand = torch.where(hit, torch.arange(E).view(-1, 1).expand(E, C), torch.full((E, C), E))
    arg = torch.full((n_out, C), E, dtype=torch.int64).scatter_reduce_(0, idx, cand, "amin", include_self=True)
    return out, arg


def scatter_mean(src, index, n_out):
    E, C = src.shape
    idx = index.view(-1, 1).expand(E, C)
    return torch.zeros(n_out, C, dtype=src.dtype).scatter_reduce_(0, idx, src, "mean", include_self=False)
