"""GPU check of ssla_gla_chunk_fwd_noalloc, the allocation-free variant of
ssla_gla_chunk_fwd for callers that cannot allocate device memory: it runs
the same kernels with a static per-device scratch array in place of the
caller's workspace, so its outputs must equal the workspace entry point's
bit for bit.  Two calls in a row, the second on a smaller input, check that
the scratch left by one call does not leak into the next."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _lib():
    from ssla_amd import _lib
    return _lib, _lib.load()


def _inputs(lens, H, V, seed, dev):
    gen = torch.Generator().manual_seed(seed)
    T = int(sum(lens))
    q = (torch.randn(T, H, 64, generator=gen) / 8).bfloat16().to(dev)
    k = torch.randn(T, H, 64, generator=gen).bfloat16().to(dev)
    v = torch.randn(T, H, V, generator=gen).bfloat16().to(dev)
    g = F.logsigmoid(torch.randn(T, H, 64, generator=gen) / 16).to(dev)
    h0 = (torch.randn(len(lens), H, 64, V, generator=gen) * 0.1).to(dev)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64, device=dev)
    return q, k, v, g, cu, h0


def _both(_l, lib, q, k, v, g, cu, h0):
    T, H, K = q.shape
    V = v.shape[-1]
    N = cu.numel() - 1
    ws_bytes = lib.ssla_gla_chunk_workspace_size(N, T, H, K, V)
    assert ws_bytes > 0, "the case must use a workspace"
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    sh = _l.stream_of(q)
    outs = []
    for noalloc in (False, True):
        o = torch.full_like(v, float("nan"))
        ht = torch.full((N, H, K, V), float("nan"), device=q.device)
        common = (q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), _l.SSLA_F32, cu.data_ptr(), N, T, H, K,
                  V, 1.0, h0.data_ptr(), o.data_ptr(), ht.data_ptr(), _l.SSLA_BF16)
        if noalloc:
            st = lib.ssla_gla_chunk_fwd_noalloc(*common, sh)
        else:
            st = lib.ssla_gla_chunk_fwd(*common, ws.data_ptr(), ws_bytes, sh)
        _l.check(st, "noalloc" if noalloc else "workspace")
        outs.append((o, ht))
    torch.cuda.synchronize()
    return outs


def test_noalloc_matches_workspace_entry_point(dev):
    _l, lib = _lib()
    # C2-like first (8 sequences of 2048 tokens, 8 heads: segments and
    # scratch slots in use), then a smaller ragged batch with fewer heads
    for lens, H, V, seed in (([2048] * 8, 8, 64, 1), ([700, 129, 1, 64], 4, 32, 2)):
        print(f"noalloc vs workspace: lens={lens} H={H} V={V}", flush=True)
        q, k, v, g, cu, h0 = _inputs(lens, H, V, seed, dev)
        (o_ws, ht_ws), (o_na, ht_na) = _both(_l, lib, q, k, v, g, cu, h0)
        assert torch.isfinite(o_ws.float()).all() and torch.isfinite(ht_ws).all()
        assert torch.equal(o_na, o_ws), "o differs from the workspace entry point"
        assert torch.equal(ht_na, ht_ws), "ht differs from the workspace entry point"


def test_noalloc_argument_errors(dev):
    _l, lib = _lib()
    st = lib.ssla_gla_chunk_fwd_noalloc(None, None, None, None, 0, None, -1, 0, 1, 64, 64, 1.0, None, None, None,
                                        _l.SSLA_BF16, None)
    assert st == _l.SSLA_ERR_ARG
    st = lib.ssla_gla_chunk_fwd_noalloc(None, None, None, None, 0, None, 1, 0, 1, 32, 64, 1.0, None, None, None,
                                        _l.SSLA_BF16, None)
    assert st == _l.SSLA_ERR_UNSUPPORTED
