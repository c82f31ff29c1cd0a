"""Pins of the CPU oracle (oracle/), run on the CPU.

The reference holds no golden vectors or known-answer tests for this path
(its only self-check, ops/gla/naive.py:114-129, compares its parallel and
recurrent forms).  Each oracle function is therefore pinned by checks that
a plausible mistake (dropped term, wrong sign or index, transposed operand,
o from the previous state) fails:

* gla_recurrent: agreement with two independently coded algorithms (the
  quadratic parallel form of naive.py:6-47 and the chunked form of
  chunk.py:906-960 at several chunk sizes); closed forms for g = 0
  (cumulative linear attention), k = 0 (pure decay of S0) and T = 1;
  split-and-carry invariance; the reference's own self-check shape.
  test_planted_mistakes_are_caught shows mutated recurrences fail these.
* diag_scan: geometric closed form for constant gates, brute-force
  products, and equality with gla_recurrent at K = V = 1.
* diag_scan_bwd: torch autograd (fp64) through a loop of the forward,
  suffix-sum closed form for unit gates, central differences.
* sparse_gla_step: equality with gla_recurrent on length-1 sequences with
  initial_state = the stored state; inactive rows untouched byte for byte.
* scatter_max / scatter_mean: torch.scatter_reduce('amax'/'mean',
  include_self=False) for values, brute-force first-index argmax, forced
  ties, empty rows.
"""
import numpy as np
import pytest
import torch

import oracle


def _rand(rng, *shape):
    return rng.standard_normal(shape).astype(np.float32)


def _gla_inputs(rng, lens, H, K, V, gate=-1.0):
    T = int(sum(lens))
    q, k, v = _rand(rng, T, H, K), _rand(rng, T, H, K), _rand(rng, T, H, V)
    g = (_rand(rng, T, H, K) + gate).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    return q, k, v, g, cu


# ----------------------------------------------------------------- GLA ----
def test_recurrent_vs_parallel_and_chunked():
    rng = np.random.default_rng(0)
    q, k, v, g, cu = _gla_inputs(rng, [37, 0, 1, 64, 70], 2, 8, 5)
    o_r, _ = oracle.gla_recurrent(q, k, v, g, cu, output_final_state=False)
    o_p = oracle.gla_parallel(q, k, v, g, cu)
    assert np.allclose(o_r, o_p, rtol=1e-10, atol=1e-10)
    s0 = _rand(rng, 5, 2, 8, 5)
    o_r, h_r = oracle.gla_recurrent(q, k, v, g, cu, 0.3, s0)
    for bt in (1, 3, 16, 64):
        o_c, h_c = oracle.gla_chunk(q, k, v, g, cu, 0.3, s0, chunk_size=bt)
        assert np.allclose(o_r, o_c, rtol=1e-10, atol=1e-10), bt
        assert np.allclose(h_r, h_c, rtol=1e-10, atol=1e-10), bt


def test_reference_self_check_shape():
    """The reference's own check (ops/gla/naive.py:114-129): T=512, H=16,
    K=V=64, g = randn - 1, cu = [0, 170, 298, 512], parallel == recurrent."""
    rng = np.random.default_rng(0)
    T, H, K, V = 512, 16, 64, 64
    q, k, v = _rand(rng, T, H, K), _rand(rng, T, H, K), _rand(rng, T, H, V)
    g = (_rand(rng, T, H, K) - 1.0).astype(np.float32)
    cu = np.array([0, T // 3, T // 3 + T // 4, T])
    o_p = oracle.gla_parallel(q, k, v, g, cu)
    o_r, _ = oracle.gla_recurrent(q, k, v, g, cu, output_final_state=False)
    assert np.allclose(o_p, o_r, rtol=1e-9, atol=1e-9)


def test_zero_gates_is_cumulative_linear_attention():
    rng = np.random.default_rng(1)
    q, k, v, _, cu = _gla_inputs(rng, [20, 9], 3, 4, 6)
    g = np.zeros_like(q)
    o, _ = oracle.gla_recurrent(q, k, v, g, cu, 0.7)
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    ref = np.zeros_like(o)
    for n in range(2):
        s, e = cu[n], cu[n + 1]
        for t in range(s, e):
            for u in range(s, t + 1):
                ref[t] += 0.7 * np.einsum("hk,hk->h", q[t], k[u])[:, None] * v[u]
    assert np.allclose(o, ref, rtol=1e-10, atol=1e-10)


def test_zero_keys_is_pure_decay():
    rng = np.random.default_rng(2)
    q, _, v, g, cu = _gla_inputs(rng, [15], 2, 5, 3)
    k = np.zeros_like(q)
    s0 = _rand(rng, 1, 2, 5, 3)
    o, ht = oracle.gla_recurrent(q, k, v, g, cu, 0.5, s0)
    G = np.cumsum(g.astype(np.float64), axis=0)                 # [T, H, K]
    ref = 0.5 * np.einsum("thk,thk,hkv->thv", q, np.exp(G), s0[0])
    assert np.allclose(o, ref, rtol=1e-10, atol=1e-12)
    assert np.allclose(ht[0], np.exp(G[-1])[:, :, None] * s0[0], rtol=1e-10)


def test_single_step_closed_form():
    rng = np.random.default_rng(3)
    q, k, v, g, cu = _gla_inputs(rng, [1], 2, 4, 3)
    s0 = _rand(rng, 1, 2, 4, 3)
    o, ht = oracle.gla_recurrent(q, k, v, g, cu, 0.25, s0)
    q, k, v, s0 = (a.astype(np.float64) for a in (q, k, v, s0))
    S1 = np.exp(g[0].astype(np.float64))[:, :, None] * s0[0] + k[0][:, :, None] * v[0][:, None, :]
    assert np.allclose(ht[0], S1, rtol=1e-12)
    assert np.allclose(o[0], 0.25 * np.einsum("hk,hkv->hv", q[0], S1), rtol=1e-12)


def test_split_and_carry_state():
    rng = np.random.default_rng(4)
    q, k, v, g, cu = _gla_inputs(rng, [50], 2, 6, 4)
    s0 = _rand(rng, 1, 2, 6, 4)
    o, ht = oracle.gla_recurrent(q, k, v, g, cu, 0.4, s0)
    a = 23
    o1, h1 = oracle.gla_recurrent(q[:a], k[:a], v[:a], g[:a], [0, a], 0.4, s0)
    o2, h2 = oracle.gla_recurrent(q[a:], k[a:], v[a:], g[a:], [0, 50 - a], 0.4, h1.astype(np.float32))
    assert np.allclose(np.concatenate([o1, o2]), o, rtol=1e-6, atol=1e-6)  # h1 rounded to fp32
    assert np.allclose(h2, ht, rtol=1e-6, atol=1e-6)


def test_default_scale_and_prescaled_q():
    rng = np.random.default_rng(5)
    q, k, v, g, cu = _gla_inputs(rng, [12], 1, 16, 2)
    o1, _ = oracle.gla_recurrent(q, k, v, g, cu)                     # scale = K^-1/2
    o2, _ = oracle.gla_recurrent(q * 0.25, k, v, g, cu, 1.0)         # pre-scaled, scale = 1
    assert np.allclose(o1, o2, rtol=1e-6)


def _np_recurrent(q, k, v, g, scale, s0, mistake=None):
    """Single-sequence numpy recurrence with optional planted mistakes."""
    q, k, v, g = (a.astype(np.float64) for a in (q, k, v, g))
    S = s0.astype(np.float64).copy()
    out = []
    for t in range(q.shape[0]):
        d = np.exp(-g[t] if mistake == "sign" else g[t])[:, :, None]
        kv = k[t][:, :, None] * v[t][:, None, :]
        prev = S
        S = d * (S + kv) if mistake == "order" else d * S + kv
        src = prev if mistake == "prev" else S
        qq = k[t] if mistake == "swap" else q[t]
        out.append(scale * np.einsum("hk,hkv->hv", qq, src))
    return np.stack(out), S


@pytest.mark.parametrize("mistake", ["sign", "order", "prev", "swap"])
def test_planted_mistakes_are_caught(mistake):
    """A mutated recurrence must disagree with the oracle and with at least
    one closed form (so the pins have teeth)."""
    rng = np.random.default_rng(6)
    q, k, v, g, cu = _gla_inputs(rng, [6], 2, 4, 3)
    s0 = _rand(rng, 1, 2, 4, 3)
    good, _ = _np_recurrent(q, k, v, g, 0.5, s0[0])
    ref, _ = oracle.gla_recurrent(q, k, v, g, cu, 0.5, s0)
    assert np.allclose(good, ref, rtol=1e-10, atol=1e-12)
    bad, _ = _np_recurrent(q, k, v, g, 0.5, s0[0], mistake)
    assert not np.allclose(bad, ref, rtol=1e-3, atol=1e-3)
    # the T = 1 closed form alone also catches it
    q0, k0, v0, s00 = (a.astype(np.float64) for a in (q[0], k[0], v[0], s0[0]))
    S1 = np.exp(g[0].astype(np.float64))[:, :, None] * s00 + k0[:, :, None] * v0[:, None, :]
    closed = 0.5 * np.einsum("hk,hkv->hv", q0, S1)
    assert np.allclose(good[0], closed, rtol=1e-10)
    assert not np.allclose(bad[0], closed, rtol=1e-3, atol=1e-3)


# ---------------------------------------------------------------- scan ----
def test_scan_constant_gate_closed_form():
    T, C = 40, 3
    gval = np.array([0.5, 0.9, 0.99], np.float32)
    u = np.ones((T, C), np.float32)
    g = np.tile(gval, (T, 1))
    h = oracle.diag_scan(u, g, [0, T])
    t = np.arange(T)[:, None]
    ref = (1 - gval.astype(np.float64) ** (t + 1)) / (1 - gval.astype(np.float64))
    assert np.allclose(h, ref, rtol=1e-6)  # gval is rounded to fp32 in both


def test_scan_brute_force_and_zero_rows():
    rng = np.random.default_rng(7)
    T, C = 30, 4
    u = _rand(rng, T, C)
    g = (1 / (1 + np.exp(-_rand(rng, T, C)))).astype(np.float32)
    cu = np.array([2, 9, 9, 25])
    h = oracle.diag_scan(u, g, cu)
    ref = np.zeros((T, C))
    for s, e in ((2, 9), (25, 25), (9, 25)):
        for t in range(s, e):
            for r in range(s, t + 1):
                ref[t] += np.prod(g[r + 1:t + 1].astype(np.float64), axis=0) * u[r]
    assert np.allclose(h, ref, rtol=1e-10, atol=1e-12)
    assert (h[:2] == 0).all() and (h[25:] == 0).all()


def test_scan_is_gla_with_unit_keys():
    """scan == GLA with H = C heads, K = V = 1, q = k = 1, v = u, g = log g."""
    rng = np.random.default_rng(8)
    T, C = 25, 5
    u = _rand(rng, T, C)
    g = (1 / (1 + np.exp(-_rand(rng, T, C)))).astype(np.float32)
    cu = np.array([0, 11, 25])
    h = oracle.diag_scan(u, g, cu)
    ones = np.ones((T, C, 1), np.float32)
    o, _ = oracle.gla_recurrent(ones, ones, u[:, :, None], np.log(g)[:, :, None], cu, 1.0)
    assert np.allclose(h, o[:, :, 0], rtol=1e-6, atol=1e-7)


def _scan_autograd(u, g, cu, dout):
    """(du, dg) by torch autograd (float64, CPU) through a plain loop of the
    forward recurrence: an independent derivation of the backward."""
    U = torch.tensor(u, dtype=torch.float64, requires_grad=True)
    G = torch.tensor(g, dtype=torch.float64, requires_grad=True)
    rows = [torch.zeros(u.shape[1], dtype=torch.float64) for _ in range(u.shape[0])]
    for s, e in zip(cu[:-1], cu[1:]):
        hprev = torch.zeros(u.shape[1], dtype=torch.float64)
        for t in range(int(s), int(e)):
            hprev = hprev * G[t] + U[t]
            rows[t] = hprev
    (torch.stack(rows) * torch.tensor(dout, dtype=torch.float64)).sum().backward()
    return U.grad.numpy(), G.grad.numpy()


def test_scan_bwd_matches_autograd():
    rng = np.random.default_rng(21)
    T, C = 37, 6
    u, dout = _rand(rng, T, C), _rand(rng, T, C)
    g = (1 / (1 + np.exp(-_rand(rng, T, C)))).astype(np.float32)
    cu = np.array([3, 10, 10, 31])   # leading / trailing rows in no sequence, an empty sequence
    du, dg = oracle.diag_scan_bwd(u, g, dout, cu)
    rdu, rdg = _scan_autograd(u, g, cu, dout)
    assert np.allclose(du, rdu, rtol=1e-12, atol=1e-12) and np.allclose(dg, rdg, rtol=1e-12, atol=1e-12)
    assert (du[:3] == 0).all() and (dg[31:] == 0).all()


def test_scan_bwd_unit_gate_closed_form_and_finite_differences():
    rng = np.random.default_rng(22)
    T, C = 20, 3
    u, dout = _rand(rng, T, C), _rand(rng, T, C)
    ones = np.ones((T, C), np.float32)
    du, dg = oracle.diag_scan_bwd(u, ones, dout, [0, T])
    suffix = np.cumsum(dout[::-1].astype(np.float64), axis=0)[::-1]   # g = 1: du_t = sum_{s>=t} do_s
    assert np.allclose(du, suffix, rtol=1e-12)
    h = np.cumsum(u.astype(np.float64), axis=0)
    assert np.allclose(dg[1:], suffix[1:] * h[:-1], rtol=1e-12) and (dg[0] == 0).all()
    # central differences of the fp64 forward along a random direction
    g = (0.5 + 0.4 * np.tanh(_rand(rng, T, C))).astype(np.float32)
    du, dg = oracle.diag_scan_bwd(u, g, dout, [0, T])
    dirg = _rand(rng, T, C).astype(np.float64)
    eps = 1e-3
    def loss(gg):
        return float((oracle.diag_scan(u, gg.astype(np.float32), [0, T]) * dout).sum())
    # the forward rounds g to fp32: use a direction exactly representable after scaling
    gp, gm = g.astype(np.float64) + eps * dirg, g.astype(np.float64) - eps * dirg
    fd = (loss(gp) - loss(gm)) / (2 * eps)
    assert abs(fd - float((dg * dirg).sum())) < 1e-3 * (1 + abs(fd))


def test_scan_bwd_planted_mistake_is_caught():
    """dg from h_t instead of h_{t-1} (an off-by-one) fails the autograd check."""
    rng = np.random.default_rng(23)
    T, C = 15, 2
    u, dout = _rand(rng, T, C), _rand(rng, T, C)
    g = (1 / (1 + np.exp(-_rand(rng, T, C)))).astype(np.float32)
    h = oracle.diag_scan(u, g, [0, T])
    du, _ = oracle.diag_scan_bwd(u, g, dout, [0, T])
    wrong_dg = du * h
    _, rdg = _scan_autograd(u, g, np.array([0, T]), dout)
    assert not np.allclose(wrong_dg, rdg, rtol=1e-3, atol=1e-3)


# --------------------------------------------------------- sparse step ----
def test_sparse_step_is_recurrent_on_length_one():
    rng = np.random.default_rng(9)
    n_sites, H, K, V = 30, 2, 4, 4
    state = _rand(rng, n_sites, H, K, V)
    before = state.copy()
    sites = np.array([1, 4, 5, 17, 29], np.int32)
    n = sites.size
    q, k, g = _rand(rng, n, H, K), _rand(rng, n, H, K), (_rand(rng, n, H, K) - 1).astype(np.float32)
    v = _rand(rng, n, H, V)
    o = oracle.sparse_gla_step(sites, q, k, v, g, state, 0.3)
    o_ref, h_ref = oracle.gla_recurrent(q, k, v, g, np.arange(n + 1), 0.3, before[sites])
    assert np.allclose(o, o_ref, rtol=1e-6, atol=1e-6)
    assert np.allclose(state[sites], h_ref, rtol=1e-6, atol=1e-6)
    inactive = np.setdiff1d(np.arange(n_sites), sites)
    assert state[inactive].tobytes() == before[inactive].tobytes()


# ------------------------------------------------------------- scatter ----
def _torch_reduce(src, index, n_out, how):
    out = torch.zeros(n_out, src.shape[1])
    idx = torch.from_numpy(index).unsqueeze(1).expand(-1, src.shape[1])
    return out.scatter_reduce(0, idx, torch.from_numpy(src), reduce=how, include_self=False).numpy()


@pytest.mark.parametrize("ties", [False, True])
def test_scatter_max_vs_torch_and_brute_force(ties):
    rng = np.random.default_rng(10)
    E, C, n_out = 400, 6, 30
    src = rng.integers(-2, 3, size=(E, C)).astype(np.float32) if ties else _rand(rng, E, C)
    index = rng.integers(0, n_out - 3, size=E)
    out, arg = oracle.scatter_max(src, index, n_out)
    assert np.array_equal(out, _torch_reduce(src, index, n_out, "amax"))
    for r in range(n_out):
        rows = np.nonzero(index == r)[0]
        for c in range(C):
            if rows.size == 0:
                assert out[r, c] == 0 and arg[r, c] == E
            else:
                m = src[rows, c].max()
                assert arg[r, c] == rows[src[rows, c] == m][0]    # smallest index wins
                assert out[r, c] == m


def test_scatter_max_nan_never_wins_and_neg_inf_ties():
    """NaN never wins (all-NaN rows count as empty, as with an initial value
    below every number); -inf is an ordinary value whose ties keep the
    first event."""
    nan, inf = np.nan, np.inf
    src = np.array([[nan], [5.0], [nan], [nan], [-inf], [-inf], [2.0], [nan]], np.float32)
    index = np.array([0, 0, 1, 1, 2, 2, 3, 3])
    out, arg = oracle.scatter_max(src, index, 5)
    assert arg[:, 0].tolist() == [1, 8, 4, 6, 8]
    assert out[:, 0].tolist() == [5.0, 0.0, -inf, 2.0, 0.0]


def test_scatter_max_signed_zero_takes_first_bits():
    src = np.array([[0.0], [-0.0], [-1.0]], np.float32)
    out, arg = oracle.scatter_max(src[[1, 0, 2]], np.array([0, 0, 0]), 1)
    assert arg[0, 0] == 0 and np.signbit(out[0, 0])     # -0.0 came first


def test_scatter_mean_vs_torch():
    rng = np.random.default_rng(11)
    E, C, n_out = 500, 5, 40
    src = _rand(rng, E, C)
    index = rng.integers(0, n_out - 2, size=E)
    out = oracle.scatter_mean(src, index, n_out)
    assert np.allclose(out, _torch_reduce(src, index, n_out, "mean"), rtol=1e-5, atol=1e-6)
    cnt = np.bincount(index, minlength=n_out)
    ref = np.stack([np.bincount(index, weights=src[:, c].astype(np.float64), minlength=n_out)
                    for c in range(C)], 1) / np.maximum(cnt, 1)[:, None]
    assert np.allclose(out, ref, rtol=1e-12, atol=1e-12)
    assert (out[cnt == 0] == 0).all()


# ------------------------------------------------------- GLA backward ----
def _gla_autograd(q, k, v, g, cu, scale, h0, dout, dht):
    """Gradients by torch autograd (float64, CPU) through a plain loop of the
    recurrence S_t = e^{g_t} S_{t-1} + k_t v_t^T, o_t = scale q_t S_t."""
    tq, tk, tv, tg = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v, g))
    th0 = None if h0 is None else torch.tensor(h0, dtype=torch.float64, requires_grad=True)
    T, H, K = q.shape
    V = v.shape[-1]
    outs = [None] * T
    finals = []
    for n in range(len(cu) - 1):
        S = th0[n] if th0 is not None else torch.zeros(H, K, V, dtype=torch.float64)
        for t in range(int(cu[n]), int(cu[n + 1])):
            S = torch.exp(tg[t])[:, :, None] * S + tk[t][:, :, None] * tv[t][:, None, :]
            outs[t] = torch.einsum("hk,hkv->hv", tq[t] * scale, S)
        finals.append(S)
    o = torch.stack([x if x is not None else torch.zeros(H, V, dtype=torch.float64) for x in outs])
    loss = (o * torch.tensor(dout, dtype=torch.float64)).sum()
    if dht is not None:
        loss = loss + (torch.stack(finals) * torch.tensor(dht, dtype=torch.float64)).sum()
    loss.backward()
    return tq.grad.numpy(), tk.grad.numpy(), tv.grad.numpy(), tg.grad.numpy(), (
        None if th0 is None else th0.grad.numpy())


@pytest.mark.parametrize("with_state", [False, True])
def test_gla_bwd_matches_autograd(with_state):
    rng = np.random.default_rng(31)
    lens, H, K, V = [70, 0, 5, 140], 2, 6, 5   # crosses the oracle's 64-step checkpoints
    q, k, v, g, cu = _gla_inputs(rng, lens, H, K, V, gate=-0.5)
    g = np.minimum(g, 0).astype(np.float32)
    dout = _rand(rng, q.shape[0], H, V)
    h0 = _rand(rng, len(lens), H, K, V) * 0.3 if with_state else None
    dht = _rand(rng, len(lens), H, K, V) if with_state else None
    got = oracle.gla_recurrent_bwd(q, k, v, g, cu, dout, 0.7, h0, dht)
    ref = _gla_autograd(q, k, v, g, cu, 0.7, h0, dout, dht)
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dh0"), got, ref):
        if b is None:
            assert a is None
            continue
        assert np.allclose(a, b, rtol=1e-10, atol=1e-10), name


def test_gla_bwd_dg_identity_and_finite_differences():
    """dg = reverse cumsum of (q dq - k dk) plus dht . ht (per sequence), and
    a central difference of the fp64 forward along a random direction."""
    rng = np.random.default_rng(32)
    lens, H, K, V = [90], 1, 4, 3
    q, k, v, g, cu = _gla_inputs(rng, lens, H, K, V, gate=-0.5)
    g = np.minimum(g, 0).astype(np.float32)
    dout = _rand(rng, 90, H, V)
    h0 = _rand(rng, 1, H, K, V) * 0.3
    dht = _rand(rng, 1, H, K, V)
    dq, dk, dv, dg, dh0 = oracle.gla_recurrent_bwd(q, k, v, g, cu, dout, 1.0, h0, dht)
    _, ht = oracle.gla_recurrent(q, k, v, g, cu, 1.0, h0, True)
    r = q.astype(np.float64) * dq - k.astype(np.float64) * dk
    want = np.cumsum(r[::-1], axis=0)[::-1] + (dht[0] * ht[0]).sum(-1)[None]
    assert np.allclose(dg, want, rtol=1e-9, atol=1e-9)
    d = _rand(rng, 90, H, K).astype(np.float64)
    eps = 1e-4

    def loss(gg):
        o, s = oracle.gla_recurrent(q, k, v, gg.astype(np.float32), cu, 1.0, h0, True)
        return float((o * dout).sum() + (s * dht).sum())
    fd = (loss(g + eps * d) - loss(g - eps * d)) / (2 * eps)
    assert abs(fd - float((dg * d).sum())) < 2e-3 * (1 + abs(fd))


def test_chunk_rounding_emulation_pinned():
    """oracle.chunk_ref (the reference's chunk pipeline with its rounding
    points) pinned two ways: with every rounding dropped it equals the fp64
    recurrence to fp32 precision on ragged sequences with chunk remainders
    and an initial state (so its chunk algebra -- sub-chunk A with the
    re-centred decays, the diagonal blocks, the entering states, the state
    update -- is right); with the roundings on, its error is that of bf16
    operands (an RMS ratio of a few 1e-3, and not zero), and its o values are
    bf16 values."""
    from oracle import chunk_ref
    rng = np.random.default_rng(5)
    lens = [70, 1, 64, 130, 17]
    T, H, K, V = sum(lens), 2, 32, 48
    q = (rng.standard_normal((T, H, K)) * K ** -0.5).astype(np.float32)
    k = rng.standard_normal((T, H, K)).astype(np.float32)
    v = rng.standard_normal((T, H, V)).astype(np.float32)
    g = np.log(1 / (1 + np.exp(-rng.standard_normal((T, H, K)) / 2))).astype(np.float32)   # logsigmoid
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    h0 = (rng.standard_normal((len(lens), H, K, V)) * 0.1).astype(np.float32)
    qb, kb, vb = (chunk_ref.bf16(x) for x in (q, k, v))
    ro, rht = oracle.gla_recurrent(qb, kb, vb, g, cu, 1.0, h0, True)
    eo, eht = chunk_ref.chunk_gla(qb, kb, vb, g, cu, 1.0, h0, exact=True)
    np.testing.assert_allclose(eo, ro, rtol=2e-4, atol=2e-4 * np.sqrt(np.mean(ro ** 2)))
    np.testing.assert_allclose(eht, rht, rtol=2e-4, atol=2e-4 * np.sqrt(np.mean(rht ** 2)))
    bo, bht = chunk_ref.chunk_gla(q, k, v, g, cu, 1.0, h0)
    ratio = np.sqrt(np.mean((bo - ro) ** 2) / np.mean(ro ** 2))
    assert 1e-4 < ratio < 1e-2, ratio
    assert np.array_equal(chunk_ref.bf16(bo), bo)
    # a planted mistake in the emulation (the state entering a chunk taken
    # after the chunk's update) is caught by the exact comparison
    bad = chunk_ref._chunk
    try:
        def swapped(q_, k_, v_, G_, S_, scale_, rb, rt):
            _, S2 = bad(q_, k_, v_, G_, S_, scale_, rb, rt)
            o2, _ = bad(q_, k_, v_, G_, S2, scale_, rb, rt)
            return o2, S2
        chunk_ref._chunk = swapped
        wo, _ = chunk_ref.chunk_gla(qb, kb, vb, g, cu, 1.0, h0, exact=True)
    finally:
        chunk_ref._chunk = bad
    assert not np.allclose(wo, ro, rtol=2e-4, atol=2e-4 * np.sqrt(np.mean(ro ** 2)))
