"""GPU parity: chunk_gla backward (ChunkGLAFunction.backward ->
ssla_gla_chunk_bwd) vs the fp64 CPU oracle of the recurrent backward
(oracle.gla_recurrent_bwd, pinned against torch autograd in
tests/test_oracle.py).  The products run as split bf16 triples with fp32
accumulation and the gradients are rounded to the input dtype at the end.
Each gradient of each case is held to twice its measured error on the
MI355X: every element within `band * rms` and RMSE / RMS within
`ratio_max` (measured: dq, dk, dv 0.17 %, which is bf16 output rounding;
dg <= 0.7 % with gates below -5; the north star's bar for bf16 is 2e-2)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu

# (band, ratio_max) per case and gradient, <= 2x measured (dg of the
# strong-gate case keeps the earlier 1e-2 ratio bound, 1.5x measured)
_B16 = {"dq": (0.053, 3.3e-3), "dk": (0.051, 3.3e-3), "dv": (0.05, 3.3e-3), "dg": (1.1e-3, 1e-4), "dh0": (1.1e-4, 4e-6)}
BANDS = {
    "logsig": _B16,
    "randn-1": {"dq": (0.31, 3.4e-3), "dk": (0.45, 3.4e-3), "dv": (0.24, 3.3e-3), "dg": (3.4e-3, 7e-5),
                "dh0": (3.3e-4, 4.9e-6)},
    "strong": {"dq": (0.059, 3.3e-3), "dk": (0.059, 3.3e-3), "dv": (0.059, 3.3e-3), "dg": (0.127, 1e-2),
               "dh0": (2.1e-6, 6.8e-8)},
    "zero": {"dq": (0.041, 3.3e-3), "dk": (0.041, 3.3e-3), "dv": (0.03, 3.3e-3), "dg": (3.4e-5, 4.4e-6),
             "dh0": (2.5e-6, 1.3e-7)},
    "no h0": {"dq": (0.027, 3.3e-3), "dk": (0.046, 3.3e-3), "dv": (0.027, 3.3e-3), "dg": (4.4e-4, 8.7e-5)},
    "fp16": {"dq": (6.9e-3, 4.2e-4), "dk": (6.7e-3, 4.2e-4), "dv": (3.3e-3, 4e-4), "dg": (6.4e-4, 9.3e-5),
             "dh0": (9.3e-5, 6.3e-6)},
    "long": {"dq": (0.053, 3.3e-3), "dk": (0.054, 3.3e-3), "dv": (0.053, 3.3e-3), "dg": (9.4e-4, 1e-4),
             "dh0": (6e-5, 5e-6)},
    "16-bit g bf16": {"dq": (0.11, 3.2e-3), "dk": (0.22, 3.4e-3), "dv": (0.099, 3.4e-3), "dg": (0.14, 3.1e-3),
                      "dh0": (2.4e-4, 4.8e-6)},
    "K=32": {"dq": (0.042, 3.3e-3), "dk": (0.027, 3.4e-3), "dv": (0.05, 3.3e-3), "dg": (6.6e-4, 9.5e-5),
             "dh0": (7.9e-5, 4.6e-6)},
    "K=128": {"dq": (0.053, 3.3e-3), "dk": (0.051, 3.3e-3), "dv": (0.058, 4.9e-3), "dg": (6.2e-4, 1e-4),
              "dh0": (6.9e-5, 3.7e-6)},
    "16-bit g fp16": {"dq": (0.02, 4.3e-4), "dk": (0.016, 4.1e-4), "dv": (8.4e-3, 4.2e-4), "dg": (0.016, 3.8e-4),
                      "dh0": (3.6e-4, 6.8e-6)},
    # value groups: the bf16 bands of the logsig case (one more rounding
    # of dq, dk, dg, which add up over the groups in fp32)
    "value groups": _B16,
}


def _inputs(lens, H, V, dtype, seed, gate="logsig", h0=True, K=64):
    gen = torch.Generator().manual_seed(seed)
    T = int(sum(lens))
    q, k = torch.randn(T, H, K, generator=gen), torch.randn(T, H, K, generator=gen)
    v = torch.randn(T, H, V, generator=gen)
    if gate == "logsig":
        g = F.logsigmoid(torch.randn(T, H, K, generator=gen) / 16)
    elif gate == "randn-1":
        g = torch.randn(T, H, K, generator=gen) - 1.0
    elif gate == "strong":
        g = -5.0 - torch.rand(T, H, K, generator=gen)
    else:
        g = torch.zeros(T, H, K)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int64)
    s0 = torch.randn(len(lens), H, K, V, generator=gen) * 0.1 if h0 else None
    do = torch.randn(T, H, V, generator=gen)
    dht = torch.randn(len(lens), H, K, V, generator=gen) * 0.1 if h0 else None
    return q.to(dtype), k.to(dtype), v.to(dtype), g, cu, s0, do.to(dtype), dht


def _gpu_grads(dev, q, k, v, g, cu, s0, do, dht, scale):
    from ssla_amd.gla import chunk_gla
    leaves = [t.to(dev).requires_grad_() for t in (q, k, v, g)]
    h0 = s0.to(dev).requires_grad_() if s0 is not None else None
    o, ht = chunk_gla(*leaves, cu.to(dev), scale=scale, initial_state=h0, output_final_state=dht is not None)
    loss = (o.float() * do.to(dev).float()).sum()
    if dht is not None:
        loss = loss + (ht * dht.to(dev)).sum()
    loss.backward()
    out = [t.grad.float().cpu().numpy() for t in leaves]
    out.append(h0.grad.cpu().numpy() if h0 is not None else None)
    return out


def _check(dev, lens, H, V, dtype, seed, gate="logsig", h0=True, scale=64 ** -0.5, tag="", case=None, K=64):
    q, k, v, g, cu, s0, do, dht = _inputs(lens, H, V, dtype, seed, gate, h0, K=K)
    print(f"gla bwd {tag}: lens={lens} H={H} V={V} {dtype} gate={gate} h0={h0}", flush=True)
    got = _gpu_grads(dev, q, k, v, g, cu, s0, do, dht, scale)
    ref = oracle.gla_recurrent_bwd(q.float().numpy(), k.float().numpy(), v.float().numpy(), g.numpy(), cu.numpy(),
                                   do.float().numpy(), scale, None if s0 is None else s0.numpy(),
                                   None if dht is None else dht.numpy())
    bands = BANDS[case or gate]
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dh0"), got, ref):
        if b is None:
            assert a is None
            continue
        band, ratio_max = bands[name]
        assert_close(a, b, 0.0, f"{name}[{tag}]", band=band, ratio_max=ratio_max)


@pytest.mark.parametrize("V", [16, 32, 48, 64])
@pytest.mark.parametrize("gate", ["logsig", "randn-1", "strong", "zero"])
def test_chunk_bwd_varlen(dev, V, gate):
    """Ragged sequences (empty, 1, chunk - 1, chunk, chunk + 1, long) in
    every gate regime, with an initial state and a final-state gradient."""
    _check(dev, [0, 1, 63, 64, 65, 200, 7], 3, V, torch.bfloat16, seed=V, gate=gate, tag=f"{gate} V={V}")


def test_chunk_bwd_no_state_and_fp16(dev):
    _check(dev, [150, 90], 2, 64, torch.bfloat16, seed=3, h0=False, tag="no h0", case="no h0")
    _check(dev, [150, 90], 2, 64, torch.float16, seed=4, tag="fp16", case="fp16")


def test_chunk_bwd_long_sequences(dev):
    """Two 4096-token sequences (64 chunks each), H = 4: the state passes
    carry 64 chunks."""
    _check(dev, [4096, 4096], 4, 64, torch.bfloat16, seed=5, tag="long", case="long")


@pytest.mark.parametrize("K", [32, 128])
def test_chunk_bwd_key_widths(dev, K):
    """K other than 64: the backward runs per group of 64 keys (the last one
    zero-padded) and dv adds up over the groups."""
    _check(dev, [0, 1, 63, 64, 65, 200, 7], 3, 32, torch.bfloat16, seed=K, tag=f"K={K}", case=f"K={K}", K=K,
           scale=K ** -0.5)


@pytest.mark.parametrize("K,V", [(64, 128), (64, 80), (32, 256), (128, 128)])
def test_chunk_bwd_value_widths(dev, K, V):
    """V above 64: the backward runs per group of 64 value columns (each
    state column evolves on its own), dq, dk, dg add up over the groups and
    dv, dh0 are their columns; K above 64 adds the key groups inside."""
    _check(dev, [0, 1, 63, 64, 65, 200, 7], 2, V, torch.bfloat16, seed=K + V, tag=f"K={K} V={V}", case="value groups",
           K=K, scale=K ** -0.5)


def test_chunk_bwd_unsupported_raises(dev):
    from ssla_amd.gla import chunk_gla
    q = torch.randn(10, 1, 64, device=dev, dtype=torch.bfloat16, requires_grad=True)
    v = torch.randn(10, 1, 272, device=dev, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        chunk_gla(q, q.detach(), v, torch.zeros(10, 1, 64, device=dev), torch.tensor([0, 10], device=dev))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_chunk_bwd_16bit_gates(dev, dtype):
    """g in the input dtype (the kernels' 16-bit gate path; dg comes back in
    that dtype): the oracle sees the same rounded gates."""
    q, k, v, g, cu, s0, do, dht = _inputs([150, 64, 37, 1], 2, 64, dtype, seed=11, gate="randn-1")
    g16 = g.to(dtype)
    print(f"gla bwd 16-bit gates: {dtype}", flush=True)
    got = _gpu_grads(dev, q, k, v, g16, cu, s0, do, dht, 64 ** -0.5)
    ref = oracle.gla_recurrent_bwd(q.float().numpy(), k.float().numpy(), v.float().numpy(), g16.float().numpy(),
                                   cu.numpy(), do.float().numpy(), 64 ** -0.5, s0.numpy(), dht.numpy())
    bands = BANDS["16-bit g bf16" if dtype == torch.bfloat16 else "16-bit g fp16"]
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dh0"), got, ref):
        band, ratio_max = bands[name]
        assert_close(a, b, 0.0, f"{name}[16-bit g {dtype}]", band=band, ratio_max=ratio_max)


def test_chunk_bwd_all_sequences_empty(dev):
    """T == 0 with sequences present: ht equals h0, so the initial-state
    gradient is exactly the final-state gradient (zero without one)."""
    from ssla_amd.gla import chunk_gla
    H, N = 2, 3
    gen = torch.Generator().manual_seed(21)
    z = [torch.zeros(0, H, 64, device=dev, dtype=torch.bfloat16).requires_grad_() for _ in range(3)]
    g = torch.zeros(0, H, 64, device=dev).requires_grad_()
    cu = torch.zeros(N + 1, dtype=torch.int64, device=dev)
    dht = (torch.randn(N, H, 64, 64, generator=gen) * 0.1).to(dev)
    print("gla bwd: every sequence empty", flush=True)
    h0 = (torch.randn(N, H, 64, 64, generator=gen) * 0.1).to(dev).requires_grad_()
    o, ht = chunk_gla(z[0], z[1], z[2], g, cu, initial_state=h0, output_final_state=True)
    assert o.shape == (0, H, 64) and torch.equal(ht, h0.detach())
    (ht * dht).sum().backward()
    assert torch.equal(h0.grad, dht)
    h0b = h0.detach().clone().requires_grad_()
    o, _ = chunk_gla(z[0], z[1], z[2], g, cu, initial_state=h0b, output_final_state=False)
    torch.autograd.backward([o], [torch.zeros_like(o)])
    assert h0b.grad is not None and not h0b.grad.any()


@pytest.mark.parametrize("K,V", [(64, 64), (32, 48), (128, 128)])
@pytest.mark.parametrize("gate", ["logsig", "randn-1", "strong", "zero"])
def test_chunk_bwd_fp32(dev, K, V, gate):
    """fp32 backward (ssla_gla_chunk_f32_bwd, in groups of 64 keys by 64
    value columns): dq, dk, dv, dg, dh0 of o and the final state against the
    fp64 recurrent backward at the fp32 bar (rtol 1e-4, atol 1e-4 of each
    gradient's RMS)."""
    q, k, v, g, cu, s0, do, dht = _inputs([0, 1, 63, 64, 65, 200, 7], 2, V, torch.float32, seed=K + V, gate=gate, K=K)
    scale = K ** -0.5
    print(f"gla bwd fp32 K={K} V={V} gate={gate}", flush=True)
    got = _gpu_grads(dev, q, k, v, g, cu, s0, do, dht, scale)
    ref = oracle.gla_recurrent_bwd(q.numpy(), k.numpy(), v.numpy(), g.numpy(), cu.numpy(), do.numpy(), scale,
                                   s0.numpy(), dht.numpy())
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dh0"), got, ref):
        assert_close(a, b, 1e-4, f"fp32 {name} K={K} V={V} {gate}")


def test_chunk_bwd_fp32_long(dev):
    """Two 4096-token fp32 sequences (64 chunks each), H = 4, without an
    initial state: the backward's forward pass and reverse walk carry 64
    chunks."""
    q, k, v, g, cu, s0, do, dht = _inputs([4096, 4096], 4, 64, torch.float32, seed=6, h0=False)
    print("gla bwd fp32 long", flush=True)
    got = _gpu_grads(dev, q, k, v, g, cu, s0, do, dht, 64 ** -0.5)
    ref = oracle.gla_recurrent_bwd(q.numpy(), k.numpy(), v.numpy(), g.numpy(), cu.numpy(), do.numpy(), 64 ** -0.5)
    for name, a, b in zip(("dq", "dk", "dv", "dg"), got, ref):
        assert_close(a, b, 1e-4, f"fp32 long {name}")
    assert got[4] is None and ref[4] is None
