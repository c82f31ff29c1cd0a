"""GPU parity: scatter_max / scatter_mean (torch_scatter semantics as called
at reference layers/sparse_pooling.py:33) vs the CPU oracle.
scatter_max values and argmax bit-exact; scatter_mean rtol 1e-5."""
import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_close

pytestmark = pytest.mark.gpu


def _check(dev, src, index, n_out, sorted_index=False):
    from ssla_amd.scatter import scatter_max, scatter_mean
    s, i = src.to(dev), index.to(dev)
    with torch.no_grad():
        out, arg = scatter_max(s, i.unsqueeze(1).expand(-1, src.shape[1]), dim=0, dim_size=n_out,
                               sorted_index=sorted_index)
        mean = scatter_mean(s, i, dim=0, dim_size=n_out, sorted_index=sorted_index)
    ro, ra = oracle.scatter_max(src.numpy(), index.numpy(), n_out)
    out_np = out.cpu().numpy()
    assert np.array_equal(out_np.view(np.uint32), ro.view(np.uint32)), "scatter_max values differ"
    assert np.array_equal(arg.cpu().numpy(), ra), "scatter_max argmax differs"
    assert_close(mean.cpu().numpy(), oracle.scatter_mean(src.numpy(), index.numpy(), n_out), 1e-5,
                 "scatter_mean", atol_scale=1e-6)


@pytest.mark.parametrize("C", [1, 3, 4, 12, 64, 65, 100, 256, 300])
def test_random_unsorted(dev, C):
    gen = torch.Generator().manual_seed(C)
    E, n_out = 5000, 300
    src = torch.randn(E, C, generator=gen)
    index = torch.randint(0, n_out - 20, (E,), generator=gen)   # last rows stay empty
    _check(dev, src, index, n_out)


def test_ties_and_heavy_rows(dev):
    """Integer-valued features force ties (smallest index must win); one row
    holds 40% of the events (multi-piece rows); signed zeros tie."""
    gen = torch.Generator().manual_seed(1)
    E, C, n_out = 20000, 16, 64
    src = torch.randint(-3, 4, (E, C), generator=gen).float()
    src[::7, 0] = -0.0
    index = torch.randint(0, n_out, (E,), generator=gen)
    index[torch.rand(E, generator=gen) < 0.4] = 5
    _check(dev, src, index, n_out)


def test_sorted_segments(dev):
    """The reference's call: index is a unique_consecutive inverse (sorted)."""
    gen = torch.Generator().manual_seed(2)
    E, C = 30000, 24
    index = torch.sort(torch.randint(0, 900, (E,), generator=gen)).values
    src = torch.randn(E, C, generator=gen)
    _check(dev, src, index, 1000, sorted_index=True)
    _check(dev, src, index, 1000, sorted_index=False)


@pytest.mark.parametrize("C", [1, 3, 64, 65, 100, 300])
def test_random_sorted(dev, C):
    """Sorted (segment) path across channel blocks, with empty leading,
    inner and trailing rows."""
    gen = torch.Generator().manual_seed(100 + C)
    E, n_out = 5000, 400
    index = torch.sort(torch.randint(3, n_out - 20, (E,), generator=gen)).values
    index = index[(index % 7) != 0]          # inner empty rows
    src = torch.randn(index.numel(), C, generator=gen)
    _check(dev, src, index, n_out, sorted_index=True)


def test_sorted_rows_spanning_many_tiles(dev):
    """Rows longer than 64 tiles (the fix-up reads 64 tile flags at a time),
    rows ending exactly on tile boundaries, ties."""
    gen = torch.Generator().manual_seed(7)
    lens = [1, 63, 64, 128, 5000, 1, 64 * 70 + 3, 2, 129]
    index = torch.cat([torch.full((n,), r * 3, dtype=torch.int64) for r, n in enumerate(lens)])
    src = torch.randint(-2, 3, (index.numel(), 8), generator=gen).float()
    _check(dev, src, index, 3 * len(lens) + 5, sorted_index=True)


def test_sorted_special_values(dev):
    """-inf ties (first index wins), NaN never wins (a row of only NaN is
    treated as having no winner), signed zeros."""
    index = torch.tensor([0, 0, 0, 1, 1, 2, 2, 2, 4])
    src = torch.tensor([[-np.inf, 1.0], [-np.inf, 1.0], [-5.0, np.nan],
                        [np.nan, -0.0], [np.nan, 0.0],
                        [2.0, -np.inf], [np.nan, -np.inf], [2.0, 3.0],
                        [0.0, -0.0]], dtype=torch.float32)
    from ssla_amd.scatter import scatter_max
    o_s, a_s = scatter_max(src.to(dev), index.to(dev), dim=0, dim_size=6, sorted_index=True)
    o_u, a_u = scatter_max(src.to(dev), index.to(dev), dim=0, dim_size=6, sorted_index=False)
    assert np.array_equal(o_s.cpu().numpy().view(np.uint32), o_u.cpu().numpy().view(np.uint32))
    assert np.array_equal(a_s.cpu().numpy(), a_u.cpu().numpy())
    ro, ra = oracle.scatter_max(src.numpy(), index.numpy(), 6)
    assert np.array_equal(a_s.cpu().numpy(), ra)


@pytest.mark.parametrize("n_out", [40000, 300000])
def test_many_rows_global_counting(dev, n_out):
    """Many output rows: 625 buckets (LDS histogram) and 4688 buckets, more
    than the LDS histogram holds (global-counter path, whose histogram kernel
    also clears the chunk arrival counters), plus a row of 5000 events whose
    bucket spans several reduce chunks (the last one to arrive folds)."""
    gen = torch.Generator().manual_seed(3)
    E, C = 60000, 8
    src = torch.randn(E, C, generator=gen)
    index = torch.randint(0, n_out, (E,), generator=gen)
    index[:5000] = 7
    _check(dev, src, index, n_out)
    # the same workspace shape again: counters left by the first call are cleared
    _check(dev, src.flip(0).contiguous(), index.flip(0).contiguous(), n_out)


def test_repeated_calls_reuse_workspace(dev):
    """Calls of different shapes back to back (stale workspace contents from
    the previous call must not leak into the next)."""
    gen = torch.Generator().manual_seed(4)
    for E, C, n_out in [(20000, 16, 50), (3000, 16, 2000), (20000, 16, 50), (0, 16, 10)]:
        src = torch.randn(E, C, generator=gen)
        index = torch.randint(0, n_out, (E,), generator=gen)
        _check(dev, src, index, n_out)


def test_empty_and_single(dev):
    src = torch.randn(1, 8)
    _check(dev, src, torch.tensor([3]), 5)
    from ssla_amd.scatter import scatter_max
    with torch.no_grad():
        out, arg = scatter_max(torch.zeros(0, 8, device=dev), torch.zeros(0, dtype=torch.int64, device=dev),
                               dim=0, dim_size=4)
    assert (out == 0).all() and (arg == 0).all()


def test_out_of_range_index_raises(dev):
    from ssla_amd.scatter import scatter_max
    src = torch.randn(10, 8, device=dev)
    idx = torch.arange(10, device=dev)
    with pytest.raises(NotImplementedError):
        scatter_max(src, idx, dim_size=10)          # torch_scatter's default dim=-1
    with pytest.raises(ValueError):
        scatter_max(src, idx, dim=0, dim_size=5)
    with pytest.raises(ValueError):
        scatter_max(src, idx.flip(0), dim=0, dim_size=10, sorted_index=True)


def test_c4_full(dev):
    """Config 4 (C4) at full size: 1e6 clustered events, C=64, 152x120
    cells; shuffled (bucketing path) and sorted (segment path)."""
    from ssla_amd import synthetic
    src, index, n_out = synthetic.pooling_events()
    _check(dev, src, index, n_out)
    order = torch.argsort(index, stable=True)
    _check(dev, src[order].contiguous(), index[order].contiguous(), n_out, sorted_index=True)
