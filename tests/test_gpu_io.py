"""GPU parity: .dat records -> padded batch tensor (ssla_dat_decode_batch via
ssla_amd.io.pad_batches) vs the oracle of the reference's pad_batches
(model_base.py:82-117).  Bit-exact (integer fields and float32 rounding of
t)."""
import numpy as np
import pytest
import torch

import oracle.events as OE
from ssla_amd import io
from tests.dat_files import encode, random_stream, write_dat

pytestmark = pytest.mark.gpu


def _check(dev, recs, dataset="Gen1"):
    batch = io.pad_batches([(r, np.zeros((len(r) % 3, 5), np.float32)) for r in recs], dataset, dev)
    want, lens = OE.pad_batches([OE.dat_decode(r) for r in recs], dataset)
    got = batch["events"].cpu().numpy()
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), dataset
    assert np.array_equal(batch["lengths"].numpy(), lens)
    assert list(batch["labels_lengths"].numpy()) == [len(r) % 3 for r in recs]


@pytest.mark.parametrize("dataset", ["Gen1", "NCaltech101", "other"])
def test_random_batches(dev, dataset):
    rng = np.random.default_rng(0)
    recs = []
    for b, n in enumerate([1000, 0, 1, 4093, 250]):
        t = np.sort(rng.integers(0, 2 ** 32, n, dtype=np.uint64))   # large t: float32 rounding
        recs.append(encode(t, rng.integers(0, 16384, n), rng.integers(0, 16384, n), rng.integers(0, 2, n)))
    _check(dev, recs, dataset)


def test_edge_batches(dev):
    _check(dev, [encode([], [], [], [])] * 3)   # every sample empty: [3, 0, 4]
    _check(dev, [encode([2 ** 24 + 1, 2 ** 32 - 1], [16383, 0], [0, 16383], [1, 1])])


def test_from_files_through_the_loader(dev, tmp_path):
    """Gen1.__getitem__'s window (seek_time(ts - window), load_delta_t(window
    + 1)) from .dat files, batched on the device."""
    recs = []
    for s in range(4):
        f = tmp_path / f"s{s}.dat"
        t, x, y, p = random_stream(20000 + 1000 * s, seed=10 + s, t_max=2_000_000)
        write_dat(f, t, x, y, p)
        ld = io.PSEELoader(str(f))
        ts = int(t[len(t) // 2])
        ld.seek_time(ts - 50_000)
        recs.append(ld.load_delta_t_raw(50_000 + 1))
    _check(dev, recs)


def test_full_size_batch(dev):
    """Eight 300k-event windows (a large Gen1 batch)."""
    rng = np.random.default_rng(5)
    recs = []
    for n in rng.integers(100_000, 300_000, 8):
        t, x, y, p = random_stream(int(n), seed=int(n), t_max=50_000_000)
        recs.append(encode(t, x, y, p))
    _check(dev, recs)


def test_bad_layout_and_sizes(dev):
    lib = __import__("ssla_amd._lib", fromlist=["load"]).load()
    out = torch.empty(4, device=dev)
    assert lib.ssla_dat_decode_batch(None, 0, None, 1, 1, 7, out.data_ptr(), None) != 0
    assert lib.ssla_dat_decode_batch(None, -1, None, 1, 1, 0, out.data_ptr(), None) != 0
