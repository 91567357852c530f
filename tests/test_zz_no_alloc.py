"""lux3d_sparse_neighbors_noalloc (hash table in the library's per-device
static array, no allocation) against lux3d_sparse_neighbors (caller-provided
table) through the C ABI: identical neighbour tables and bad-coordinate
counts on two calls in a row, the second smaller than the first, so a table
left over from the first call must not leak into the second."""
import numpy as np
import pytest
import torch

from lux3d_fused import _lib
from lux3d_fused.ops import desc

pytestmark = pytest.mark.gpu


def _coords(n, seed, extent=64, bad=0):
    rng = np.random.default_rng(seed)
    flat = rng.choice(extent ** 3, size=n, replace=False)
    c = np.stack([flat // (extent * extent), (flat // extent) % extent, flat % extent], axis=1).astype(np.int32)
    c -= extent // 2                           # negative coordinates too
    if bad:
        c[rng.choice(n, size=bad, replace=False), 1] = (1 << 20) + 5   # outside the packable range
    return c


def _both(dev, c):
    co = torch.from_numpy(c).to(dev)
    n = c.shape[0]
    cap = 16
    while cap < 2 * n:
        cap *= 2
    keys = torch.empty(cap, dtype=torch.int64, device=dev)
    vals = torch.empty(cap, dtype=torch.int32, device=dev)
    want = torch.full((n, 27), -7, dtype=torch.int32, device=dev)
    got = torch.full((n, 27), -7, dtype=torch.int32, device=dev)
    bad_w = torch.full((1,), 99, dtype=torch.int32, device=dev)
    bad_g = torch.full((1,), 99, dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    d = desc
    torch.cuda.synchronize(dev)
    print(f"noalloc: N={n}", flush=True)
    _lib.call("lux3d_sparse_neighbors", d(co), d(keys), d(vals), d(want), d(bad_w), s)
    _lib.call("lux3d_sparse_neighbors_noalloc", d(co), d(got), d(bad_g), s)
    torch.cuda.synchronize(dev)
    return want.cpu().numpy(), got.cpu().numpy(), int(bad_w.item()), int(bad_g.item())


def test_noalloc_neighbors_match_the_workspace_entry_on_two_calls():
    dev = torch.device("cuda:0")
    for n, seed, bad in ((40000, 11, 7), (5000, 12, 0)):
        want, got, bw, bg = _both(dev, _coords(n, seed, bad=bad))
        assert np.array_equal(got, want), f"N={n}: {np.count_nonzero(got != want)} entries differ"
        assert bg == bw == bad
        assert (want >= 0).sum() > n                  # self + at least some neighbours found


def test_noalloc_rejects_more_voxels_than_its_table():
    dev = torch.device("cuda:0")
    n = (1 << 20) + 1
    co = torch.zeros((n, 3), dtype=torch.int32, device=dev)
    nbr = torch.empty((n, 27), dtype=torch.int32, device=dev)
    d = desc
    rc, msg = _lib.call_status("lux3d_sparse_neighbors_noalloc", d(co), d(nbr), None,
                               torch.cuda.current_stream(dev).cuda_stream)
    assert rc == _lib.ERR_SHAPE and "limit" in msg
