"""GPU parity of the TRELLIS.2 sparse ops (runtime/trellis2_sparse.rs) against
the oracle (pinned in tests/test_oracle_pins.py against the reference's own
tests and torch conv3d): the neighbour table and C2S bit-exact, row gathers
bit-exact, the sparse convolution to f32 accumulation error
(|err| <= 2^-16 sum |W x| + 2^-23 |want|; the reference's own test allows
1e-4 absolute)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def ops(dev):
    from lux3d_fused import ops as _ops
    return _ops


@pytest.fixture(scope="module")
def orc():
    import lux3d_oracle as o
    o.set_threads(16)
    return o


def _case(**kw):
    print("\n[case] sparse " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def random_coords(n, res, seed, surface=False):
    rng = np.random.default_rng(seed)
    if surface:  # voxels near a sphere shell, the kind of set TRELLIS.2 decodes
        pts = rng.standard_normal((n * 3, 3))
        pts = pts / np.linalg.norm(pts, axis=1, keepdims=True) * (res * 0.4) + res / 2
        c = np.unique(np.floor(pts).astype(np.int32), axis=0)
        return c[rng.permutation(len(c))[:n]].astype(np.int32)
    cells = rng.choice(res ** 3, n, replace=False)
    return np.stack([cells // (res * res), (cells // res) % res, cells % res], axis=1).astype(np.int32)


def grid_with_holes(res=4):
    return np.array([[x, y, z] for x in range(res) for y in range(res) for z in range(res)
                     if (x * res * res + y * res + z) % 5 != 0], dtype=np.int32)


@pytest.mark.parametrize("case", ["holes", "random40k", "negative", "duplicates", "empty_neighbourhood"])
def test_sparse_neighbors(dev, ops, orc, case):
    _case(op="neighbors", case=case)
    if case == "holes":
        c = grid_with_holes()
    elif case == "random40k":
        c = random_coords(40000, 64, 1)
    elif case == "negative":
        c = random_coords(500, 16, 2) - 8
    elif case == "duplicates":
        c = np.concatenate([random_coords(300, 8, 3), random_coords(50, 8, 3)])
    else:
        c = np.array([[0, 0, 0], [10, 10, 10], [20, 0, 5]], dtype=np.int32)
    nbr = ops.sparse_neighbors(torch.from_numpy(c).to(dev))
    torch.cuda.synchronize()
    assert np.array_equal(nbr.cpu().numpy(), orc.sparse_neighbors(c))


def _conv_check(got, want, abs_sum):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bound = 2.0 ** -16 * abs_sum.astype(np.float64) + 2.0 ** -23 * np.abs(want) + 1e-30
    bad = err > bound
    assert not bad.any(), f"{int(bad.sum())} outputs off; worst {err.max():.3e}"


def test_sparse_conv3d_reference_cases(dev, ops, orc):
    """The reference's dense-parity case (3 -> 5 channels on the 4^3 grid with
    holes) and its identity / shift kernels, on the generic kernel."""
    _case(op="conv3d", case="reference")
    coords = grid_with_holes()
    pat = lambda i: ((np.asarray(i) % 23).astype(np.float32) - np.float32(11.0)) * np.float32(0.1)  # noqa: E731
    x = np.array([[pat(i * 13 + c * 7) for c in range(3)] for i in range(len(coords))], dtype=np.float32)
    w_ck = np.zeros((5, 3, 3, 3, 3), dtype=np.float32)  # the checkpoint's [Cout, kd, kh, kw, Cin]
    for o in range(5):
        for k in range(27):
            for c in range(3):
                w_ck[o, k // 9, (k % 9) // 3, k % 3, c] = pat(o * 31 + k * 5 + c * 3) * np.float32(0.5)
    bias = np.array([((o * 3) % 7) * 0.02 - 0.06 for o in range(5)], dtype=np.float32)
    conv = ops.SparseConv3d(torch.from_numpy(w_ck).to(dev), torch.from_numpy(bias).to(dev), 3, 5)
    out = conv.forward(torch.from_numpy(coords).to(dev), torch.from_numpy(x).to(dev))
    torch.cuda.synchronize()
    nbr = orc.sparse_neighbors(coords)
    want, a = orc.sparse_conv3d(x, nbr, conv.weight27.cpu().numpy(), bias, with_abs=True)
    _conv_check(out.cpu().numpy(), want, a)
    assert np.abs(out.cpu().numpy() - want).max() < 1e-4
    # identity (centre tap) and +x shift (k = 22) kernels
    hc = np.array([[0, 0, 0], [1, 0, 0], [1, 1, 0], [3, 0, 0]], dtype=np.int32)
    hx = pat(np.arange(8)).reshape(4, 2)
    for k, want in ((13, hx), (22, np.stack([hx[1], np.zeros(2), np.zeros(2), np.zeros(2)]).astype(np.float32))):
        w = np.zeros((2, 27, 2), dtype=np.float32)
        w[:, k, :] = np.eye(2)
        conv = ops.SparseConv3d(torch.from_numpy(w).to(dev), None, 2, 2)
        got = conv.forward(torch.from_numpy(hc).to(dev), torch.from_numpy(hx).to(dev)).cpu().numpy()
        assert np.array_equal(got, want), k


@pytest.mark.parametrize("n,cin,cout,res,surface", [
    (3000, 64, 96, 32, False),
    (5000, 128, 128, 64, True),
    (777, 32, 40, 16, False),
    (20000, 256, 256, 64, True),
    (1500, 48, 40, 16, False),
    (1500, 512, 600, 24, True),
    (700, 640, 512, 16, False),
])
@pytest.mark.parametrize("path", ["output_stationary", "rulebook"])
def test_sparse_conv3d_mfma(dev, ops, orc, n, cin, cout, res, surface, path):
    _case(op="conv3d", n=n, cin=cin, cout=cout, surface=surface, path=path)
    coords = random_coords(n, res, n + cin, surface)
    n = len(coords)
    rng = np.random.default_rng(cin)
    x = rng.standard_normal((n, cin)).astype(np.float32)
    w27 = (rng.standard_normal((27, cout, cin)) / np.sqrt(27 * cin)).astype(np.float32)
    bias = rng.standard_normal(cout).astype(np.float32)
    wt = torch.from_numpy(w27).permute(1, 0, 2).contiguous()  # back to [Cout, 27, Cin]
    conv = ops.SparseConv3d(wt.to(dev), torch.from_numpy(bias).to(dev), cin, cout)
    nbr_d = ops.sparse_neighbors(torch.from_numpy(coords).to(dev))
    arg = ops.SparseRulebook(nbr_d) if path == "rulebook" else nbr_d
    out = conv.forward(arg, torch.from_numpy(x).to(dev))
    torch.cuda.synchronize()
    nbr = orc.sparse_neighbors(coords)
    rows = np.arange(n) if n * cin * cout <= 5e8 else np.sort(np.random.default_rng(1).choice(n, 600, replace=False))
    want, a = orc.sparse_conv3d(x, nbr[rows], w27, bias, with_abs=True)
    _conv_check(out.cpu().numpy()[rows], want, a)


def test_sparse_conv3d_output_stationary_128_row_tiles(dev, ops, orc):
    """More than 65535 * 64 voxels: the output-stationary conv takes 128-row
    tiles (the 64-row grid would exceed the launch's y limit); 4.3M random
    voxels in 256^3, 16 -> 16 channels, checked on sampled rows."""
    n, cin, cout = 4_300_000, 16, 16
    _case(op="conv3d", n=n, cin=cin, cout=cout, path="output_stationary 128-row tiles")
    coords = random_coords(n, 256, 77)
    rng = np.random.default_rng(78)
    x = rng.standard_normal((n, cin)).astype(np.float32)
    w27 = (rng.standard_normal((27, cout, cin)) / np.sqrt(27 * cin)).astype(np.float32)
    bias = rng.standard_normal(cout).astype(np.float32)
    wt = torch.from_numpy(w27).permute(1, 0, 2).contiguous()
    conv = ops.SparseConv3d(wt.to(dev), torch.from_numpy(bias).to(dev), cin, cout)
    nbr_d = ops.sparse_neighbors(torch.from_numpy(coords).to(dev))
    out = conv.forward(nbr_d, torch.from_numpy(x).to(dev))
    torch.cuda.synchronize()
    rows = np.sort(np.concatenate([np.arange(64), np.arange(n - 200, n),
                                   np.random.default_rng(3).choice(n, 400, replace=False)]))
    nbr = orc.sparse_neighbors(coords)
    want, a = orc.sparse_conv3d(x, nbr[rows], w27, bias, with_abs=True)
    _conv_check(out[torch.from_numpy(rows).to(dev)].cpu().numpy(), want, a)


@pytest.mark.parametrize("dt,ids_dt,row", [("f32", "i64", (64,)), ("bf16", "i32", (6, 8)), ("f32", "i32", (3,)),
                                           ("bf16", "i64", (5,)), ("f32", "i64", (128,)), ("f32", "i32", (1028,)),
                                           ("bf16", "i32", (16, 64))])
def test_index_select_rows(dev, ops, dt, ids_dt, row):
    _case(op="index_select", dt=dt, ids=ids_dt, row=row)
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16}[dt]
    g = torch.Generator().manual_seed(5)
    src = torch.randn((1000,) + row, generator=g).to(tdt)
    ids = torch.randint(0, 1000, (4321,), generator=g)
    ids[::97] = 1000   # out of range: zero rows
    ids[1::89] = -1
    ids = ids.to(torch.int64 if ids_dt == "i64" else torch.int32)
    bad = torch.full((1,), 12345, dtype=torch.int32, device=dev)   # the entry sets it
    got = ops.index_select_rows(src.to(dev), ids.to(dev), bad_ids=bad).cpu()
    valid = (ids >= 0) & (ids < 1000)
    want = torch.zeros((4321,) + row, dtype=tdt)
    want[valid] = src[ids[valid].long()]
    assert torch.equal(got, want)
    assert int(bad.item()) == int((~valid).sum())
    # all ids valid: the count is zero
    ops.index_select_rows(src.to(dev), ids[valid].to(dev), bad_ids=bad)
    assert int(bad.item()) == 0


def test_sparse_neighbors_counts_unpackable_coords(dev, ops, orc):
    """Coordinates outside [-2^20, 2^20 - 1) are neither inserted nor found
    and are counted into bad_coords; the others keep their neighbours."""
    _case(op="neighbors", case="out of range")
    c = random_coords(400, 8, 7)
    far = np.array([[1 << 20, 0, 0], [0, -(1 << 20) - 1, 0], [3, 3, 2 ** 30]], dtype=np.int32)
    allc = np.concatenate([c, far])
    bad = torch.full((1,), -7, dtype=torch.int32, device=dev)
    nbr = ops.sparse_neighbors(torch.from_numpy(allc).to(dev), bad_coords=bad).cpu().numpy()
    torch.cuda.synchronize()
    assert int(bad.item()) == 3
    assert np.array_equal(nbr[:400], orc.sparse_neighbors(c))
    assert (nbr[400:] == -1).all()


@pytest.mark.parametrize("n,c,fdt,ldt", [(3, 16, "f32", "f32"), (5000, 64, "f32", "f32"), (3000, 128, "bf16", "bf16"),
                                         (1025, 8, "f32", "f16"), (0, 8, "f32", "f32"), (2000, 2048, "f32", "f32")])
def test_channel_to_spatial(dev, ops, orc, n, c, fdt, ldt):
    _case(op="c2s", n=n, c=c, feats=fdt, logits=ldt)
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
    if n == 3:  # the reference's hand case (tests/trellis2_sparse.rs:274-318)
        coords = np.array([[0, 0, 0], [1, 0, 0], [0, 1, 1]], dtype=np.int32)
        feats = (np.arange(48, dtype=np.float32) / 10.0).reshape(3, 16)
        logits = -np.ones((3, 8), dtype=np.float32)
        logits[0, [0, 3, 5]] = 1.0
        logits[1, 1] = 1.0
    else:
        coords = random_coords(n, 64, 7) if n else np.zeros((0, 3), dtype=np.int32)
        rng = np.random.default_rng(n)
        feats = rng.standard_normal((n, c)).astype(np.float32)
        logits = rng.standard_normal((n, 8)).astype(np.float32)
        logits[::13] = 0.0  # logits == 0 is not a leaf
    ft = torch.from_numpy(feats).to(tdt[fdt])
    lt = torch.from_numpy(logits).to(tdt[ldt])
    oc, of, sub = ops.channel_to_spatial(torch.from_numpy(coords).to(dev), ft.to(dev), lt.to(dev))
    torch.cuda.synchronize()
    woc, wof, _, wsub = orc.channel_to_spatial(coords, ft.float().numpy(), lt.float().numpy())
    assert np.array_equal(oc.cpu().numpy(), woc)
    assert torch.equal(of.cpu(), torch.from_numpy(wof).to(tdt[fdt]))
    assert np.array_equal(sub.cpu().numpy(), wsub)
    if n == 3:
        assert oc.cpu().tolist() == [[0, 0, 0], [1, 1, 0], [1, 0, 1], [3, 0, 0]]


@pytest.mark.parametrize("n", [1, 255, 256, 257, 4000])
def test_sparse_rulebook_pairs(dev, ops, orc, n):
    """Every present neighbour appears once in its tap's list, nothing else
    (one workgroup per 256 voxels: partial, exact and one-over sizes)."""
    coords = random_coords(n, 32 if n > 300 else 8, 21 + n, n > 300)[:n]
    nbr = orc.sparse_neighbors(coords)
    rb = ops.SparseRulebook(torch.from_numpy(nbr).to(dev))
    torch.cuda.synchronize()
    pairs, counts = rb.pairs.cpu().numpy(), rb.counts.cpu().numpy()
    for k in range(27):
        want = {(i, int(nbr[i, k])) for i in range(len(coords)) if nbr[i, k] >= 0}
        got = {(int(d), int(s_)) for d, s_ in pairs[k, :counts[k]]}
        assert counts[k] == len(want) and got == want, k


@pytest.mark.parametrize("cin,cout", [(32, 48), (512, 520)])
def test_sparse_conv3d_rulebook_matches_reference_order(dev, ops, orc, cin, cout):
    """The rulebook path adds the taps in the reference's order; on inputs
    whose products and partial sums are exact in f32 it equals the oracle
    bit for bit (64- and 128-wide tap tiles)."""
    _case(op="conv3d exact", cin=cin, cout=cout)
    coords = random_coords(2000, 24, 22, True)
    rng = np.random.default_rng(23)
    x = rng.integers(-4, 5, (len(coords), cin)).astype(np.float32)
    w27 = (rng.integers(-3, 4, (27, cout, cin)) * 0.25).astype(np.float32)
    bias = (rng.integers(-8, 9, cout) * 0.5).astype(np.float32)
    conv = ops.SparseConv3d(torch.from_numpy(w27).permute(1, 0, 2).contiguous().to(dev), torch.from_numpy(bias).to(dev),
                            cin, cout)
    nbr = ops.sparse_neighbors(torch.from_numpy(coords).to(dev))
    got = conv.forward(ops.SparseRulebook(nbr), torch.from_numpy(x).to(dev)).cpu().numpy()
    want = orc.sparse_conv3d(x, orc.sparse_neighbors(coords), w27, bias)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("ldt", ["f32", "bf16"])
def test_channel_to_spatial_unaligned_logits(dev, ops, orc, ldt):
    """Logits that start 1 element past a 16-byte boundary take the count
    kernel's per-element path; children, features and sub_binary equal the
    oracle's, as on the aligned path."""
    n, c = 2000, 64
    _case(op="c2s unaligned logits", n=n, c=c, logits=ldt)
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16}[ldt]
    coords = random_coords(n, 64, 17)
    rng = np.random.default_rng(17)
    feats = rng.standard_normal((n, c)).astype(np.float32)
    logits = rng.standard_normal((n, 8)).astype(np.float32)
    lt = torch.from_numpy(logits).to(tdt)
    buf = torch.empty(n * 8 + 1, dtype=tdt, device=dev)
    lv = buf[1:].view(n, 8)
    lv.copy_(lt.to(dev))
    assert lv.data_ptr() % 16 != 0
    oc, of, sub = ops.channel_to_spatial(torch.from_numpy(coords).to(dev), torch.from_numpy(feats).to(dev), lv)
    torch.cuda.synchronize()
    woc, wof, _, wsub = orc.channel_to_spatial(coords, feats, lt.float().numpy())
    assert np.array_equal(oc.cpu().numpy(), woc)
    assert torch.equal(of.cpu(), torch.from_numpy(wof))
    assert np.array_equal(sub.cpu().numpy(), wsub)
