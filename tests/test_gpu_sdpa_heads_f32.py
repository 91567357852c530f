"""GPU parity of lux3d_sdpa_heads_f32, the reference's exact_sdpa_heads
(attention_math.rs:244-259): q, k, v widened to f32, scores, softmax and P v
in f32, the result narrowed to the input dtype. Checked against the oracle's
double-precision attention (or_sdpa, pinned in tests/test_oracle_pins.py):

- with an f32 `out`, every element to the f32 bar of the generic kernel,
  |err| <= 1e-5 * wabs + 2^-23 |want| (wabs = sum_j p_j |v_j| / sum_j p_j);
  probabilities rounded to bf16 carry up to 2^-9 relative error each, far
  above this bar;
- with a bf16 / f16 `out`, bit for bit the f32 result of the same call
  rounded once to nearest-even: the only rounding after the f32 arithmetic.
Shapes: the DINOv3 attention (1029 tokens, 16 heads, D 64; trellis2_dino.rs:
392), D 128 with moving maxima (TripoSG cross-attention, triposg_dit.rs:499),
a query count above 4096 (two query tiles per wavefront), partial key
blocks, and the generic-kernel cases (f16, D 80, unaligned rows)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

TDT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


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


def host(t, dt):
    t = t.detach().contiguous().cpu()
    if dt == "bf16":
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def oracle(orc, q, k, v, scale, dt):
    code = {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}[dt]
    # the exact result rounded once to f32
    return orc.sdpa(host(q, dt), host(k, dt), host(v, dt), scale, dt=code, out_dt=orc.F32, with_abs=True)


def f32_bar_violations(got, want, wabs):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bound = 1e-5 * wabs.astype(np.float64) + 2.0 ** -23 * np.abs(want.astype(np.float64))
    return err > bound + 1e-30, err, bound


def qkv_views(dev, b, n, h, d, dt, seed, kscale=1.0, rising=False):
    """q, k, v as the permuted views of a fused [B, N, 3, H, D] buffer."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn((b, n, 3, h, d), generator=g, dtype=torch.float32)
    x[:, :, 1] *= kscale
    if rising:
        x[:, :, 1] *= torch.linspace(0.5, 3.0, n).view(1, n, 1, 1)
    qkv = x.to(dev).to(TDT[dt]).permute(2, 0, 3, 1, 4)
    return qkv[0], qkv[1], qkv[2]


def _case(**kw):
    print("\n[case] sdpa_heads_f32 " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _check(ops, orc, q, k, v, scale, dt, what):
    out32 = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    ops.exact_sdpa_heads(q, k, v, scale, out=out32)
    out = ops.exact_sdpa_heads(q, k, v, scale)
    torch.cuda.synchronize()
    assert out.dtype == q.dtype
    want, wabs = oracle(orc, q, k, v, scale, dt)
    bad, err, bound = f32_bar_violations(out32.cpu().numpy(), want, wabs)
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} f32 outputs out of tolerance; worst err "
                           f"{err.max():.3e} (bound there {bound.reshape(-1)[np.argmax(err)]:.3e})")
    rounded = out32.to(q.dtype)
    diff = int((rounded.view(torch.int16) != out.view(torch.int16)).sum()) if dt != "f32" else \
        int((rounded != out).sum())
    assert diff == 0, f"{what}: {diff} narrowed outputs differ from the f32 result rounded once"


@pytest.mark.parametrize("b,n,h,d,kscale,rising,seed", [
    (1, 1029, 16, 64, 1.0, False, 1),     # DINOv3: 1024 patches + 5 prefix tokens
    (1, 517, 3, 128, 2.0, True, 2),       # D 128, peaky and moving maxima
    (2, 129, 2, 128, 1.0, False, 3),      # one full block + one key
    (1, 65, 1, 64, 4.0, False, 4),
    (1, 4200, 2, 64, 1.0, True, 5),       # > 4096 queries: two query tiles per wavefront
    (1, 2100, 16, 64, 1.0, False, 6),
])
def test_sdpa_heads_f32_bf16_matrix_cores(dev, ops, orc, b, n, h, d, kscale, rising, seed):
    _case(b=b, n=n, h=h, d=d, seed=seed)
    q, k, v = qkv_views(dev, b, n, h, d, "bf16", 100 + seed, kscale, rising)
    _check(ops, orc, q, k, v, 1.0 / np.sqrt(d), "bf16", f"bf16 {b}x{h}x{n}x{d}")


@pytest.mark.parametrize("lq,lk,d", [(300, 517, 128), (1, 1, 64), (5, 1, 64), (257, 64, 64), (77, 200, 128),
                                     (40, 129, 64), (100, 200, 64)])
def test_sdpa_heads_f32_cross_attention(dev, ops, orc, lq, lk, d):
    """Cross-attention shapes (TripoSG's exact_sdpa_heads call sits on the
    encoder's keys), including single keys and partial key blocks."""
    _case(lq=lq, lk=lk, d=d)
    g = torch.Generator(device="cpu").manual_seed(lq * 5 + lk)
    q = torch.randn((2, 3, lq, d), generator=g).to(dev).to(torch.bfloat16)
    k = (2 * torch.randn((2, 3, lk, d), generator=g)).to(dev).to(torch.bfloat16)
    v = torch.randn((2, 3, lk, d), generator=g).to(dev).to(torch.bfloat16)
    _check(ops, orc, q, k, v, 1.0 / np.sqrt(d), "bf16", f"cross {lq}x{lk}x{d}")


@pytest.mark.parametrize("case", ["f16_d64", "bf16_d80", "bf16_unaligned", "f32_d64"])
def test_sdpa_heads_f32_other_paths(dev, ops, orc, case):
    """f16 (generic kernel), bf16 with D 80 or unaligned rows (generic
    kernel), f32 (the three-term split kernel for f32 inputs)."""
    _case(case=case)
    dt = case.split("_")[0]
    d = 80 if case.endswith("d80") else 64
    g = torch.Generator(device="cpu").manual_seed(len(case) + d)
    lq, lk = 77, 130
    if case.endswith("unaligned"):
        q = torch.randn((1, 2, lq, d + 1), generator=g).to(dev).to(TDT[dt])[..., 1:]
    else:
        q = torch.randn((1, 2, lq, d), generator=g).to(dev).to(TDT[dt])
    k = torch.randn((1, 2, lk, d), generator=g).to(dev).to(TDT[dt])
    v = torch.randn((1, 2, lk, d), generator=g).to(dev).to(TDT[dt])
    _check(ops, orc, q, k, v, 1.0 / np.sqrt(d), dt, case)


@pytest.mark.parametrize("d,lk", [(128, 200), (64, 130)])
def test_sdpa_heads_f32_keys_past_lk_are_not_read(dev, ops, orc, d, lk):
    """K and V rows Lk .. Lk + 63 of every head hold NaN: a kernel that read
    a key past Lk would give NaN outputs (the D 128 case runs the direct
    global -> LDS loads)."""
    _case(op="nan tail", d=d, lk=lk)
    b, h, lq = 2, 3, 96
    g = torch.Generator(device="cpu").manual_seed(lk * 7 + d)
    buf = torch.full((2, b, h, lk + 64, d), float("nan"))
    buf[:, :, :, :lk] = torch.randn((2, b, h, lk, d), generator=g)
    buf = buf.to(dev).to(torch.bfloat16)
    k, v = buf[0, :, :, :lk], buf[1, :, :, :lk]
    q = torch.randn((b, h, lq, d), generator=g).to(dev).to(torch.bfloat16)
    out = ops.exact_sdpa_heads(q, k, v, 1.0 / np.sqrt(d))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all(), "a key past Lk reached the output"
    _check(ops, orc, q, k, v, 1.0 / np.sqrt(d), "bf16", f"nan tail d={d}")

