"""Per-op bandwidth ceilings for bench.py: copy kernels that move exactly an
op's activation bytes with no arithmetic (liblux3d_ceiling.so, built from
csrc/ceiling.hip), timed like the op itself (graph replay, rotation sets
larger than the 256 MB Infinity Cache).

Two ceilings per op:
- `copy`: the same bytes as plain contiguous streams (as many input and
  output streams as the op has), one 16-byte chunk per thread per stream;
- `pattern`: the op's own access pattern (the row kernels' rows / threads
  per row / chunks per thread, or the head kernels' strided [B, H, N, D]
  views and workgroup shape), also without arithmetic.
The op's pattern is a dict on its Workload (`Workload.pattern`).

And a third, `best`: the fastest of a family of plain copies of the same
streams (`BEST_VARIANTS`: one-shot grids with 1-8 chunks per thread,
persistent grids striding over tiles, persistent grids that load the next
tile before storing the current one; 256-1024 threads per workgroup), the
bound "no kernel on this chip moves these bytes faster than this" that the
op's fraction of peak is read against. `sweep_variants()` is the wider
family `bench.py --ceiling-sweep` runs over copy sizes.
"""
from __future__ import annotations

import ctypes
import math
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "liblux3d_ceiling.so")
MALL_BYTES = 256 << 20


def _load():
    import torch  # noqa: F401  (bind to the HIP runtime torch loaded)
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run `make -C candle-3d_amd`")
    lib = ctypes.CDLL(LIB_PATH)
    P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    PP = ctypes.POINTER(ctypes.c_void_p)
    lib.lux3d_ceiling_streams.argtypes = [PP, I, PP, I, I64, I64, P]
    lib.lux3d_ceiling_rows.argtypes = [PP, I, PP, I, I64, I64, I, I, P]
    lib.lux3d_ceiling_best.argtypes = [PP, I, PP, I, I64, I64, I, I, I, I, P]
    lib.lux3d_ceiling_heads.argtypes = [P, P, P, P, I64, I64, I64, I64, I, ctypes.POINTER(I64),
                                        ctypes.POINTER(I64), I, I, P]
    for f in (lib.lux3d_ceiling_streams, lib.lux3d_ceiling_rows, lib.lux3d_ceiling_heads, lib.lux3d_ceiling_best):
        f.restype = ctypes.c_int
    return lib


LIB = _load()


def _ptrs(ts):
    arr = (ctypes.c_void_p * len(ts))()
    for i, t in enumerate(ts):
        arr[i] = t.data_ptr()
    return arr


def _sets(bytes_per_set: int) -> int:
    return int(min(64, max(2, math.ceil(3 * MALL_BYTES / max(bytes_per_set, 1)))))


def _check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what}: ceiling kernel rejected its arguments (status {rc})")


class Copy:
    """A copy workload: `launch(i)` enqueues one copy on rotation set i % sets
    on the current stream; `bytes` is what it moves (read + written)."""

    def __init__(self, dev, pattern: dict, same_size: bool):
        self.dev = dev
        kind = pattern["kind"]
        stream = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
        if kind == "rows" and not same_size:
            nin, nout, rows, rb = pattern["nin"], pattern["nout"], pattern["rows"], pattern["row_bytes"]
            per_set = (nin + nout) * rows * rb
            n = _sets(per_set)
            bufs = [([torch.empty(rows * rb, dtype=torch.uint8, device=dev).fill_(k + 1) for _ in range(nin)],
                     [torch.empty(rows * rb, dtype=torch.uint8, device=dev) for _ in range(nout)]) for k in range(n)]
            args = [(_ptrs(i), _ptrs(o)) for i, o in bufs]

            def launch(i):
                a = args[i % n]
                # the row kernels move 16-byte units for every dtype (8 bf16 /
                # f16 elements, or half of an f32 chunk)
                _check(LIB.lux3d_ceiling_rows(a[0], nin, a[1], nout, rows, rb, pattern["tpr"],
                                              int(pattern.get("row_per_block", False)), stream()), "rows")
            self.bytes = per_set
        elif kind == "heads" and not same_size:
            B, H, N, D, eb = pattern["B"], pattern["H"], pattern["N"], pattern["D"], pattern["eb"]
            ntens = pattern["ntens"]
            # the input views live in a buffer of `in_numel` elements (e.g. the packed qkv)
            in_numel, ins, outs = pattern["in_numel"], pattern["in_strides"], pattern["out_strides"]
            in_off = pattern["in_offsets"]          # element offset of each tensor's view in the buffer
            per_set = in_numel * eb + ntens * B * H * N * D * eb
            n = _sets(per_set)
            bufs = [(torch.empty(in_numel * eb, dtype=torch.uint8, device=dev).fill_(k + 1),
                     [torch.empty(B * H * N * D * eb, dtype=torch.uint8, device=dev) for _ in range(ntens)])
                    for k in range(n)]
            si = (ctypes.c_int64 * 3)(*ins)
            so = (ctypes.c_int64 * 3)(*outs)

            def launch(i):
                src, dst = bufs[i % n]
                q = src.data_ptr() + in_off[0] * eb
                k = src.data_ptr() + in_off[1] * eb if ntens == 2 else None
                _check(LIB.lux3d_ceiling_heads(q, k, dst[0].data_ptr(), dst[1].data_ptr() if ntens == 2 else None,
                                               B, H, N, D, eb, si, so, int(pattern.get("both_in_one", False)),
                                               int(pattern.get("rows_per_thread", 0)), stream()), "heads")
            self.bytes = 2 * ntens * B * H * N * D * eb
        else:
            nin, nout = pattern["nin"], pattern["nout"]
            ib, ob = pattern["in_bytes"], pattern["out_bytes"]
            per_set = nin * ib + nout * ob
            n = _sets(per_set)
            bufs = [([torch.empty(ib, dtype=torch.uint8, device=dev).fill_(k + 1) for _ in range(nin)],
                     [torch.empty(ob, dtype=torch.uint8, device=dev) for _ in range(nout)]) for k in range(n)]
            args = [(_ptrs(i), _ptrs(o)) for i, o in bufs]

            def launch(i):
                a = args[i % n]
                _check(LIB.lux3d_ceiling_streams(a[0], nin, a[1], nout, ib, ob, stream()), "streams")
            self.bytes = per_set
        self.launch = launch
        self.sets = n
        self._keep = bufs


def same_size_streams(pattern: dict) -> dict:
    """The op's activation bytes as contiguous streams (same stream counts)."""
    kind = pattern["kind"]
    if kind == "rows":
        b = pattern["rows"] * pattern["row_bytes"]
        return {"kind": "streams", "nin": pattern["nin"], "nout": pattern["nout"], "in_bytes": b, "out_bytes": b}
    if kind == "heads":
        b = pattern["B"] * pattern["H"] * pattern["N"] * pattern["D"] * pattern["eb"]
        nt = pattern["ntens"]
        return {"kind": "streams", "nin": nt, "nout": nt, "in_bytes": b, "out_bytes": b}
    return dict(pattern)


# (form, chunks per thread, threads per workgroup, workgroups; 0 = one per tile)
# form 0: one-shot grid; 1: persistent, striding over tiles; 2: persistent,
# the next tile's loads issued before the current tile's stores; 3 / 4: forms
# 1 / 0 with one store in flight per wavefront; 5 / 6: with two.
def sweep_variants():
    out = [(0, c, b, 0) for b in (256, 512, 1024) for c in (1, 2, 4, 8)]
    for form in (1, 2):
        for b in (256, 512, 1024):
            for c in (1, 2, 4, 8):
                for wpc in (8, 16, 32):  # resident wavefronts per CU the grid asks for (256 CUs)
                    g = 256 * wpc * 64 // b
                    if g >= 256:
                        out.append((form, c, b, g))
    return out


# the subset bench.py times for every HBM op's `best_copy_us`: the winners of
# the size sweep (profiles/ceiling_sweep.md) -- persistent strided grids of
# one chunk per thread at 34-180 MB, one-shot grids of one chunk above,
# prefetching / two-chunk forms below -- and their neighbours
BEST_VARIANTS = [(0, 1, 256, 0), (0, 1, 512, 0), (0, 1, 1024, 0), (0, 2, 256, 0), (0, 2, 512, 0),
                 (1, 1, 256, 1024), (1, 1, 256, 2048), (1, 1, 512, 512), (1, 2, 256, 2048), (1, 2, 512, 1024),
                 (2, 1, 256, 2048), (2, 2, 256, 1024)]


FORM_NAMES = ["oneshot", "strided", "prefetch", "strided_st1", "oneshot_st1", "strided_st2", "oneshot_st2"]
ONESHOT_FORMS = (0, 4, 6)


def throttle_variants():
    """One-shot and persistent copies with the stores throttled to one or
    two in flight per wavefront, beside their unthrottled forms."""
    out = []
    for form in (0, 4, 6):
        for b in (256, 512, 1024):
            for c in (1, 2, 4, 8):
                out.append((form, c, b, 0))
    for form in (1, 3, 5):
        for b in (256, 512, 1024):
            for c in (1, 2, 4, 8):
                for wpc in (8, 16, 32):
                    g = 256 * wpc * 64 // b
                    if g >= 256:
                        out.append((form, c, b, g))
    return out


def variant_name(v) -> str:
    form, c, b, g = v
    return FORM_NAMES[form] + f"_c{c}_b{b}" + ("" if form in ONESHOT_FORMS else f"_g{g}")


class BestCopy:
    """A plain copy of `nin` input streams of `in_bytes` into `nout` output
    streams of `out_bytes` in launch variant `v`; `launch(i)` runs it on
    rotation set i % sets on the current stream."""

    def __init__(self, dev, nin, nout, in_bytes, out_bytes, v, bufs=None):
        self.v = v
        in_bytes = (in_bytes + 15) // 16 * 16
        out_bytes = (out_bytes + 15) // 16 * 16
        per_set = nin * in_bytes + nout * out_bytes
        if bufs is None:
            n = _sets(per_set)
            bufs = [([torch.empty(in_bytes, dtype=torch.uint8, device=dev).fill_(k + 1) for _ in range(nin)],
                     [torch.empty(out_bytes, dtype=torch.uint8, device=dev) for _ in range(nout)])
                    for k in range(n)]
        n = len(bufs)
        args = [(_ptrs(i), _ptrs(o)) for i, o in bufs]
        form, c, b, g = v
        stream = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731

        def launch(i):
            a = args[i % n]
            _check(LIB.lux3d_ceiling_best(a[0], nin, a[1], nout, in_bytes, out_bytes, form, c, b, g, stream()),
                   "best")
        self.launch = launch
        self.bytes = per_set
        self.sets = n
        self.bufs = bufs


def stream_shape(pattern: dict):
    """(nin, nout, in_bytes, out_bytes) of an op's activation streams."""
    s = same_size_streams(pattern)
    return s["nin"], s["nout"], s["in_bytes"], s["out_bytes"]
