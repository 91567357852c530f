"""bench.py's final stdout line (CPU only): the driver parses the last line
of bench.py's output, and a line carrying the whole per-op table (~28 KB)
once failed to parse. These tests build the line from a table of the bench's
size and shape and check that it stays one JSON line of a few KB that
carries every field of the measurement contract."""
import importlib.util
import json
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)  # module level imports only the standard library
    return mod


def _row(op, target, mfma):
    """One per-op table row with every field bench.py's loop writes."""
    r = {"op": op, "config": 1, "dtype": "bf16", "shape": "q,k [8,16,1374,64] in qkv", "bytes": 90135424,
         "us": 17.288, "gbs": 5213.7, "warm_us": 17.301, "warm_gbs": 5209.8, "frac_peak": 0.6517,
         "target_70pct": target, "meets_70pct": False if target else None, "rotation_sets": 8,
         "trace_us": 18.344, "trace_frac_peak": 0.6142, "trace_kernel": "void lux3d::(anonymous namespace)::"
         "head_kernel<lux3d::BF16, 64, 1, 2, 2, 1, true>(lux3d::HeadParams, int)", "traffic_bytes": 90861488,
         "cpu": {"sample": "1 of 8 frames", "sample_bytes": 11266816, "threads": 16, "us": 3170.2, "gbs": 3.554,
                 "us_1thread": 32911.0, "gbs_1thread": 0.342}, "gpu_over_cpu": 1466.9}
    if mfma:
        r.update({"bound": "mfma", "tflops": 431.9, "mfma_peak_tflops": 2500.0, "frac_mfma_peak": 0.1728})
    else:
        r.update({"runtime_copy_us": 19.11, "copy_us": 16.749, "pattern_us": 17.246, "copy_bytes": 90046464,
                  "frac_of_pattern": 0.9964, "best_copy_us": 16.142, "best_copy_variant": "prefetch_c2_b256_g1024",
                  "best_copy_frac_peak": 0.6973, "frac_of_best_copy": 0.9337})
    return r


def _out(bench):
    return {
        "metric": bench.METRIC, "value": 5166.3, "unit": "GB/s", "pct_of_peak": 64.58, "n_gpus": 1, "steps": 200,
        "warmup": 20, "ms_per_step": 0.03488, "us_per_step": 34.88, "ms_per_step_eager_launch": 0.03512,
        "timing": "HIP graph of the K steps replayed once between HIP events on the launch stream",
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, BASELINE.json parameter distributions)",
        "config": {"workload": "configs[1] VGGT frame-attention pre-block: residual(+LayerScale)+LayerNorm on "
                               "x[8,1374,1024] then QK-LayerNorm+2D-RoPE on q,k[8,16,1374,64] (bf16)",
                   "step_bytes": 180194176, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": 5213.7, "peak": 8000.0, "unit": "GB/s", "frac": 0.6517,
                     "traffic": 90861488, "kernel": "head_kernel<BF16,64,LN,R1>", "op": "cfg1_qk_layernorm_rope2d",
                     "us": 17.288, "algorithmic_bytes": 90135424,
                     "timing": "HIP events around a graph of 100 cold launches replayed 5 times (the launch stream)",
                     "trace": {"file": "profiles/kernel_trace_cfg1_qk_layernorm_rope2d.md", "kernel": "void lux3d::"
                               "(anonymous namespace)::head_kernel<lux3d::BF16, 64, 1, 2, 2, 1, true>"
                               "(lux3d::HeadParams, int)", "us": 18.344, "launches": 603, "frac": 0.6142,
                               "events_over_trace": 0.9424},
                     "runtime_copy": {"us": 19.11, "gbs": 4716.6, "what": "hipMemcpyAsync D2D of the same bytes "
                                                                         "(half read, half written)"},
                     "best_copy": {"us": 16.142, "variant": "prefetch_c2_b256_g1024", "frac_peak": 0.6973,
                                   "kernel_over_copy": 0.9337}},
        "cpu_baseline": {"value": 3.561, "unit": "GB/s", "cores": 16, "kind": "port",
                         "sample": "configs[1] step on 1 of 8 frames: F1 residual+LayerScale+LN on [1374,1024] "
                                   "bf16, Rope2d tables, QK LN+RoPE on q,k [1,16,1374,64] bf16; median of 20 runs "
                                   "after 3 warm-ups, per thread count", "value_1thread": 0.342,
                         "os_cpu_count": 16, "affinity_cpus": 16, "threads_used": 16,
                         "what": "C restatement of candle's CPU path (oracle/lux3d_oracle.c, gcc -O2), rows split "
                                 "over threads like candle's rayon-over-rows; candle itself is not buildable here",
                         "statistic": "median of 20 runs after 3 warm-ups, per thread count"},
    }


def _table(n_target=12, n_mfma=24, n_other=16):
    rows = [_row(f"cfg{k % 5}_target_op_with_a_long_name_{k:02d}", True, False) for k in range(n_target)]
    rows += [_row(f"cfg{k % 5}_matrix_core_op_with_a_long_name_{k:02d}", False, True) for k in range(n_mfma)]
    rows += [_row(f"cfg{k % 5}_other_op_with_a_long_name_{k:02d}", False, False) for k in range(n_other)]
    return rows


def test_headline_line_is_one_short_json_line():
    bench = _bench()
    line = bench.headline_json(_out(bench), _table())
    assert "\n" not in line
    assert len(line.encode()) < 8192, f"final line is {len(line.encode())} bytes"
    d = json.loads(line)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in d, key
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in d["roofline"], key
    for key in ("value", "unit", "cores", "kind", "sample"):
        assert key in d["cpu_baseline"], key
    assert "workload" in d["config"]


def test_headline_ops_entries_stay_compact():
    """One short entry per target or matrix-core op (the other rows stay in
    the full table): op, us, frac and the best copy or the matrix-core
    fraction, nothing else."""
    bench = _bench()
    table = _table()
    d = json.loads(bench.headline_json(_out(bench), table))
    assert len(d["ops"]) == 12 + 24
    for e in d["ops"]:
        assert set(e) <= {"op", "us", "frac", "best_copy_us", "frac_mfma"}, e
    # the table passed in is not modified (it is also written out in full)
    assert "cpu" in table[0] and "ops" not in _out(bench)
