"""Turn rocprofv3 CSV output into the short text summaries kept in profiles/.

  python -m lux3d_fused.rocprof_summary stats <kernel_stats.csv> "<command>" > profiles/<name>.md
  python -m lux3d_fused.rocprof_summary trace <kernel_stats.csv> <kernel-substring> <bytes> "<command>" \
        [<stdout of the profiled command> [<flops per launch> <peak TFLOP/s>]] > profiles/kernel_trace_<op>.md
  python -m lux3d_fused.rocprof_summary traffic <fetch.csv> <write.csv> <cal_fetch.csv> <cal_write.csv> \
        <kernel-substring> "<command>" > profiles/<name>.md
  python -m lux3d_fused.rocprof_summary counters <counter_collection.csv> <kernel-substring> "<command>" \
        > profiles/<name>.md
  python -m lux3d_fused.rocprof_summary sweep <kernel_trace.csv> <stdout of the traced sweep> "<command>" \
        [<stdout of the unprofiled sweep> "<its command>"] > profiles/ceiling_sweep.md
  python -m lux3d_fused.rocprof_summary rotation <kernel_trace.csv> <kernel-substring> \
        <stdout of bench.py --profile> "<command>" > profiles/rotation_<op>.md

`trace` reports the kernels whose name contains <kernel-substring> (the op's
own kernels, alternatives separated by `|`; the workload set-up kernels are
listed apart), each with its
average duration and the achieved bandwidth for <bytes> algorithmic bytes
per launch (and, for matrix-core ops, the achieved TFLOP/s for <flops> per
launch against <peak>), in a JSON block that bench.py reads back.
`counters` reports the median per-dispatch value of every counter in the
file for the matching kernels, and per-wavefront instruction counts when
SQ_WAVES was collected.

`sweep` reports the plain-copy sweep of `bench.py --ceiling-sweep`: the
traced copies sliced per (size, variant) by the manifest that run printed
(its timed graph replays only), their average duration and bandwidth, and
the fastest variant per size; with the unprofiled run's stdout it adds that
run's HIP-event table of the whole variant family.

`rotation` splits the per-dispatch durations of one op's kernel (the trace
of `bench.py --profile <op>`) by rotation set and by position in the timed
graph, to show where the spread between the fastest and slowest launches
comes from.

`traffic` reports the per-dispatch HBM bytes of the kernels whose name
contains <kernel-substring>, with FETCH_SIZE and WRITE_SIZE (KiB per
dispatch) scaled by what the same counters read for a copy kernel of known
size (bench.py --profile copy_1gib: 1 GiB read + 1 GiB written).
"""
import csv
import json
import statistics
import sys


NOTE = ("`$REPO` is the repository root; this file is `python -m lux3d_fused.rocprof_summary` (run from "
        "`candle-3d_amd/`) of the CSV that command writes.")


def _rows(path):
    with open(path) as f:
        return list(csv.DictReader(f))


def stats(path, command):
    rows = _rows(path)
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    out = ["# rocprofv3 kernel statistics", "", f"Command: `{command}`", "",
           "| kernel | calls | avg us | min us | max us | % time |", "|---|---|---|---|---|---|"]
    for r in rows:
        name = r["Name"].replace("|", "/")
        if len(name) > 110:
            name = name[:107] + "..."
        out.append(f"| `{name}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.3f} | "
                   f"{float(r['MinNs']) / 1e3:.3f} | {float(r['MaxNs']) / 1e3:.3f} | {float(r['Percentage']):.2f} |")
    return "\n".join(out) + "\n"


def _profiled_line(log_path):
    """The JSON line `bench.py --profile` printed while it ran under the
    profiler (HIP-event time per launch, op launches, bytes, flops), or {}."""
    if not log_path:
        return {}
    for line in open(log_path):
        if line.startswith("{") and '"us_per_launch_graph"' in line:
            return json.loads(line)
    return {}


def trace(path, kernel_sub, nbytes, command, log_path=None, flops=None, peak_tflops=None):
    rows = _rows(path)
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    subs = kernel_sub.split("|")
    mine = [r for r in rows if any(s in r["Name"] for s in subs)]
    rest = [r for r in rows if r not in mine]
    nbytes = int(nbytes)
    flops = int(flops) if flops else None
    peak = float(peak_tflops) if peak_tflops else None
    res = {"bytes_per_launch": nbytes, "kernels": []}
    if flops:
        res.update({"flops_per_launch": flops, "peak_tflops": peak})
    single = len(mine) == 1  # per-kernel rates only when one kernel is the whole op
    for r in mine:
        avg = float(r["AverageNs"]) / 1e3
        k = {"name": r["Name"], "calls": int(r["Calls"]), "avg_us": round(avg, 3),
             "min_us": round(float(r["MinNs"]) / 1e3, 3), "max_us": round(float(r["MaxNs"]) / 1e3, 3)}
        if single:
            k.update({"gbs": round(nbytes / avg / 1e3, 1), "frac_of_8tbs": round(nbytes / avg / 8e6, 4)})
            if flops:
                k.update({"tflops": round(flops / avg / 1e6, 1),
                          "frac_of_peak_tflops": round(flops / avg / 1e6 / peak, 4)})
        res["kernels"].append(k)
    what = (f"bandwidth = {nbytes:,} algorithmic bytes per launch / average duration" +
            (f"; rate = {flops:,} flops per launch / average duration, against {peak} TFLOP/s" if flops else ""))
    out = ["# rocprofv3 kernel trace", "", f"Command: `{command}`", "", NOTE, "",
           f"Kernels matching `{kernel_sub}` (the op's own launches, all on cold rotation sets); {what}.", ""]
    if flops:
        out += ["| kernel | calls | avg us | min us | max us | GB/s | TFLOP/s | of peak |",
                "|---|---|---|---|---|---|---|---|"]
    else:
        out += ["| kernel | calls | avg us | min us | max us | GB/s | of 8 TB/s |", "|---|---|---|---|---|---|---|"]
    for k in res["kernels"]:
        name = k["name"].replace("|", "/")
        if single:
            rates = f"{k['gbs']:,.1f} | " + (f"{k['tflops']:,.1f} | {k['frac_of_peak_tflops']:.4f} |" if flops
                                              else f"{k['frac_of_8tbs']:.4f} |")
        else:
            rates = "- | - | - |" if flops else "- | - |"
        out.append(f"| `{name[:110]}` | {k['calls']} | {k['avg_us']:.3f} | {k['min_us']:.3f} | {k['max_us']:.3f} | "
                   + rates)
    run = _profiled_line(log_path)
    if run.get("launches") and len(res["kernels"]) > 1:
        # several kernels per op launch: the op's time is their summed durations per launch
        op_us = sum(float(r["TotalDurationNs"]) for r in mine) / 1e3 / run["launches"]
        res["op_us_per_launch"] = round(op_us, 3)
        out += ["", f"Op time per launch (the matching kernels' summed durations / {run['launches']} op launches): "
                    f"{op_us:.3f} us" + (f", {flops / op_us / 1e6:,.1f} TFLOP/s ({flops / op_us / 1e6 / peak:.4f} of "
                                         f"{peak} TFLOP/s)" if flops else f", {nbytes / op_us / 1e3:,.1f} GB/s") + "."]
    ev = run.get("us_per_launch_graph")
    if ev is not None:
        res["events_us_under_profiler"] = ev
        out += ["", f"The same launches timed with HIP events around the graph replays, inside the profiled run: "
                    f"{ev:.3f} us per launch. Each traced dispatch carries the profiler's own per-dispatch cost; "
                    f"bench.py's unprofiled graph timing of the same launches (its ops[].us) is lower by that cost."]
    if rest:
        out += ["", "Other kernels in the process (workload set-up):", ""]
        for r in rest[:6]:
            out.append(f"- `{r['Name'][:90]}`: {r['Calls']} calls, {float(r['AverageNs']) / 1e3:.3f} us avg")
    out += ["", "```json", json.dumps(res, indent=1), "```"]
    return "\n".join(out) + "\n"


def counters(path, kernel_sub, command):
    vals = {}
    for r in _rows(path):
        if kernel_sub not in r["Kernel_Name"]:
            continue
        vals.setdefault(r["Kernel_Name"], {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    res = {}
    for name, cs in vals.items():
        med = {c: statistics.median(v) for c, v in cs.items()}
        d = {"dispatches": max(len(v) for v in cs.values()), "median_per_dispatch": med}
        waves = med.get("SQ_WAVES")
        if waves:
            d["per_wavefront"] = {c: round(v / waves, 2) for c, v in med.items() if c.startswith("SQ_INSTS")}
        if med.get("SQ_BUSY_CYCLES") and med.get("SQ_WAVE_CYCLES"):
            d["wave_cycles_over_busy_cycles"] = round(med["SQ_WAVE_CYCLES"] / med["SQ_BUSY_CYCLES"], 2)
        res[name] = d
    out = ["# rocprofv3 counters (median per dispatch)", "", f"Command: `{command}`", "", NOTE, ""]
    for name, d in res.items():
        out += [f"Kernel `{name[:120]}` ({d['dispatches']} dispatches):", "",
                "| counter | median per dispatch |", "|---|---|"]
        for c, v in sorted(d["median_per_dispatch"].items()):
            out.append(f"| {c} | {v:,.0f} |")
        if "per_wavefront" in d:
            out += ["", "Per wavefront: " + ", ".join(f"{c} {v}" for c, v in d["per_wavefront"].items())]
        out.append("")
    out += ["```json", json.dumps(res, indent=1), "```"]
    return "\n".join(out) + "\n"


def _per_kernel(path, counter):
    vals = {}
    for r in _rows(path):
        if r["Counter_Name"] != counter:
            continue
        vals.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
    return vals


def traffic(fetch, write, cal_fetch, cal_write, kernel_sub, command):
    f = _per_kernel(fetch, "FETCH_SIZE")
    w = _per_kernel(write, "WRITE_SIZE")
    cf = _per_kernel(cal_fetch, "FETCH_SIZE")
    cw = _per_kernel(cal_write, "WRITE_SIZE")
    cal_name = max(cf, key=lambda k: statistics.median(cf[k]))  # the 1 GiB copy dominates
    gib_kib = float(1 << 20)
    f_scale = gib_kib / statistics.median(cf[cal_name])
    w_scale = gib_kib / statistics.median(cw[cal_name])
    res = {"fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4), "calibration_kernel": cal_name,
           "kernels": {}}
    for name in f:
        if kernel_sub not in name:
            continue
        fk = statistics.median(f[name]) * f_scale * 1024
        wk = statistics.median(w.get(name, [0.0])) * w_scale * 1024
        res["kernels"][name] = {"read_bytes": int(fk), "write_bytes": int(wk), "hbm_bytes": int(fk + wk),
                                "dispatches": len(f[name])}
    lines = ["# HBM traffic per dispatch (rocprofv3 FETCH_SIZE / WRITE_SIZE)", "",
             f"Command: `{command}`", "", NOTE, "",
             f"Calibration: `{cal_name}` (1 GiB read + 1 GiB written) reads FETCH_SIZE x{f_scale:.4f}, "
             f"WRITE_SIZE x{w_scale:.4f} of the true bytes; the factors below are applied.", "",
             "| kernel | dispatches | read bytes | write bytes | total |", "|---|---|---|---|---|"]
    for name, v in res["kernels"].items():
        lines.append(f"| `{name[:100]}` | {v['dispatches']} | {v['read_bytes']:,} | {v['write_bytes']:,} | "
                     f"{v['hbm_bytes']:,} |")
    lines += ["", "```json", json.dumps(res, indent=1), "```"]
    return "\n".join(lines) + "\n"


def _trace_rows(path, kernel_sub):
    subs = kernel_sub.split("|")
    rows = [r for r in _rows(path) if any(s in r["Kernel_Name"] for s in subs)]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    return [(r["Kernel_Name"], (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3) for r in rows]


def _json_lines(log_path, key):
    out = []
    for line in open(log_path):
        if line.startswith("{") and f'"{key}"' in line:
            out.append(json.loads(line))
    return out


def sweep(trace_csv, log_path, command, events_log=None, events_command=None):
    """Per (size, variant) average duration of the traced copies."""
    man = _json_lines(log_path, "manifest")[0]["manifest"]
    best_line = _json_lines(log_path, "sweep_best")[0]
    iters = best_line["iters"]
    durs = [d for _, d in _trace_rows(trace_csv, "best_kernel")]
    pos, table = 0, {}
    for e in man:
        seg = durs[pos:pos + e["dispatches"]]
        pos += e["dispatches"]
        timed = seg[3 + iters:]  # skip the eager warm-ups and the first graph replay
        table.setdefault(e["mb"], {})[e["variant"]] = sum(timed) / len(timed)
    out = ["# Plain-copy ceiling by copy size (rocprofv3 kernel trace)", "",
           f"Command: `{command}`", "", NOTE, "",
           "Each size moves MB x 10^6 bytes per launch, half read and half written, over rotation sets "
           "that together exceed the 256 MB Infinity Cache; durations are the traced average of the timed "
           "graph replays. Variants: oneshot = one workgroup per tile; strided = a persistent grid of g "
           "workgroups striding over tiles; prefetch = persistent, the next tile loaded before the current "
           "one is stored; c = 16-byte chunks per thread per tile, b = threads per workgroup.", "",
           "| MB | fastest variant | us | GB/s | of 8 TB/s | oneshot_c1_b256 us |", "|---|---|---|---|---|---|"]
    res = {}
    for mb, vs in table.items():
        k = min(vs, key=vs.get)
        gbs = mb * 1e6 / vs[k] / 1e3
        res[mb] = {"variant": k, "us": round(vs[k], 3), "gbs": round(gbs, 1), "frac": round(gbs / 8000.0, 4),
                   "all_us": {v: round(u, 3) for v, u in vs.items()}}
        base = vs.get("oneshot_c1_b256")
        out.append(f"| {mb} | {k} | {vs[k]:.3f} | {gbs:,.1f} | {gbs / 8000.0:.4f} | "
                   + (f"{base:.3f}" if base else "-") + " |")
    if events_log:
        ev = _json_lines(events_log, "sweep_mb")
        out += ["", f"The whole variant family, HIP events around the graph replays (unprofiled): "
                    f"`{events_command}`", "",
                "| MB | fastest | us | GB/s | of 8 TB/s | oneshot_c1_b256 | strided_c1_b256_g1024 |",
                "|---|---|---|---|---|---|---|"]
        for e in ev:
            us = e["us"]
            k = min(us, key=us.get)
            gbs = e["bytes"] / us[k] / 1e3
            out.append(f"| {e['sweep_mb']} | {k} | {us[k]:.3f} | {gbs:,.1f} | {gbs / 8000.0:.4f} | "
                       f"{us.get('oneshot_c1_b256', float('nan')):.3f} | "
                       f"{us.get('strided_c1_b256_g1024', float('nan')):.3f} |")
    out += ["", "```json", json.dumps(res, indent=1), "```"]
    return "\n".join(out) + "\n"


def rotation(trace_csv, kernel_sub, log_path, command):
    """Durations of one op's launches by rotation set and graph position."""
    prof = next(line for line in open(log_path) if line.startswith("[profile]"))
    sets = int(prof.split("sets=")[1].split()[0])
    iters = int(prof.split("iters=")[1].split()[0])
    d = [u for _, u in _trace_rows(trace_csv, kernel_sub)]
    # time_graph: 3 eager launches (sets 0..2), then the graph of `iters`
    # launches (launch i on set i % sets) replayed 6 times
    graph = d[3:]
    by_set, by_pos = {}, {}
    for j, u in enumerate(graph):
        i = j % iters
        by_set.setdefault(i % sets, []).append(u)
        by_pos.setdefault(min(i, 3) if i < 3 else "3+", []).append(u)
    s = sorted(graph)
    pct = lambda q: s[min(len(s) - 1, int(q * len(s)))]  # noqa: E731
    out = ["# Per-launch durations by rotation set and graph position (rocprofv3 kernel trace)", "",
           f"Command: `{command}`", "", NOTE, "",
           f"Kernels matching `{kernel_sub}`: {len(graph)} graph launches ({iters} per replay, {sets} rotation "
           f"sets). min {s[0]:.3f}, p10 {pct(0.1):.3f}, median {pct(0.5):.3f}, p90 {pct(0.9):.3f}, "
           f"max {s[-1]:.3f} us.", "", "| rotation set | launches | avg us | min us | max us |", "|---|---|---|---|---|"]
    for k in sorted(by_set):
        v = by_set[k]
        out.append(f"| {k} | {len(v)} | {sum(v) / len(v):.3f} | {min(v):.3f} | {max(v):.3f} |")
    out += ["", "| position in the graph | launches | avg us | min us | max us |", "|---|---|---|---|---|"]
    for k in [0, 1, 2, "3+"]:
        v = by_pos.get(k, [])
        if v:
            out.append(f"| {k} | {len(v)} | {sum(v) / len(v):.3f} | {min(v):.3f} | {max(v):.3f} |")
    res = {"sets": sets, "iters": iters, "launches": len(graph), "min": s[0], "median": pct(0.5), "max": s[-1],
           "by_set_avg": {k: round(sum(v) / len(v), 3) for k, v in by_set.items()},
           "by_position_avg": {str(k): round(sum(v) / len(v), 3) for k, v in by_pos.items()}}
    out += ["", "```json", json.dumps(res, indent=1), "```"]
    return "\n".join(out) + "\n"


def main(argv):
    if argv[0] == "stats":
        sys.stdout.write(stats(argv[1], argv[2]))
    elif argv[0] == "trace":
        sys.stdout.write(trace(*argv[1:8]))
    elif argv[0] == "counters":
        sys.stdout.write(counters(*argv[1:4]))
    elif argv[0] == "traffic":
        sys.stdout.write(traffic(*argv[1:7]))
    elif argv[0] == "sweep":
        sys.stdout.write(sweep(*argv[1:6]))
    elif argv[0] == "rotation":
        sys.stdout.write(rotation(*argv[1:5]))
    else:
        raise SystemExit(__doc__)


if __name__ == "__main__":
    main(sys.argv[1:])
