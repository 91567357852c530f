"""Turn rocprofv3 CSV output into the short text summaries kept in profiles/.

  python -m lux3d_fused.rocprof_summary stats <kernel_stats.csv> "<command>" > profiles/<name>.md
  python -m lux3d_fused.rocprof_summary traffic <fetch.csv> <write.csv> <cal_fetch.csv> <cal_write.csv> \
        <kernel-substring> "<command>" > profiles/<name>.md

`traffic` reports the per-dispatch HBM bytes of the kernels whose name
contains <kernel-substring>, with FETCH_SIZE and WRITE_SIZE (KiB per
dispatch) scaled by what the same counters read for a copy kernel of known
size (bench.py --profile copy_1gib: 1 GiB read + 1 GiB written).
"""
import csv
import json
import statistics
import sys


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
             f"Command: `{command}`", "",
             f"Calibration: `{cal_name}` (1 GiB read + 1 GiB written) reads FETCH_SIZE x{f_scale:.4f}, "
             f"WRITE_SIZE x{w_scale:.4f} of the true bytes; the factors below are applied.", "",
             "| kernel | dispatches | read bytes | write bytes | total |", "|---|---|---|---|---|"]
    for name, v in res["kernels"].items():
        lines.append(f"| `{name[:100]}` | {v['dispatches']} | {v['read_bytes']:,} | {v['write_bytes']:,} | "
                     f"{v['hbm_bytes']:,} |")
    lines += ["", "```json", json.dumps(res, indent=1), "```"]
    return "\n".join(lines) + "\n"


def main(argv):
    if argv[0] == "stats":
        sys.stdout.write(stats(argv[1], argv[2]))
    elif argv[0] == "traffic":
        sys.stdout.write(traffic(*argv[1:7]))
    else:
        raise SystemExit(__doc__)


if __name__ == "__main__":
    main(sys.argv[1:])
