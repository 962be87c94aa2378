"""Summaries of rocprofv3 output for the profiles/ directory.

    python -m tgo_amd.prof stats <dir>/<name>_kernel_stats.csv
        per-kernel calls, total and average duration (from --kernel-trace --stats
        --output-format csv).
    python -m tgo_amd.prof pmc <fetch_counter_collection.csv> <write_counter_collection.csv>
        per-kernel mean FETCH_SIZE and WRITE_SIZE per dispatch (KiB), each scaled by
        what the same counter reads for the copy-probe dispatch (torch.neg over a
        known number of bytes, bench.py --copy-probe-mib), and the attention
        kernel's scaled HBM bytes per launch.
"""
import collections
import csv
import sys


def short(name):
    if "neg_kernel" in name:
        return "copy-probe (torch.neg f32)"
    return name.split("(")[0].replace("void ", "")


def stats(path):
    rows = list(csv.DictReader(open(path)))
    tot = sum(float(r["TotalDurationNs"]) for r in rows)
    print("%-52s %7s %12s %11s %6s" % ("kernel", "calls", "total_ms", "avg_us", "pct"))
    for r in rows:
        print("%-52s %7d %12.3f %11.2f %6.2f" % (
            short(r["Name"])[:52], int(r["Calls"]), float(r["TotalDurationNs"]) / 1e6,
            float(r["AverageNs"]) / 1e3, 100 * float(r["TotalDurationNs"]) / tot))


def pmc(fetch_path, write_path, probe_mib):
    vals = {}
    for path, counter in ((fetch_path, "FETCH_SIZE"), (write_path, "WRITE_SIZE")):
        agg = collections.defaultdict(list)
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] == counter:
                agg[short(r["Kernel_Name"])].append(float(r["Counter_Value"]))
        vals[counter] = agg
    probe = "copy-probe (torch.neg f32)"
    known_kib = probe_mib * 1024.0
    f_scale = known_kib / vals["FETCH_SIZE"][probe][0]
    w_scale = known_kib / vals["WRITE_SIZE"][probe][0]
    print("copy probe: %d MiB read and written; FETCH_SIZE reads %.1f KiB -> scale %.4f; "
          "WRITE_SIZE reads %.1f KiB -> scale %.4f" % (
              probe_mib, vals["FETCH_SIZE"][probe][0], f_scale, vals["WRITE_SIZE"][probe][0],
              w_scale))
    print("%-52s %6s %14s %14s %14s" % ("kernel", "disp", "fetch_MB", "write_MB", "hbm_MB"))
    names = sorted(set(vals["FETCH_SIZE"]) & set(vals["WRITE_SIZE"]),
                   key=lambda n: -sum(vals["FETCH_SIZE"][n]))
    for n in names:
        f = vals["FETCH_SIZE"][n]
        w = vals["WRITE_SIZE"][n]
        fm = sum(f) / len(f) * f_scale * 1024 / 1e6
        wm = sum(w) / len(w) * w_scale * 1024 / 1e6
        print("%-52s %6d %14.3f %14.3f %14.3f" % (n[:52], len(f), fm, wm, fm + wm))
        if n.startswith("tgohip::attn_kernel"):
            attn = (fm + wm) * 1e6
    print("traffic_bytes_per_launch attn_kernel: %.0f" % attn)


if __name__ == "__main__":
    if sys.argv[1] == "stats":
        stats(sys.argv[2])
    elif sys.argv[1] == "pmc":
        pmc(sys.argv[2], sys.argv[3], int(sys.argv[4]) if len(sys.argv) > 4 else 1024)
    else:
        sys.exit(__doc__)
