"""Summaries of rocprofv3 output for the profiles/ directory.

    python -m tgo_amd.prof stats <dir>/<name>_kernel_stats.csv
        per-kernel calls, total and average duration (from --kernel-trace --stats
        --output-format csv).
    python -m tgo_amd.prof mfma <counter_collection.csv> <label>
        per projection of the step (QKV, O, gate/up, down, LM head, told apart by their
        place in the layer's launch sequence): dispatches, mean duration, the dense f16
        MFMA flops executed (SQ_INSTS_VALU_MFMA_MOPS_F16 x 512) per second and as a
        fraction of 2.5 PFLOP/s, and the MFMA busy fraction
        (SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 x 1024 SIMDs): the CSV's
        GRBM_GUI_ACTIVE is the sum over the 8 XCDs, each counting the dispatch's cycles,
        which its ratio to the duration shows), from one rocprofv3 --pmc pass over those
        three counters.
    python -m tgo_amd.prof grids <dir>/<name>_kernel_trace.csv
        per (kernel, grid size): dispatches and the median and mean duration, so
        launches of one kernel at different shapes stay apart (from --kernel-trace
        --output-format csv).
    python -m tgo_amd.prof pmcproj <fetch_counter_collection.csv> <write_counter_collection.csv> [probe_mib [label]]
        the same scaled FETCH_SIZE / WRITE_SIZE per projection of the step (labelled as
        by mfma), with the fetch over the projection's int4-sym weight bytes at the C4
        (Qwen3-8B) shapes; with a label, also one line per projection
        "traffic <label> <proj> <fetch bytes> <write bytes>" per dispatch.
    python -m tgo_amd.prof sq <pass_a_counter_collection.csv> <pass_b_counter_collection.csv> <label>
        per projection: the MFMA unit's busy fraction of the SIMD cycles, the cycles
        other VALU instructions issue, how many of those co-issue with a busy MFMA unit,
        and the cycles with neither (from the counters named in sq's docstring).
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


def grids(path):
    agg = collections.defaultdict(list)
    for r in csv.DictReader(open(path)):
        key = (short(r["Kernel_Name"]), int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) *
               int(r["Grid_Size_Z"]), int(r["Workgroup_Size_X"]))
        agg[key].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    print("%-52s %10s %6s %7s %10s %10s" % ("kernel", "threads", "wg", "disp", "median_us",
                                           "mean_us"))
    for (name, grid, wg), d in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        d = sorted(d)
        print("%-52s %10d %6d %7d %10.2f %10.2f" % (name[:52], grid, wg, len(d), d[len(d) // 2],
                                                   sum(d) / len(d)))


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


# int4-sym weight + scale bytes of the C4 (Qwen3-8B) projections: K*N*(0.5 + 2/32)
C4_WEIGHT_BYTES = {"qkv": 4096 * 6144 * 0.5625, "o": 4096 * 4096 * 0.5625,
                   "gateup": 4096 * 24576 * 0.5625, "down": 12288 * 4096 * 0.5625,
                   "lm_head": 4096 * 151936 * 0.5625}


def pmcproj(fetch_path, write_path, probe_mib, label=None):
    probe = "copy-probe (torch.neg f32)"
    known_kib = probe_mib * 1024.0
    res = {}
    for path, counter in ((fetch_path, "FETCH_SIZE"), (write_path, "WRITE_SIZE")):
        per = {}
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] == counter:
                d = per.setdefault(int(r["Dispatch_Id"]), {"name": short(r["Kernel_Name"]), "v": 0.0})
                d["v"] += float(r["Counter_Value"])
        ids = sorted(per)
        names = [per[i]["name"] for i in ids]
        scale = known_kib / next(per[i]["v"] for i in ids if per[i]["name"] == probe)
        agg = collections.defaultdict(list)
        for i, lab in zip(ids, label_projections(names)):
            if lab:
                agg[lab].append(per[i]["v"] * scale * 1024)
        res[counter] = agg
    print("%-8s %6s %12s %12s %14s %12s" % ("proj", "disp", "fetch_MB", "write_MB", "weights_MB",
                                             "fetch/wts"))
    for lab in ("qkv", "o", "gateup", "down", "lm_head"):
        f = res["FETCH_SIZE"].get(lab)
        w = res["WRITE_SIZE"].get(lab)
        if not f or not w:
            continue
        fm, wm = sum(f) / len(f) / 1e6, sum(w) / len(w) / 1e6
        wb = C4_WEIGHT_BYTES[lab] / 1e6
        print("%-8s %6d %12.2f %12.2f %14.2f %12.3f" % (lab, len(f), fm, wm, wb, fm / wb))
    if label:
        # machine-readable: HBM bytes per dispatch (fetch + write), for bench.py's roofline
        for lab in ("qkv", "o", "gateup", "down", "lm_head"):
            f = res["FETCH_SIZE"].get(lab)
            w = res["WRITE_SIZE"].get(lab)
            if f and w:
                print("traffic %s %s %.0f %.0f" % (label, lab, sum(f) / len(f), sum(w) / len(w)))


MFMA_PEAK_TFLOPS = 2500.0
SIMDS = 1024  # 256 CUs x 4
XCDS = 8      # GRBM_GUI_ACTIVE is reported summed over the XCDs


def label_projections(names):
    """The projection each GEMM dispatch computes, from the step's launch order: per layer
    rmsnorm, QKV, qk_rope_kv (unless the QKV epilogue does its work), attention (+ combine),
    O, rmsnorm, gate/up, down; after the
    last layer a gathered rmsnorm and the LM head, followed by the greedy selection
    (argmax_part_kernel; zero_idle_rows_kernel in traces of earlier builds)."""
    labels = [None] * len(names)
    prev_gemm = None
    for i, n in enumerate(names):
        if "gemm_reduce" in n or "repack" in n or not ("gemm_" in n):
            continue
        before = next((names[j] for j in range(i - 1, -1, -1)
                       if "gemm_reduce" not in names[j]), "")
        after = names[i + 1] if i + 1 < len(names) else ""
        if "zero_idle" in after or "argmax" in after:
            lab = "lm_head"
        elif "attn_" in before:
            lab = "o"
        elif "gemm_" in before:
            lab = "down"
        elif "rmsnorm" in before:
            lab = "gateup" if prev_gemm == "o" else "qkv"
        else:
            lab = None
        labels[i] = lab
        prev_gemm = lab
    return labels


def mfma(path, label):
    per = collections.defaultdict(dict)  # dispatch -> {counter: value, name, t}
    for r in csv.DictReader(open(path)):
        d = per[int(r["Dispatch_Id"])]
        d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        d["name"] = short(r["Kernel_Name"])
        d["ns"] = float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
    ids = sorted(per)
    names = [per[i]["name"] for i in ids]
    labels = label_projections(names)
    agg = collections.defaultdict(lambda: collections.defaultdict(float))
    for i, lab in zip(ids, labels):
        if lab is None:
            continue
        d = per[i]
        a = agg[lab]
        a["n"] += 1
        a["ns"] += d["ns"]
        a["mops"] += d.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0)
        a["busy"] += d.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0)
        a["gui"] += d.get("GRBM_GUI_ACTIVE", 0.0)
        a["kernel"] = d["name"]
    print("%-8s %-44s %5s %10s %7s %12s %9s %9s" % ("proj", "kernel", "disp", "avg_us", "GHz",
                                                    "mfma_TFLOP/s", "of_peak", "busy"))
    for lab in ("qkv", "o", "gateup", "down", "lm_head"):
        a = agg.get(lab)
        if not a:
            continue
        tflops = a["mops"] * 512 / (a["ns"] * 1e-9) / 1e12
        busy = a["busy"] / (a["gui"] / XCDS * SIMDS) if a["gui"] else 0.0
        print("%-8s %-44s %5d %10.2f %7.3f %12.1f %9.4f %9.4f" % (
            lab, a["kernel"][:44], a["n"], a["ns"] / a["n"] / 1e3, a["gui"] / XCDS / a["ns"],
            tflops, tflops / MFMA_PEAK_TFLOPS, busy))
    for lab in ("qkv", "o", "gateup", "down", "lm_head"):
        a = agg.get(lab)
        if a:
            tflops = a["mops"] * 512 / (a["ns"] * 1e-9) / 1e12
            busy = a["busy"] / (a["gui"] / XCDS * SIMDS) if a["gui"] else 0.0
            print("mfma %s %s %.1f %.4f %.4f" % (label, lab, tflops, tflops / MFMA_PEAK_TFLOPS, busy))


def _per_label(path):
    """Counter sums, dispatch counts and durations per projection label."""
    per = collections.defaultdict(dict)
    for r in csv.DictReader(open(path)):
        d = per[int(r["Dispatch_Id"])]
        d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        d["name"] = short(r["Kernel_Name"])
        d["ns"] = float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
    ids = sorted(per)
    out = collections.defaultdict(lambda: collections.defaultdict(float))
    for i, lab in zip(ids, label_projections([per[i]["name"] for i in ids])):
        if lab is None:
            continue
        for k, v in per[i].items():
            if k != "name":
                out[lab][k] += v
        out[lab]["n"] += 1
    return out


def sq(path_a, path_b, label):
    """Where a projection's SIMD cycles go, from two passes: A = SQ_VALU_MFMA_BUSY_CYCLES,
    SQ_VALU_MFMA_COEXEC_CYCLES, SQ_INSTS_VALU, GRBM_GUI_ACTIVE; B = SQ_INSTS_MFMA,
    GRBM_GUI_ACTIVE. SIMD cycles = GRBM_GUI_ACTIVE / 8 x 1024. SQ_INSTS_VALU counts the
    MFMAs too; each other VALU instruction issues over 4 cycles (a wave64 on a 16-lane
    SIMD). co-issued = cycles with the MFMA unit busy and a VALU instruction issued."""
    a, b = _per_label(path_a), _per_label(path_b)
    print("%-8s %5s %9s %10s %10s %11s %10s %8s" % (
        "proj", "disp", "avg_us", "mfma_busy", "valu_issue", "co-issued", "valu_only", "neither"))
    for lab in ("qkv", "o", "gateup", "down", "lm_head"):
        if lab not in a or lab not in b:
            continue
        A, B = a[lab], b[lab]
        cyc = A["GRBM_GUI_ACTIVE"] / XCDS * SIMDS
        busy = A["SQ_VALU_MFMA_BUSY_CYCLES"] / cyc
        coex = A["SQ_VALU_MFMA_COEXEC_CYCLES"] / cyc
        valu = 4 * (A["SQ_INSTS_VALU"] / A["n"] - B["SQ_INSTS_MFMA"] / B["n"]) * A["n"] / cyc
        only = max(0.0, valu - coex)
        print("%-8s %5d %9.2f %10.3f %10.3f %11.3f %10.3f %8.3f" % (
            lab, A["n"], A["ns"] / A["n"] / 1e3, busy, valu, coex, only, max(0.0, 1 - busy - only)))
        print("sq %s %s %.4f %.4f %.4f %.4f" % (label, lab, busy, valu, coex, only))


if __name__ == "__main__":
    if sys.argv[1] == "stats":
        stats(sys.argv[2])
    elif sys.argv[1] == "grids":
        grids(sys.argv[2])
    elif sys.argv[1] == "mfma":
        mfma(sys.argv[2], sys.argv[3])
    elif sys.argv[1] == "pmcproj":
        pmcproj(sys.argv[2], sys.argv[3], int(sys.argv[4]) if len(sys.argv) > 4 else 1024,
                sys.argv[5] if len(sys.argv) > 5 else None)
    elif sys.argv[1] == "sq":
        sq(sys.argv[2], sys.argv[3], sys.argv[4])
    elif sys.argv[1] == "pmc":
        pmc(sys.argv[2], sys.argv[3], int(sys.argv[4]) if len(sys.argv) > 4 else 1024)
    else:
        sys.exit(__doc__)
