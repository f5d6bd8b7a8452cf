"""Summaries of rocprofv3 output kept under profiles/ (text only).

  python sageattention-rdna3_amd/profile_summary.py stats KERNEL_TRACE_CSV OUT_MD TITLE COMMAND [LAST_N]
      kernel trace -> markdown table of this library's kernels, one row per kernel and launch size (LAST_N:
      also the average of each row's last LAST_N calls, bench.py's HIP-event loop)
  python sageattention-rdna3_amd/profile_summary.py traffic FETCH_CSV WRITE_CSV OUT_JSON OUT_MD COMMAND
      two --pmc runs of `bench.py --kernels-only` (FETCH_SIZE, then WRITE_SIZE) -> HBM bytes per
      launch of every path kernel, each counter scaled by what it reads for the 1 GiB device copy
      the same run performs (a kernel of known traffic)
  python sageattention-rdna3_amd/profile_summary.py counters OUT_MD COMMAND CSV [CSV ...]
      --pmc runs -> per-kernel mean of every counter collected
"""
import collections
import csv
import json
import sys

COPY_BYTES = 1 << 30
KERNELS = ("attn_fwd_kernel", "prep_kv_kernel", "quant_qk_i8_kernel", "v_layout_kernel", "k_mean_partial_kernel",
           "k_mean_final_kernel", "attn_merge_kernel")


def short_name(name):
    if "sage::" in name:
        return name.split("(anonymous namespace)::")[1].split("(sage")[0]
    if "copyBuffer" in name:
        return "copy_1GiB"
    return None


def per_kernel(path, counter=None):
    """{kernel: [value per dispatch]} summed over counter dimensions."""
    acc = collections.defaultdict(float)
    names = {}
    for r in csv.DictReader(open(path)):
        if counter and r["Counter_Name"] != counter:
            continue
        k = short_name(r["Kernel_Name"])
        if k is None:
            continue
        key = (r["Dispatch_Id"], r["Counter_Name"])
        acc[key] += float(r["Counter_Value"])
        names[key] = k
    out = collections.defaultdict(lambda: collections.defaultdict(list))
    for key, v in acc.items():
        out[names[key]][key[1]].append(v)
    return out


def stats(trace_csv, out_md, title, command, last_n=0):
    """Per (kernel, grid) statistics from the kernel trace: one kernel runs at several shapes in one
    bench.py run (the NS workload and the direct-path probe), and each shape gets its own row.  With
    last_n, a column also averages each row's last last_n calls: for the path kernels of bench.py those
    are its HIP-event loop (after the warm-up and the timed steps), the calls `roofline` times."""
    groups = collections.defaultdict(list)
    for r in csv.DictReader(open(trace_csv)):
        k = short_name(r["Kernel_Name"])
        if k is None or k == "copy_1GiB":
            continue
        grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        blocks = grid // max(1, int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"]))
        groups[(k, blocks)].append((int(r["Start_Timestamp"]),
                                    (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
    total = sum(sum(x for _, x in v) for v in groups.values())
    last_n = int(last_n)
    extra = f" avg of last {last_n} (us) |" if last_n else ""
    lines = [f"# {title}", "", "Command (repo root on the GPU box):", "", f"    {command}", "",
             "Calls include bench.py's warmup, timed steps and its per-kernel HIP-event loops; one row per kernel "
             "and launch size (workgroups).", "",
             "| kernel | workgroups | calls | avg (us) | median (us) | min (us) | max (us) | share |" + extra,
             "|---|---|---|---|---|---|---|---|" + ("---|" if last_n else "")]
    for (k, blocks), calls in sorted(groups.items(), key=lambda kv: -sum(x for _, x in kv[1])):
        d = [x for _, x in sorted(calls)]
        med = sorted(d)[len(d) // 2]
        row = (f"| `{k}` | {blocks} | {len(d)} | {sum(d) / len(d):.1f} | {med:.1f} | {min(d):.1f} | "
               f"{max(d):.1f} | {100 * sum(d) / total:.2f}% |")
        if last_n:
            tail = d[-last_n:]
            row += f" {sum(tail) / len(tail):.1f} |"
        lines.append(row)
    open(out_md, "w").write("\n".join(lines) + "\n")


def traffic(fetch_csv, write_csv, out_json, out_md, command):
    fetch = per_kernel(fetch_csv, "FETCH_SIZE")
    write = per_kernel(write_csv, "WRITE_SIZE")
    mean = lambda d, k, c: sum(d[k][c]) / len(d[k][c]) * 1024.0  # KiB -> bytes
    f_scale = COPY_BYTES / mean(fetch, "copy_1GiB", "FETCH_SIZE")
    w_scale = COPY_BYTES / mean(write, "copy_1GiB", "WRITE_SIZE")
    res = {"fetch_scale": f_scale, "write_scale": w_scale, "kernels": {}}
    for k in fetch:
        if k == "copy_1GiB" or k not in write:
            continue
        fb = mean(fetch, k, "FETCH_SIZE") * f_scale
        wb = mean(write, k, "WRITE_SIZE") * w_scale
        res["kernels"][k] = {"fetch_bytes": fb, "write_bytes": wb, "bytes": fb + wb}
    # attn_fwd_kernel<D, QK, CAUSAL, OUT_BF16>: QK 3 is the INT8 kernel that quantises Q itself (the
    # one sageattn runs), QK 0 the INT8 kernel of the two-kernel op path
    names = {k.replace(" ", ""): v for k, v in res["kernels"].items()}
    attn = [v for k, v in names.items() if k.startswith(("attn_fwd_kernel<128,3,", "attn_fwd_kernel<64,3,"))]
    attn += [v for k, v in names.items() if k.startswith(("attn_fwd_kernel<128,0,", "attn_fwd_kernel<64,0,"))]
    if attn:
        res["attn_bytes_per_launch"] = attn[0]["bytes"]
    json.dump(res, open(out_json, "w"), indent=1)
    lines = ["# HBM traffic per launch (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)", "",
             "Commands (repo root on the GPU box), one counter per run:", ""]
    lines += [f"    {c}" for c in command.split(" ;; ")]
    lines += ["", f"Calibration with the 1 GiB device copy of the same runs: FETCH_SIZE x {f_scale:.3f}, "
              f"WRITE_SIZE x {w_scale:.3f}.", "",
              "| kernel | fetch (MB) | write (MB) | total (MB) |", "|---|---|---|---|"]
    for k, v in res["kernels"].items():
        lines.append(f"| `{k}` | {v['fetch_bytes'] / 1e6:.1f} | {v['write_bytes'] / 1e6:.1f} | {v['bytes'] / 1e6:.1f} |")
    open(out_md, "w").write("\n".join(lines) + "\n")


def dispatch_facts(path):
    """{kernel: {"duration_us": mean, "scratch": .., "LDS": ..}} of a counter CSV."""
    dur = collections.defaultdict(dict)
    res = collections.defaultdict(dict)
    for r in csv.DictReader(open(path)):
        k = short_name(r["Kernel_Name"])
        if k is None:
            continue
        dur[k][r["Dispatch_Id"]] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        res[k].update(scratch=int(r["Scratch_Size"]), LDS=int(r["LDS_Block_Size"]))
    for k, d in dur.items():
        res[k]["duration_us"] = sum(d.values()) / len(d)
    return res


def counters(out_md, command, paths, xcds=8, simds=1024):
    """Mean of every counter per kernel over the runs' dispatches, with derived figures: the kernel's cycles
    (GRBM_GUI_ACTIVE counts each XCD's clocks, summed over the XCDs), the MFMA pipe's busy share of every
    SIMD's cycles, and instructions per MFMA.  The dispatch time under the profiler includes the counter
    set-up, so cycles over it understate the clock; use a kernel trace's duration for that."""
    merged = collections.defaultdict(dict)
    facts = collections.defaultdict(dict)
    for pth in paths:
        for k, cs in per_kernel(pth).items():
            for c, vals in cs.items():
                merged[k][c] = sum(vals) / len(vals)
        for k, f in dispatch_facts(pth).items():
            facts[k].setdefault("durations", []).append(f.pop("duration_us"))
            facts[k].update(f)
    lines = ["# rocprofv3 --pmc counters per kernel (mean over dispatches, summed over dimensions)", "",
             "Commands (repo root on the GPU box), one counter group per run:", ""]
    lines += [f"    {c}" for c in command.split(" ;; ")]
    lines += ["", f"Derived: cycles = GRBM_GUI_ACTIVE / {xcds} XCDs; MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / {simds} SIMDs / "
              "cycles; per-MFMA ratios divide by SQ_INSTS_MFMA.  The dispatch time under the profiler includes the "
              "counter set-up: a kernel trace gives the kernel's own duration.", ""]
    for k in sorted(merged):
        c = merged[k]
        f = facts.get(k, {})
        lines += [f"## `{k}`", ""]
        if f:
            t = sum(f["durations"]) / len(f["durations"])
            lines += [f"Dispatch: {t:.1f} us under the profiler; scratch {f['scratch']} B, LDS {f['LDS']} B.", ""]
            derived = []
            if "GRBM_GUI_ACTIVE" in c:
                cyc = c["GRBM_GUI_ACTIVE"] / xcds
                derived.append(f"{cyc:.4g} cycles")
                if "SQ_VALU_MFMA_BUSY_CYCLES" in c:
                    derived.append(f"MFMA busy {c['SQ_VALU_MFMA_BUSY_CYCLES'] / simds / cyc:.1%} of each SIMD's cycles")
            if c.get("SQ_INSTS_MFMA"):
                for name in ("SQ_INSTS_VALU", "SQ_INSTS_VALU_TRANS_F32", "SQ_INSTS_LDS"):
                    if name in c:
                        derived.append(f"{name} per MFMA {c[name] / c['SQ_INSTS_MFMA']:.2f}")
            if derived:
                lines += ["Derived: " + "; ".join(derived) + ".", ""]
        lines += ["| counter | value |", "|---|---|"]
        lines += [f"| {n} | {v:.4g} |" for n, v in sorted(c.items())]
        lines += [""]
    open(out_md, "w").write("\n".join(lines) + "\n")


if __name__ == "__main__":
    mode = sys.argv[1]
    if mode == "stats":
        stats(*sys.argv[2:7])
    elif mode == "traffic":
        traffic(*sys.argv[2:7])
    elif mode == "counters":
        counters(sys.argv[2], sys.argv[3], sys.argv[4:])
    else:
        raise SystemExit(__doc__)
