"""Turn a rocprofv3 kernel-stats CSV into the markdown summary kept under profiles/.

Usage: python sageattention-rdna3_amd/profile_summary.py STATS_CSV OUT_MD "TITLE" "COMMAND"
"""
import csv
import sys


def main():
    stats, out, title, command = sys.argv[1:5]
    rows = list(csv.DictReader(open(stats)))
    lines = [f"# {title}", "", "Command (repo root on the GPU box):", "", f"    {command}", "",
             "Calls include bench.py's warmup, timed steps and its per-kernel HIP-event loops.", "",
             "| kernel | calls | avg (us) | min (us) | max (us) | share |", "|---|---|---|---|---|---|"]
    for r in rows:
        name = r["Name"]
        if "sage::" not in name:
            continue
        short = name.split("(anonymous namespace)::")[1].split("(sage")[0]
        lines.append(f"| `{short}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                     f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | {r['Percentage']}% |")
    open(out, "w").write("\n".join(lines) + "\n")


if __name__ == "__main__":
    main()
