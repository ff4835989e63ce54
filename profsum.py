"""Summaries of rocprofv3 CSV output for the DiT step (kernel time table, calibrated HBM bytes per launch).

    python profsum.py stats  <kernel_stats.csv>  [top]
    python profsum.py grids  <kernel_trace.csv>  [name filter]
    python profsum.py pmc    <fetch counter_collection.csv> <write counter_collection.csv> [copy MiB]

`stats` prints the per-kernel time table of `rocprofv3 --kernel-trace --stats --output-format csv`.
`grids` prints, from the kernel trace, the launches, average and minimum duration per kernel and grid (one line
per shape of a benchmark that launches one kernel at several shapes).
`pmc` averages FETCH_SIZE and WRITE_SIZE (KiB per dispatch) per kernel and grid, and scales each counter by what
it reads for the plain uint8 bitwise_not copy of `copy MiB` that `bench.py --copy-probe` runs first (known bytes:
MiB read, MiB written), so that the reported figures are HBM bytes per launch.
"""

from __future__ import annotations

import collections
import csv
import re
import sys

KERNELS = re.compile(r"(w4a4_gemm_kernel<[^>]*>|w4a4_gemm_sk_kernel<[^>]*>|w4a4_gemm_bal_kernel<[^>]*>|"
                     r"w4a4_merge_kernel<[^>]*>|attn_merge_kernel|"
                     r"sage_attn_kernel|quant_kernel|quant_kv_kernel|colstats_kernel|"
                     r"qk_norm_rope_kernel|quant_q_kernel|row_stats_kernel|lora_sum_kernel|kv_append_kernel<[^>]*>|"
                     r"finalize_kernel|bitwise_not)")


def short(name: str) -> str:
    m = KERNELS.search(name)
    return m.group(1) if m else name[:60]


def stats(path: str, top: int = 20) -> str:
    # the spin kernel bench.py runs ahead of its instrumented step (torch.cuda._sleep) is not part of the step
    rows = [r for r in csv.DictReader(open(path)) if "spin_kernel" not in r["Name"]]
    total = sum(float(r["TotalDurationNs"]) for r in rows)
    out = ["| kernel | calls | total ms | avg us | % |", "|---|---:|---:|---:|---:|"]
    for r in rows[:top]:
        out.append(f"| `{short(r['Name'])}` | {int(r['Calls'])} | {float(r['TotalDurationNs']) / 1e6:.2f} | "
                   f"{float(r['AverageNs']) / 1e3:.1f} | {100 * float(r['TotalDurationNs']) / total:.2f} |")
    out.append(f"| all kernels but the spin | {sum(int(r['Calls']) for r in rows)} | {total / 1e6:.2f} | | 100 |")
    return "\n".join(out)


def grids(path: str, name_filter: str = "") -> str:
    runs = collections.defaultdict(list)
    for r in csv.DictReader(open(path)):
        if "spin_kernel" in r["Kernel_Name"] or name_filter not in r["Kernel_Name"]:
            continue
        grid = f"{r['Grid_Size_X']}x{r['Grid_Size_Y']}x{r['Grid_Size_Z']}"
        runs[(short(r["Kernel_Name"]), grid)].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    out = ["| kernel | grid (threads) | launches | avg us | min us |", "|---|---|---:|---:|---:|"]
    for (k, grid), d in runs.items():
        out.append(f"| `{k}` | {grid} | {len(d)} | {sum(d) / len(d):.1f} | {min(d):.1f} |")
    return "\n".join(out)


def _per_kernel(path: str):
    agg = collections.defaultdict(list)
    for r in csv.DictReader(open(path)):
        agg[(short(r["Kernel_Name"]), int(r["Grid_Size"]))].append(float(r["Counter_Value"]))
    return agg


def pmc(fetch_path: str, write_path: str, copy_mib: int = 1024) -> str:
    fetch, write = _per_kernel(fetch_path), _per_kernel(write_path)
    known_kib = copy_mib * 1024.0
    cal_f = [v for (k, _), vs in fetch.items() if k == "bitwise_not" for v in vs]
    cal_w = [v for (k, _), vs in write.items() if k == "bitwise_not" for v in vs]
    if not cal_f or not cal_w:
        raise SystemExit("no bitwise_not copy-probe dispatches in the counter files")
    ff = known_kib / (sum(cal_f) / len(cal_f))
    fw = known_kib / (sum(cal_w) / len(cal_w))
    out = [f"calibration: a {copy_mib} MiB uint8 copy reads FETCH_SIZE {sum(cal_f) / len(cal_f):.0f} KiB and "
           f"WRITE_SIZE {sum(cal_w) / len(cal_w):.0f} KiB per dispatch -> factors fetch x{ff:.3f}, write x{fw:.3f}",
           "", "| kernel | grid (threads) | dispatches | fetch MB/launch | write MB/launch | HBM MB/launch |",
           "|---|---:|---:|---:|---:|---:|"]
    keys = sorted(k for k in fetch if k[0] != "bitwise_not" and KERNELS.search(k[0]))
    for k in keys:
        f = sum(fetch[k]) / len(fetch[k]) * ff * 1024 / 1e6
        w = (sum(write[k]) / len(write[k]) * fw * 1024 / 1e6) if k in write else float("nan")
        out.append(f"| `{k[0]}` | {k[1]} | {len(fetch[k])} | {f:.1f} | {w:.1f} | {f + w:.1f} |")
    # the main-loop launches of the W4A4 GEMM (one-pass, balanced and stream-K; the stream-K merge is listed above)
    gemm = [k for k in keys if k[0].startswith(("w4a4_gemm_kernel", "w4a4_gemm_sk_kernel", "w4a4_gemm_bal_kernel"))]
    if gemm:
        n = sum(len(fetch[k]) for k in gemm)
        fb = sum(sum(fetch[k]) for k in gemm) / n * ff * 1024
        wb = sum(sum(write[k]) for k in gemm if k in write) / sum(len(write[k]) for k in gemm if k in write) * fw * 1024
        out += ["", f"w4a4_gemm_kernel, all launches: HBM bytes per launch (calibrated): {fb + wb:.0f} "
                    f"(fetch {fb:.0f}, write {wb:.0f}; {n} dispatches)"]
    return "\n".join(out)


def main(argv):
    if len(argv) >= 2 and argv[0] == "stats":
        print(stats(argv[1], int(argv[2]) if len(argv) > 2 else 20))
    elif len(argv) >= 2 and argv[0] == "grids":
        print(grids(argv[1], argv[2] if len(argv) > 2 else ""))
    elif len(argv) >= 3 and argv[0] == "pmc":
        print(pmc(argv[1], argv[2], int(argv[3]) if len(argv) > 3 else 1024))
    else:
        raise SystemExit(__doc__)


if __name__ == "__main__":
    main(sys.argv[1:])
