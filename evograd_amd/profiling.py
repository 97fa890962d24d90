"""Summaries of rocprofv3 CSV output (``--output-format csv``) as short markdown.

    python -m evograd_amd.profiling stats    <prefix>_kernel_stats.csv [FILTER]
    python -m evograd_amd.profiling counters <prefix>_counter_collection.csv [FILTER]
    python -m evograd_amd.profiling traffic  FETCH.csv WRITE.csv KERNEL_SUBSTRING [KEY]
    python -m evograd_amd.profiling mfma     COUNTERS.csv KERNEL_STATS.csv [FILTER] [GHZ]
    python -m evograd_amd.profiling clock    COUNTERS.csv [FILTER]

``traffic`` turns the FETCH_SIZE and WRITE_SIZE readings (KiB per dispatch,
summed over the L2 channels) of one kernel into HBM bytes per launch, scaled by
what the same counters read for the calibration copy that ``bench.py --profile``
runs (a torch elementwise multiply reading and writing 256 MiB each), and prints
the JSON entry recorded in profiles/traffic.json.
"""

from __future__ import annotations

import collections
import csv
import json
import re
import statistics
import sys

COPY_KERNEL = "MulFunctor<float>"
COPY_BYTES = 256 << 20
COPY_GRID = COPY_BYTES // 16  # threads of the calibration copy: 4 floats per thread


def short_name(name: str) -> str:
    """Kernel name without namespaces, argument lists and most template noise."""
    n = re.sub(r"^void\s+", "", name)
    n = n.replace("(anonymous namespace)::", "")
    depth, out = 0, []
    for ch in n:  # drop the argument list: everything from the first '(' at depth 0
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            break
        out.append(ch)
    n = "".join(out)
    n = n.replace("at::native::", "at::")
    n = n.replace("eg::bf16_t", "bf16").replace("eg::f16_t", "f16")
    return n[:110]


def stats(path: str, filt: str = "") -> str:
    rows = list(csv.DictReader(open(path)))
    lines = ["| kernel | calls | avg us | min us | max us | share % |", "|---|---:|---:|---:|---:|---:|"]
    for r in rows:
        if filt and filt not in r["Name"]:
            continue
        lines.append(
            f"| `{short_name(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
            f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.1f} |"
        )
    return "\n".join(lines)


def _counter_table(path: str, grid: int = 0):
    """kernel name -> counter -> list of per-dispatch values (only dispatches of
    `grid` threads when it is given)."""
    per = collections.defaultdict(lambda: collections.defaultdict(dict))
    for r in csv.DictReader(open(path)):
        if grid and int(r["Grid_Size"]) != grid:
            continue
        per[r["Kernel_Name"]][r["Counter_Name"]][r["Dispatch_Id"]] = (
            per[r["Kernel_Name"]][r["Counter_Name"]].get(r["Dispatch_Id"], 0.0)
            + float(r["Counter_Value"])
        )
    return {k: {c: list(d.values()) for c, d in cs.items()} for k, cs in per.items()}


def counters(path: str, filt: str = "") -> str:
    table = _counter_table(path)
    lines = ["| kernel | counter | dispatches | mean per dispatch |", "|---|---|---:|---:|"]
    for k, cs in table.items():
        if filt and filt not in k:
            continue
        for c, vals in sorted(cs.items()):
            lines.append(f"| `{short_name(k)}` | {c} | {len(vals)} | {statistics.mean(vals):.6g} |")
    return "\n".join(lines)


def mfma(counter_csv: str, stats_csv: str, filt: str = "", ghz: float = 2.4) -> str:
    """MFMA utilisation per kernel: SQ_VALU_MFMA_BUSY_CYCLES (summed over all
    SIMDs; a 32x32x16 bf16 MFMA keeps its SIMD busy 32 cycles) divided by the
    kernel's mean duration (kernel trace) x clock x 1024 SIMDs (256 CUs x 4), and
    the executed MFMA FLOPs (SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512)."""
    table = _counter_table(counter_csv)
    dur = {}
    for r in csv.DictReader(open(stats_csv)):
        dur[short_name(r["Name"])] = float(r["AverageNs"]) * 1e-9
    lines = ["| kernel | mean us (trace) | MFMA busy % | executed MFMA TFLOP | executed TFLOP/s |",
             "|---|---:|---:|---:|---:|"]
    for k, cs in table.items():
        if filt and filt not in k:
            continue
        name = short_name(k)
        t = dur.get(name)
        busy = cs.get("SQ_VALU_MFMA_BUSY_CYCLES")
        mops = cs.get("SQ_INSTS_VALU_MFMA_MOPS_BF16")
        if t is None or not busy:
            continue
        util = statistics.mean(busy) / (t * ghz * 1e9 * 1024)
        flops = statistics.mean(mops) * 512 if mops else float("nan")
        lines.append(f"| `{name}` | {t * 1e6:.1f} | {100 * util:.1f} | {flops / 1e12:.3f} | "
                     f"{flops / t / 1e12:.1f} |")
    return "\n".join(lines)


def clock(counter_csv: str, filt: str = "", shader_engines: int = 32, simds: int = 1024,
          nominal_ghz: float = 2.4) -> str:
    """Effective engine clock and MFMA busy share per kernel, from one counter run
    holding SQ_BUSY_CYCLES and SQ_VALU_MFMA_BUSY_CYCLES. SQ_BUSY_CYCLES is summed
    over the shader engines (32 on an MI355X: the agent's Num_Shader_Banks), so
    busy / engines / dispatch duration is the clock the kernel ran at;
    SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x those cycles) is the share of cycles the
    matrix cores were busy. A fraction of the published peak is the product of the
    two: busy share x clock / nominal clock. Durations are the counter rows'
    dispatch timestamps; the median over a kernel's dispatches is reported."""
    per = collections.defaultdict(lambda: collections.defaultdict(dict))
    span = {}
    for r in csv.DictReader(open(counter_csv)):
        k, d = r["Kernel_Name"], r["Dispatch_Id"]
        cs = per[k][d]
        cs[r["Counter_Name"]] = cs.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        span[(k, d)] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9
    lines = ["| kernel | dispatches | median us | clock GHz | MFMA busy % of cycles | "
             f"fraction of peak at {nominal_ghz} GHz |", "|---|---:|---:|---:|---:|---:|"]
    for k, ds in per.items():
        if filt and filt not in k:
            continue
        rows = []
        for d, cs in ds.items():
            t = span[(k, d)]
            busy, mfma = cs.get("SQ_BUSY_CYCLES"), cs.get("SQ_VALU_MFMA_BUSY_CYCLES")
            if not busy or t <= 0:
                continue
            cyc = busy / shader_engines
            share = (mfma or 0.0) / (simds * cyc)
            rows.append((t, cyc / t / 1e9, share))
        if not rows:
            continue
        t = statistics.median(r[0] for r in rows)
        ghz = statistics.median(r[1] for r in rows)
        share = statistics.median(r[2] for r in rows)
        lines.append(f"| `{short_name(k)}` | {len(rows)} | {t * 1e6:.1f} | {ghz:.3f} | "
                     f"{100 * share:.1f} | {100 * share * ghz / nominal_ghz:.1f}% |")
    return "\n".join(lines)


def traffic(fetch_csv: str, write_csv: str, kernel: str, key: str = "") -> dict:
    f, w = _counter_table(fetch_csv), _counter_table(write_csv)

    def pick(table, sub, counter, how=statistics.median):
        vals = [v for k, cs in table.items() if sub in k for v in cs.get(counter, [])]
        if not vals:
            raise SystemExit(f"no {counter} readings for kernels matching {sub!r}")
        return how(vals)

    # the calibration copy is told from other kernels of its kind (an input recipe
    # may scale its tensors with the same kernel, smaller or larger) by its grid:
    # torch's vectorized float kernel runs one thread per 4 elements
    cf, cw = _counter_table(fetch_csv, COPY_GRID), _counter_table(write_csv, COPY_GRID)
    copy_fetch_kib = pick(cf, COPY_KERNEL, "FETCH_SIZE")
    copy_write_kib = pick(cw, COPY_KERNEL, "WRITE_SIZE")
    fetch_scale = COPY_BYTES / (copy_fetch_kib * 1024.0)
    write_scale = COPY_BYTES / (copy_write_kib * 1024.0)
    kf = pick(f, kernel, "FETCH_SIZE") * 1024.0 * fetch_scale
    kw = pick(w, kernel, "WRITE_SIZE") * 1024.0 * write_scale
    return {
        "kernel": kernel,
        "key": key or kernel,
        "fetch_bytes_per_launch": round(kf),
        "write_bytes_per_launch": round(kw),
        "hbm_bytes_per_launch": round(kf + kw),
        "copy_calibration": {
            "bytes_each_way": COPY_BYTES,
            "fetch_kib_read": copy_fetch_kib,
            "write_kib_read": copy_write_kib,
            "fetch_scale": fetch_scale,
            "write_scale": write_scale,
        },
    }


def main(argv: list) -> int:
    if len(argv) < 2:
        print(__doc__)
        return 2
    cmd = argv[0]
    if cmd == "stats":
        print(stats(argv[1], argv[2] if len(argv) > 2 else ""))
    elif cmd == "counters":
        print(counters(argv[1], argv[2] if len(argv) > 2 else ""))
    elif cmd == "mfma":
        print(mfma(argv[1], argv[2], argv[3] if len(argv) > 3 else "",
                   float(argv[4]) if len(argv) > 4 else 2.4))
    elif cmd == "clock":
        print(clock(argv[1], argv[2] if len(argv) > 2 else ""))
    elif cmd == "traffic":
        print(json.dumps(traffic(argv[1], argv[2], argv[3], argv[4] if len(argv) > 4 else ""), indent=1))
    else:
        print(__doc__)
        return 2
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
