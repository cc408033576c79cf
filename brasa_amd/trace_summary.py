"""Per-kernel duration summary of a rocprofv3 kernel trace, cold dispatches left out.

    python -m brasa_amd.trace_summary DIR [--skip N] [--match SUBSTR] [--bytes B | --flop F]
    python -m brasa_amd.trace_summary DIR --counters [--match SUBSTR]

DIR is the output directory of ``rocprofv3 --kernel-trace -d DIR`` (its SQLite database, table
``kernels``, one row per dispatch in dispatch order). For every kernel whose name contains SUBSTR
(all kernels by default) the first N dispatches are dropped -- ``bench.py --profile decode*``
runs one cold step of 36 launches before the warm ones -- and the rest are summarised as a
markdown table: calls, average, median, min and max duration in microseconds. With --bytes or
--flop the average and median are also turned into GB/s or TFLOP/s per call. With --counters
DIR is a ``rocprofv3 --pmc`` run instead: every counter's value per dispatch (summed over the
dispatch's instances), averaged over the matching kernels' dispatches.
"""
from __future__ import annotations

import argparse
import collections
import glob
import re
import sqlite3
import statistics


def short(name: str) -> str:
    name = name.replace("brasa::(anonymous namespace)::", "brasa::").replace("void ", "")
    return re.sub(r"\(.*", "", name)


def durations(directory: str) -> "collections.OrderedDict[str, list[float]]":
    dbs = glob.glob(directory + "/**/*.db", recursive=True)
    if not dbs:
        raise SystemExit(f"no rocprofv3 database under {directory}")
    con = sqlite3.connect(dbs[0])
    by: collections.OrderedDict[str, list[float]] = collections.OrderedDict()
    for name, dur in con.execute("select name, duration from kernels"):
        by.setdefault(short(name), []).append(dur / 1000.0)
    return by


def summary(directory: str, skip: int = 0, match: str = "", nbytes: float = 0.0,
            flop: float = 0.0) -> str:
    out = ["| kernel | calls | avg µs | median µs | min µs | max µs |" +
           (" avg GB/s | median GB/s |" if nbytes else "") +
           (" avg TFLOP/s | median TFLOP/s |" if flop else ""),
           "|---|---|---|---|---|---|" + ("---|---|" if nbytes or flop else "")]
    for name, v in durations(directory).items():
        if match and match not in name:
            continue
        w = v[skip:] if len(v) > skip else v
        avg, med = statistics.mean(w), statistics.median(w)
        row = f"| `{name}` | {len(w)} | {avg:.2f} | {med:.2f} | {min(w):.2f} | {max(w):.2f} |"
        if nbytes:
            row += f" {nbytes / avg / 1e3:.0f} | {nbytes / med / 1e3:.0f} |"
        if flop:
            row += f" {flop / avg / 1e6:.0f} | {flop / med / 1e6:.0f} |"
        out.append(row)
    return "\n".join(out)


def counters(directory: str, match: str = "") -> str:
    dbs = glob.glob(directory + "/**/*.db", recursive=True)
    if not dbs:
        raise SystemExit(f"no rocprofv3 database under {directory}")
    con = sqlite3.connect(dbs[0])
    rows = con.execute("select dispatch_id, name, counter_name, sum(counter_value) from pmc_events "
                       "group by dispatch_id, counter_name").fetchall()
    by: dict[tuple[str, str], list[float]] = collections.defaultdict(list)
    for _, name, counter, value in rows:
        if match and match not in short(name):
            continue
        by[(short(name), counter)].append(value)
    out = ["| kernel | counter | dispatches | average per dispatch |", "|---|---|---|---|"]
    for (name, counter), v in sorted(by.items()):
        out.append(f"| `{name}` | {counter} | {len(v)} | {statistics.mean(v):,.0f} |")
    return "\n".join(out)


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("dir")
    ap.add_argument("--skip", type=int, default=0, help="cold dispatches dropped per kernel")
    ap.add_argument("--match", default="", help="only kernels whose name contains this")
    ap.add_argument("--bytes", type=float, default=0.0, help="algorithmic bytes per call")
    ap.add_argument("--flop", type=float, default=0.0, help="algorithmic flop per call")
    ap.add_argument("--counters", action="store_true", help="a --pmc run: counter averages")
    a = ap.parse_args()
    if a.counters:
        print(counters(a.dir, a.match))
    else:
        print(summary(a.dir, a.skip, a.match, a.bytes, a.flop))


if __name__ == "__main__":
    main()
