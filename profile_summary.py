"""Reduce rocprofv3 CSV output of a bench.py run to the figures the bench reports.

    python3 profile_summary.py trace  <dir> [--blocks 100,900,300,900] [--idle NAME,FIRST,COUNT]
    python3 profile_summary.py pmc    <dir> [--skip 100 --take 900]
    python3 profile_summary.py traffic <fetch dir> <write dir> \
        <copy fetch dir> <copy write dir> [--skip 100 --take 900]

``trace`` reads ``*_kernel_stats.csv`` / ``*_kernel_trace.csv`` of a
``--kernel-trace --stats -f csv`` run and prints per-kernel durations, plus the
mean of consecutive dispatch blocks of each kernel (bench.py issues its
matching-kernel launches as warm-up W, timed K, latency replay, event replay).
With ``--idle`` it also reports how much of the time from dispatch FIRST to
dispatch FIRST + COUNT - 1 of the kernel whose name starts with NAME no kernel
was running (the gaps between back-to-back launches), per dispatch.
``pmc`` prints per-dispatch means of every counter in ``*_counter_collection.csv``.
``traffic`` turns FETCH_SIZE and WRITE_SIZE (KiB per dispatch) into HBM bytes per
launch, each scaled by what the same counter reads for bench.py's
``--copy-calibration`` run (a 1 GiB device copy): bytes = KiB * 1024 * (2^30 /
copy KiB * 1024). Output is markdown on stdout. Means are over dispatches
[skip, skip + take) of each kernel; with ``bench.py --phases A`` the matching
kernel's dispatch d is step d, so the window is the bench's ``timed_steps``, and
the ``traffic_bytes_per_launch[kernel][first,end]`` lines that bench.py reads
carry it.
"""
from __future__ import annotations

import argparse
import collections
import csv
import glob
import os
import statistics


def _one(dirpath: str, suffix: str) -> str:
    found = sorted(glob.glob(os.path.join(dirpath, "**", "*" + suffix), recursive=True))
    if not found:
        raise SystemExit(f"no *{suffix} under {dirpath}")
    return found[0]


def _short(name: str) -> str:
    name = name.replace("(anonymous namespace)::", "")
    return name.split("(")[0] if "(" in name else name


def idle(disp: dict, name: str, first: int, count: int) -> str:
    """Idle time on the GPU between the start of dispatch `first` and the end of
    dispatch `first + count - 1` of kernel `name` (dispatches of every kernel in
    between count as busy)."""
    own = sorted(v for k, vs in disp.items() if k.startswith(name) for v in vs)
    if len(own) < first + count:
        return f"(fewer than {first + count} dispatches of {name})"
    t0, t1 = own[first][0], own[first + count - 1][0] + own[first + count - 1][1]
    spans = sorted((s, s + d) for vs in disp.values() for s, d in vs if s < t1 and s + d > t0)
    busy, end = 0, t0
    for s, e in spans:  # union of the kernels' intervals within [t0, t1]
        s, e = max(s, end), min(e, t1)
        if e > s:
            busy += e - s
            end = e
    span = t1 - t0
    return (f"From dispatch {first} to dispatch {first + count - 1} of `{name}`: {span / 1e3:.2f} us, "
            f"of which no kernel ran {(span - busy) / 1e3:.2f} us ({(span - busy) / 1e3 / count:.2f} us "
            f"per dispatch of `{name}`).")


def trace(dirpath: str, blocks: list[int], gaps: str | None = None) -> str:
    out = []
    rows = list(csv.DictReader(open(_one(dirpath, "_kernel_stats.csv"))))
    out.append("| kernel | calls | average us | min us | max us | share |")
    out.append("|---|---|---|---|---|---|")
    for r in rows:
        out.append(f"| `{_short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                   f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
                   f"{float(r['Percentage']):.1f}% |")
    disp = collections.defaultdict(list)
    for r in csv.DictReader(open(_one(dirpath, "_kernel_trace.csv"))):
        disp[_short(r["Kernel_Name"])].append(
            (int(r["Start_Timestamp"]), int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
    out.append("")
    out.append("Mean duration of consecutive dispatch blocks (in launch order), us:")
    out.append("")
    for name, v in disp.items():
        v.sort()
        d = [x[1] / 1e3 for x in v]
        parts, i = [], 0
        for n in blocks:
            if i >= len(d):
                break
            seg = d[i:i + n]
            parts.append(f"[{i}, {i + len(seg)}): {statistics.mean(seg):.2f}")
            i += n
        out.append(f"- `{name}` ({len(d)} dispatches): " + "; ".join(parts))
    if gaps:
        name, first, count = gaps.rsplit(",", 2)
        out += ["", idle(disp, name, int(first), int(count))]
    return "\n".join(out)


def _counters(dirpath: str):
    per = collections.defaultdict(lambda: collections.defaultdict(list))
    for r in csv.DictReader(open(_one(dirpath, "_counter_collection.csv"))):
        per[_short(r["Kernel_Name"])][r["Counter_Name"]].append(
            (int(r["Dispatch_Id"]), float(r["Counter_Value"])))
    res = {}
    for k, cs in per.items():
        res[k] = {c: [x for _, x in sorted(v)] for c, v in cs.items()}
    return res


def _mean(v, skip, take):
    seg = v[skip:skip + take] if len(v) > skip else v
    return statistics.mean(seg) if seg else float("nan")


def pmc(dirpath: str, skip: int, take: int, min_dispatches: int = 100) -> str:
    out = ["| kernel | counter | dispatches | mean per dispatch |", "|---|---|---|---|"]
    for k, cs in _counters(dirpath).items():
        for c, v in sorted(cs.items()):
            if len(v) < min_dispatches:
                continue
            out.append(f"| `{k}` | {c} | {len(v)} | {_mean(v, skip, take):.6g} |")
    return "\n".join(out)


def traffic(fetch: str, write: str, cfetch: str, cwrite: str, skip: int, take: int,
            min_dispatches: int) -> str:
    def copy_kib(d, counter):
        vals = [v for k, cs in _counters(d).items() if "copyBuffer" in k or "copy" in k.lower()
                for c, vs in cs.items() if c == counter for v in vs]
        vals = [v for v in vals if v > 1024]  # the 1 GiB copies, not small set-up kernels
        return statistics.median(vals)

    gib_kib = float(1 << 20)
    f_fac = gib_kib / copy_kib(cfetch, "FETCH_SIZE")
    w_fac = gib_kib / copy_kib(cwrite, "WRITE_SIZE")
    fc, wc = _counters(fetch), _counters(write)
    out = [f"Copy calibration (1 GiB device copy): FETCH_SIZE factor {f_fac:.4f}, "
           f"WRITE_SIZE factor {w_fac:.4f}.", "",
           "| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | read bytes | written bytes | "
           "traffic bytes |",
           "|---|---|---|---|---|---|---|"]
    lines = []
    for k in fc:
        if k not in wc or "FETCH_SIZE" not in fc[k] or "WRITE_SIZE" not in wc[k]:
            continue
        if len(fc[k]["FETCH_SIZE"]) < min_dispatches:
            continue
        f = _mean(fc[k]["FETCH_SIZE"], skip, take)
        w = _mean(wc[k]["WRITE_SIZE"], skip, take)
        rb, wb = f * 1024 * f_fac, w * 1024 * w_fac
        out.append(f"| `{k}` | {len(fc[k]['FETCH_SIZE'])} | {f:.1f} | {w:.1f} | {rb:.4g} | {wb:.4g} | "
                   f"{rb + wb:.4g} |")
        lines.append(f"traffic_bytes_per_launch[{k}][{skip},{skip + take}]: {rb + wb:.0f}")
    return "\n".join(out + [""] + lines)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("dir")
    t.add_argument("--blocks", default="100,900,300,900")
    t.add_argument("--idle", default=None, help="NAME,FIRST,COUNT: idle time between those dispatches")
    p = sub.add_parser("pmc")
    p.add_argument("dir")
    p.add_argument("--skip", type=int, default=100)
    p.add_argument("--take", type=int, default=900)
    p.add_argument("--min-dispatches", type=int, default=100,
                   help="skip kernels launched fewer times (set-up fills)")
    r = sub.add_parser("traffic")
    for n in ("fetch", "write", "copy_fetch", "copy_write"):
        r.add_argument(n)
    r.add_argument("--skip", type=int, default=100)
    r.add_argument("--take", type=int, default=900)
    r.add_argument("--min-dispatches", type=int, default=100,
                   help="skip kernels launched fewer times (set-up fills)")
    a = ap.parse_args()
    if a.cmd == "trace":
        print(trace(a.dir, [int(x) for x in a.blocks.split(",")], a.idle))
    elif a.cmd == "pmc":
        print(pmc(a.dir, a.skip, a.take, a.min_dispatches))
    else:
        print(traffic(a.fetch, a.write, a.copy_fetch, a.copy_write, a.skip, a.take, a.min_dispatches))


if __name__ == "__main__":
    main()
