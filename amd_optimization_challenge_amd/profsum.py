"""Summaries of rocprofv3 CSV output for this operator's profiles.

    python -m amd_optimization_challenge_amd.profsum trace  <p_kernel_trace.csv> [--timed K] [--replays R]
    python -m amd_optimization_challenge_amd.profsum pmc    <fetch counter_collection.csv> <write counter_collection.csv>
    python -m amd_optimization_challenge_amd.profsum sq     <counter_collection.csv> [--match NAME]
    python -m amd_optimization_challenge_amd.profsum calls  <p_kernel_trace.csv>

trace: per-kernel calls / total / mean / min / max, then every run of at
least K back-to-back launches of one decode kernel (name and grid): split
its last R K launches into R blocks of K (the bench's timed graph replays),
the median over the blocks of their mean kernel duration and of their launch
period (first start to last end over K, which is what one event pair around
a replay measures: the kernel plus the boundary to the next one); these are
the bench's decode-only runs over rotating cache copies.  The other decode
launches (inside whole calls) are averaged per kernel.

pmc: FETCH_SIZE and WRITE_SIZE (KiB per dispatch) of every run of decode
launches separated only by the flush fill (a set-up kernel starts a new run),
scaled by what the counters read for the 256 MiB calibration copy
(``__amd_rocclr_copyBuffer``, 262144 KiB read and written), and the traffic
in bytes per launch of each run as ``traffic.launchN=`` lines (runs in launch
order).

sq: mean of every SQ_ counter per run, as for pmc (``--match S``: the
kernels whose name contains S instead of the decode kernels).

calls: every whole operator call in the trace (a run of the operator's own
kernels with one decode launch, ending with the combine, that follows some
other kernel, such as the flush fill), grouped by its kernels and grids: per position the
median and minimum duration and the median gap from the previous kernel's
end, and the median span from the first start to the last end.

Reads only the CSV files rocprofv3 writes (``--output-format csv``).
"""
from __future__ import annotations

import argparse
import collections
import csv
import statistics
import sys

DECODE = ("decode_h16_kernel", "decode_h128_kernel")
CALIB = "__amd_rocclr_copyBuffer"
CALIB_KIB = 262144.0


def short(name: str) -> str:
    n = name.replace("void ", "").replace("mla::(anonymous namespace)::", "").replace("mla::", "")
    return n.split("(mla::DecodeParams)")[0].split("(")[0] if "DecodeParams" in n else n[:80]


def read_trace(path):
    with open(path, newline="") as f:
        rows = list(csv.DictReader(f))
    out = []
    for r in rows:
        out.append(dict(name=r["Kernel_Name"], grid=int(r["Grid_Size_X"]), start=int(r["Start_Timestamp"]),
                        end=int(r["End_Timestamp"])))
    out.sort(key=lambda r: r["start"])
    return out


def trace_summary(path, timed, replays=1):
    ks = read_trace(path)
    agg = collections.OrderedDict()
    for k in ks:
        a = agg.setdefault(short(k["name"]), [])
        a.append(k["end"] - k["start"])
    total = sum(sum(v) for v in agg.values())
    lines = ["| kernel | calls | total us | avg us | min us | max us | % |", "|---|---|---|---|---|---|---|"]
    for name, d in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| `{name}` | {len(d)} | {sum(d) / 1e3:.1f} | {sum(d) / len(d) / 1e3:.2f} | {min(d) / 1e3:.2f} | "
                     f"{max(d) / 1e3:.2f} | {100 * sum(d) / total:.2f} |")
    lines += ["", f"Decode kernels: each run of at least {timed} back-to-back launches (decode only; the median "
                  f"over its last {replays} blocks of {timed} of their means), then the launches inside whole calls "
                  f"per kernel.", "",
              "| # | kernel | grid (threads) | run length | kernel avg us | launch period us |", "|---|---|---|---|---|---|"]
    runs, incall, cur = [], collections.OrderedDict(), None
    for k in ks:
        key = (short(k["name"]), k["grid"]) if any(d in k["name"] for d in DECODE) else None
        if key is not None and cur is not None and cur[0] == key:
            cur[1].append(k)
        else:
            if cur is not None:
                runs.append(cur)
            cur = [key, [k]] if key is not None else None
    if cur is not None:
        runs.append(cur)
    n = 0
    for key, r in runs:
        if len(r) >= timed:
            n += 1
            nb = max(1, min(replays, len(r) // timed))
            durs, periods = [], []
            for j in range(nb):
                t = r[len(r) - (nb - j) * timed:len(r) - (nb - j - 1) * timed]
                durs.append(sum(k["end"] - k["start"] for k in t) / len(t))
                periods.append((t[-1]["end"] - t[0]["start"]) / len(t))  # what one event pair around a replay measures
            dur, period = statistics.median(durs), statistics.median(periods)
            lines.append(f"| {n} | `{key[0]}` | {key[1]} | {len(r)} | {dur / 1e3:.2f} | {period / 1e3:.2f} |")
        else:
            incall.setdefault(key, []).extend(k["end"] - k["start"] for k in r)
    lines += ["", "| kernel | grid (threads) | in-call launches | avg us |", "|---|---|---|---|"]
    for key, ds in incall.items():
        lines.append(f"| `{key[0]}` | {key[1]} | {len(ds)} | {sum(ds) / len(ds) / 1e3:.2f} |")
    return "\n".join(lines)


def read_counters(path):
    """[(dispatch id, kernel name, grid, {counter: value})] in dispatch order."""
    by = collections.OrderedDict()
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            d = int(r["Dispatch_Id"])
            e = by.setdefault(d, [r["Kernel_Name"], int(r["Grid_Size"]), {}])
            e[2][r["Counter_Name"]] = e[2].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return [(d, n, g, c) for d, (n, g, c) in sorted(by.items())]


def per_decode(rows, counter, match=DECODE):
    """[(key, [values])]: runs of one kernel named by `match` (decode kernels
    by default; name, grid) whose launches are separated by nothing but the
    flush fill; any other kernel (set-up, re-layout) starts a new run."""
    groups, last, broken = [], None, True
    for _, n, g, c in rows:
        if not any(d in n for d in match):
            if "FillFunctor" not in n:
                broken = True
            continue
        if counter not in c:
            continue
        key = (short(n), g)
        if broken or key != last:
            groups.append((key, []))
        groups[-1][1].append(c[counter])
        last, broken = key, False
    return groups


def calib(rows, counter):
    v = [c[counter] for _, n, _, c in rows if CALIB in n and counter in c]
    if not v:
        raise SystemExit(f"no {CALIB} dispatch with {counter} in the profile")
    return CALIB_KIB / max(v)


def pmc_summary(fetch_path, write_path):
    fr, wr = read_counters(fetch_path), read_counters(write_path)
    ff, fw = calib(fr, "FETCH_SIZE"), calib(wr, "WRITE_SIZE")
    gf = per_decode(fr, "FETCH_SIZE")
    gw = per_decode(wr, "WRITE_SIZE")
    if [k for k, _ in gf] != [k for k, _ in gw]:
        raise SystemExit("the two passes launched different decode kernels")
    lines = [f"Calibration: FETCH_SIZE x {ff:.3f}, WRITE_SIZE x {fw:.3f} (the 256 MiB copy reads {CALIB_KIB / ff:.0f} "
             f"and writes {CALIB_KIB / fw:.0f} KiB).", "",
             "| # | kernel | grid | launches | FETCH_SIZE KiB | WRITE_SIZE KiB | read MB (scaled) | write MB (scaled) | "
             "traffic MB |", "|---|---|---|---|---|---|---|---|---|"]
    traffic = []
    for i, ((key, vf), (_, vw)) in enumerate(zip(gf, gw), 1):
        f = sum(vf) / len(vf)
        w = sum(vw) / len(vw)
        rd, wb = f * 1024 * ff, w * 1024 * fw
        traffic.append(int(round(rd + wb)))
        lines.append(f"| {i} | `{key[0]}` | {key[1]} | {len(vf)} | {f:.0f} | {w:.0f} | {rd / 1e6:.1f} | "
                     f"{wb / 1e6:.1f} | {(rd + wb) / 1e6:.1f} |")
    lines += ["", "```"] + [f"traffic.launch{i}={t}" for i, t in enumerate(traffic, 1)] + ["```"]
    return "\n".join(lines)


def sq_summary(path, match=DECODE):
    rows = read_counters(path)
    names = []
    for _, n, g, c in rows:
        for k in c:
            if k.startswith("SQ_") and k not in names:
                names.append(k)
    groups = per_decode(rows, names[0], match) if names else []
    per = collections.defaultdict(list)  # run index -> counters of its launches
    i, last, broken = -1, None, True
    for _, n, g, c in rows:
        if not any(d in n for d in match):
            if "FillFunctor" not in n:
                broken = True
            continue
        key = (short(n), g)
        if broken or key != last:
            i += 1
        per[i].append(c)
        last, broken = key, False
    lines = ["| # | kernel | grid | " + " | ".join(names) + " |", "|---|---|---|" + "---|" * len(names)]
    for j, (key, _) in enumerate(groups):
        cells = []
        for k in names:
            v = [c[k] for c in per[j] if k in c]
            cells.append(f"{sum(v) / len(v):.0f}" if v else "-")
        lines.append(f"| {j + 1} | `{key[0]}` | {key[1]} | " + " | ".join(cells) + " |")
    return "\n".join(lines)


OPERATOR = ("amax_kernel", "quant_fp8_kernel", "plan_kernel") + DECODE + ("combine_kernel",)


def calls_summary(path):
    ks = read_trace(path)
    calls, cur = [], []
    for k in ks:
        if any(o in k["name"] for o in OPERATOR):
            cur.append(k)
            if "combine_kernel" in k["name"]:
                # a whole call holds one decode launch (the bench's decode-only
                # graphs, many decodes back to back, are not calls)
                if sum(any(d in x["name"] for d in DECODE) for x in cur) == 1:
                    calls.append(cur)
                cur = []
        else:
            cur = []
    groups = collections.OrderedDict()
    for c in calls:
        groups.setdefault(tuple((short(k["name"]), k["grid"]) for k in c), []).append(c)
    lines = []
    for sig, cs in groups.items():
        lines += [f"{len(cs)} calls", "", "| # | kernel | grid (threads) | median us | min us | gap before, median us |",
                  "|---|---|---|---|---|---|"]
        for i, (name, grid) in enumerate(sig):
            d = [(c[i]["end"] - c[i]["start"]) / 1e3 for c in cs]
            gap = f"{statistics.median((c[i]['start'] - c[i - 1]['end']) / 1e3 for c in cs):.2f}" if i else "-"
            lines.append(f"| {i + 1} | `{name}` | {grid} | {statistics.median(d):.2f} | {min(d):.2f} | {gap} |")
        span = [(c[-1]["end"] - c[0]["start"]) / 1e3 for c in cs]
        lines += ["", f"first start to last end: median {statistics.median(span):.2f} us, min {min(span):.2f} us", ""]
    return "\n".join(lines).rstrip()


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("csv")
    t.add_argument("--timed", type=int, default=20)
    t.add_argument("--replays", type=int, default=1, help="timed replays of K launches at the end of each run")
    p = sub.add_parser("pmc")
    p.add_argument("fetch_csv")
    p.add_argument("write_csv")
    s = sub.add_parser("sq")
    s.add_argument("csv")
    s.add_argument("--match", default=None, help="kernel-name substring (default: the decode kernels)")
    c = sub.add_parser("calls")
    c.add_argument("csv")
    a = ap.parse_args(argv)
    if a.cmd == "trace":
        print(trace_summary(a.csv, a.timed, a.replays))
    elif a.cmd == "pmc":
        print(pmc_summary(a.fetch_csv, a.write_csv))
    elif a.cmd == "calls":
        print(calls_summary(a.csv))
    else:
        print(sq_summary(a.csv, (a.match,) if a.match else DECODE))
    return 0


if __name__ == "__main__":
    sys.exit(main())
