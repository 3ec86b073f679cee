#!/usr/bin/env python3
"""Summaries of rocprofv3 output for the chained-MTP round.

  rounds <run_results.db> [marker]
      Per-round kernel breakdown of a --kernel-trace run (rocpd SQLite output): the dispatches after
      one marker kernel (default k_accept, the last kernel of a speculative round) up to and
      including the next; the median-span round of the second half of the trace is printed.
  prefill <run_results.db>
      Per-kernel totals of the last prompt ingest in a --kernel-trace run of
      `bench.py --prefill-only` (the dispatches after the next-to-last k_argmax_final, which ends
      an ingest, up to the last one).
  counters <dir> [<dir> ...]
      Mean per dispatch of every counter of every kernel in --pmc output directories.
  traffic <fetch_dir> <write_dir> <kernel-substring> <copy_bytes> <out.json>
      HBM bytes per launch of one kernel from two --pmc passes (FETCH_SIZE, then WRITE_SIZE, KiB
      per dispatch), each scaled by the same counter's reading for the calibration copy kernel
      (k_stream_copy, which moves copy_bytes in and copy_bytes out per launch).
"""
import collections
import csv
import glob
import json
import os
import sqlite3
import sys


def rounds(db, marker="k_accept"):
    c = sqlite3.connect(db)
    rows = c.execute("select name, start, end from kernels order by start").fetchall()
    idx = [i for i, r in enumerate(rows) if marker in r[0]]
    print(f"{marker} dispatches: {len(idx)}")
    spans = []
    for a, b in zip(idx[:-1], idx[1:]):
        seg = rows[a + 1:b + 1]
        spans.append((seg[-1][2] - seg[0][1], a, b))
    late = sorted(spans[len(spans) // 2:])
    _, a, b = late[len(late) // 2]
    seg = rows[a + 1:b + 1]
    span = (seg[-1][2] - seg[0][1]) / 1e3
    busy = sum(r[2] - r[1] for r in seg) / 1e3
    agg = collections.OrderedDict()
    for n, s, e in seg:
        t = agg.setdefault(n, [0, 0.0])
        t[0] += 1
        t[1] += (e - s) / 1e3
    print(f"round: {len(seg)} kernels, span {span:.1f} us, busy {busy:.1f} us, gaps {span - busy:.1f} us")
    for n, (k, t) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        print(f"{t:10.1f} us {k:5d} x {t / k:8.2f} us  {n[:100]}")


def prefill(db):
    c = sqlite3.connect(db)
    rows = c.execute("select name, start, end from kernels order by start").fetchall()
    idx = [i for i, r in enumerate(rows) if "k_argmax_final" in r[0]]
    seg = rows[idx[-2] + 1:idx[-1] + 1] if len(idx) >= 2 else rows
    agg = collections.OrderedDict()
    for n, s, e in seg:
        t = agg.setdefault(n.split("(")[0], [0, 0.0])
        t[0] += 1
        t[1] += (e - s) / 1e3
    busy = sum(t for _, t in agg.values())
    span = (seg[-1][2] - seg[0][1]) / 1e3
    print(f"ingest: {len(seg)} kernels, span {span / 1e3:.2f} ms, busy {busy / 1e3:.2f} ms")
    for n, (k, t) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        print(f"{t / 1e3:9.2f} ms {100 * t / busy:5.1f}% {k:5d} x {t / k:9.1f} us  {n[:80]}")


def counters(dirs):
    out = collections.OrderedDict()
    for d in dirs:
        for n, cn, v in _counter_rows(d):
            out.setdefault(n.split("(")[0], collections.OrderedDict()).setdefault(cn, []).append(v)
    for n, cs in out.items():
        print(n[:80])
        for cn, v in cs.items():
            print(f"    {cn:28s} {sum(v) / len(v):16.1f}   ({len(v)} dispatches)")


def _counter_rows(d):
    """(kernel name, counter name, value) of every dispatch in a --pmc output directory."""
    out = []
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                out.append((r["Kernel_Name"], r["Counter_Name"], float(r["Counter_Value"])))
    if out:
        return out
    for f in glob.glob(os.path.join(d, "**", "*.db"), recursive=True):
        c = sqlite3.connect(f)
        tabs = [t[0] for t in c.execute("select name from sqlite_master where type in ('table','view')")]
        if "counters_collection" in tabs:
            for r in c.execute("select kernel_name, counter_name, value from counters_collection"):
                out.append((r[0], r[1], float(r[2])))
    return out


def _mean(rows, kernel, counter):
    v = [x for n, cn, x in rows if kernel in n and cn == counter]
    return (sum(v) / len(v), len(v)) if v else (None, 0)


def traffic(fetch_dir, write_dir, kernel, copy_bytes, out):
    fr, wr = _counter_rows(fetch_dir), _counter_rows(write_dir)
    kf, nkf = _mean(fr, kernel, "FETCH_SIZE")
    cf, ncf = _mean(fr, "k_stream_copy", "FETCH_SIZE")
    kw, nkw = _mean(wr, kernel, "WRITE_SIZE")
    cw, ncw = _mean(wr, "k_stream_copy", "WRITE_SIZE")
    fs = copy_bytes / (cf * 1024.0)
    ws = copy_bytes / (cw * 1024.0)
    res = {"kernel": kernel, "dispatches": {"kernel_fetch": nkf, "kernel_write": nkw, "copy_fetch": ncf,
                                            "copy_write": ncw},
           "fetch_kib": kf, "write_kib": kw, "copy_fetch_kib": cf, "copy_write_kib": cw,
           "fetch_scale": fs, "write_scale": ws,
           "traffic_bytes": round(kf * 1024.0 * fs + kw * 1024.0 * ws)}
    with open(out, "w") as fh:
        json.dump(res, fh, indent=1)
    print(json.dumps(res, indent=1))


if __name__ == "__main__":
    if len(sys.argv) >= 3 and sys.argv[1] == "rounds":
        rounds(sys.argv[2], *(sys.argv[3:4]))
    elif len(sys.argv) == 3 and sys.argv[1] == "prefill":
        prefill(sys.argv[2])
    elif len(sys.argv) >= 3 and sys.argv[1] == "counters":
        counters(sys.argv[2:])
    elif len(sys.argv) == 7 and sys.argv[1] == "traffic":
        traffic(sys.argv[2], sys.argv[3], sys.argv[4], int(sys.argv[5]), sys.argv[6])
    else:
        print(__doc__)
        sys.exit(2)
