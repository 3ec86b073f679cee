#!/usr/bin/env python3
"""Per-round kernel breakdown of a rocprofv3 trace (rocpd SQLite output).

usage: python q27x_profile.py <run_results.db> [marker-kernel-substring]

A round is the dispatches after one marker kernel (default k_accept, the last kernel of a
speculative round) up to and including the next; the median-span round of the second half of the
trace is printed with per-kernel totals, counts and averages."""
import sqlite3, sys, collections
db = sys.argv[1]; marker = sys.argv[2] if len(sys.argv) > 2 else 'k_accept'
c = sqlite3.connect(db)
rows = c.execute("select name, start, end from kernels order by start").fetchall()
idx = [i for i, r in enumerate(rows) if marker in r[0]]
print(f"{marker} dispatches: {len(idx)}")
# steady-state rounds: pairs of consecutive markers, take the median-span one among the later half
spans = []
for a, b in zip(idx[:-1], idx[1:]):
    seg = rows[a + 1:b + 1]
    spans.append((seg[-1][2] - seg[0][1], a, b))
mid = sorted(spans[len(spans)//2:])[len(spans[len(spans)//2:])//2]
_, a, b = mid
seg = rows[a + 1:b + 1]
span = (seg[-1][2] - seg[0][1]) / 1e3
busy = sum(r[2] - r[1] for r in seg) / 1e3
agg = collections.OrderedDict()
for n, s, e in seg:
    t = agg.setdefault(n, [0, 0.0]); t[0] += 1; t[1] += (e - s) / 1e3
print(f"round: {len(seg)} kernels, span {span:.1f} us, busy {busy:.1f} us, gaps {span-busy:.1f} us")
for n, (k, t) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
    print(f"{t:10.1f} us {k:5d} x {t/k:8.2f} us  {n[:100]}")
