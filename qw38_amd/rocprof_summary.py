"""Summarise a rocprofv3 SQLite output (``*_results.db``) as short text.

    python -m qw38_amd.rocprof_summary <results.db> [--match SUBSTR] [--top N]

Prints, per kernel instantiation and grid size: dispatch count and average /
min / max duration (us), and,
when the run collected ``--pmc`` counters, the per-dispatch average of every
counter; with ``--marker-trace``, the host-side duration of every roctx range
name. Used to turn rocprofv3 runs into the text summaries under profiles/.
"""
from __future__ import annotations

import argparse
import collections
import json
import re
import sqlite3
import sys


def _short(name: str) -> str:
    """Kernel base name with its template arguments (balanced <...>), without
    namespaces and the parameter list."""
    name = re.sub(r"\s+", " ", name)
    m2 = re.search(r"qw38hip::(?:\(anonymous namespace\)::)?(\w+)", name)
    if not m2:
        return name[:120]
    base, i = m2.group(1), m2.end()
    if i < len(name) and name[i] == "<":
        depth, j = 0, i
        while j < len(name):
            depth += name[j] == "<"
            depth -= name[j] == ">"
            j += 1
            if depth == 0:
                break
        base += name[i:j]
    return base[:140]


def summarize(path: str, match: str | None = None, top: int = 12) -> str:
    db = sqlite3.connect(path)
    names = [r[0] for r in db.execute("select name from sqlite_master where type in ('table','view')")]
    out = []
    # kernel durations
    # one line per (kernel instantiation, grid): shapes launched with the same
    # kernel stay apart
    kcols = [r[1] for r in db.execute("pragma table_info(kernels)")]
    has_grid = "grid_x" in kcols and "workgroup_x" in kcols
    q = "select id, name, start, end" + (", grid_x, workgroup_x" if has_grid else "") + " from kernels"
    by = collections.defaultdict(list)
    for row in db.execute(q).fetchall():
        kid, name, s, e = row[:4]
        if match and match not in name:
            continue
        blocks = (row[4] // max(row[5], 1)) if has_grid else 0
        by[(name, blocks)].append((e - s) / 1e3)
    tot = sum(sum(v) for v in by.values()) or 1.0
    out.append(f"{'kernel':<72} {'blocks':>7} {'calls':>6} {'avg_us':>9} {'min_us':>9} {'max_us':>9} {'time%':>6}")
    for (name, blocks), v in sorted(by.items(), key=lambda kv: -sum(kv[1]))[:top]:
        out.append(f"{_short(name):<72} {blocks:>7} {len(v):>6} {sum(v)/len(v):>9.3f} {min(v):>9.3f} "
                   f"{max(v):>9.3f} {100*sum(v)/tot:>6.1f}")
    # counters, when present: keyed by (kernel instantiation, grid) exactly
    # like the timing rows above and printed in the same order, so two grids of
    # one kernel can never swap their counter lines
    if "counters_collection" in names:
        cols = [r[1] for r in db.execute("pragma table_info(counters_collection)")]
        vcol = "value" if "value" in cols else "counter_value"
        ncol = "counter_name" if "counter_name" in cols else "name"
        grid = None
        if "grid_size" in cols and "workgroup_size" in cols:
            grid = "grid_size / max(workgroup_size, 1)"
        elif "grid_size_x" in cols and "workgroup_size_x" in cols:
            grid = "grid_size_x / max(workgroup_size_x, 1)"
        if "kernel_name" in cols and grid is not None:
            q = (f"select kernel_name, blocks, {ncol}, avg(v), count(*) from ("
                 f"select kernel_name, {grid} as blocks, {ncol}, dispatch_id, sum({vcol}) as v "
                 f"from counters_collection group by kernel_name, blocks, {ncol}, dispatch_id) "
                 f"group by kernel_name, blocks, {ncol}")
            agg = collections.defaultdict(dict)
            for kname, blocks, cname, avg, cnt in db.execute(q):
                if match and match not in kname:
                    continue
                agg[(kname, int(blocks))][cname] = (avg, cnt)
            order = {key: -sum(v) for key, v in by.items()}
            if agg:
                out.append("")
                out.append("per-dispatch counter averages (kernel, blocks):")
                for key, cs in sorted(agg.items(), key=lambda kv: (order.get(kv[0], 0.0), kv[0][0])):
                    vals = "  ".join(f"{c}={a:.6g}" for c, (a, _) in sorted(cs.items()))
                    n = max(c for _, c in cs.values())
                    out.append(f"  {_short(key[0])} blocks={key[1]} (dispatches={n}): {vals}")
        elif "kernel_name" in cols:
            out.append("")
            out.append("counters present but no grid column: " + ", ".join(cols))
    # roctx ranges (--marker-trace): host-side duration per range name
    if "regions" in names:
        rows = db.execute("select category, name, start, end, extdata from regions "
                          "where upper(category) like '%MARKER%'").fetchall()
        rng = collections.defaultdict(list)
        for cat, name, s, e, ext in rows:
            try:  # the range's message, when the profiler recorded one
                name = json.loads(ext).get("message", name) if ext else name
            except (ValueError, AttributeError):
                pass
            if match and match not in name:
                continue
            rng[name].append((e - s) / 1e3)
        if rng:
            out.append("")
            out.append(f"{'roctx range (host)':<96} {'calls':>6} {'avg_us':>9} {'min_us':>9}")
            for name, v in sorted(rng.items(), key=lambda kv: -sum(kv[1]))[:top]:
                out.append(f"{name[:96]:<96} {len(v):>6} {sum(v)/len(v):>9.3f} {min(v):>9.3f}")
    return "\n".join(out)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("db")
    ap.add_argument("--match")
    ap.add_argument("--top", type=int, default=12)
    ap.add_argument("--schema", action="store_true")
    a = ap.parse_args(argv)
    if a.schema:
        db = sqlite3.connect(a.db)
        for (t,) in db.execute("select name from sqlite_master where type in ('table','view')"):
            cols = [r[1] for r in db.execute(f"pragma table_info('{t}')")]
            print(t, cols)
        return 0
    print(summarize(a.db, a.match, a.top))
    return 0


if __name__ == "__main__":
    sys.exit(main())
