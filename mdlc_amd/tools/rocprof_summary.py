"""Summarise rocprofv3 SQLite output (``*_results.db``) as text.

    python -m mdlc_amd.tools.rocprof_summary trace.db                 # per-kernel durations
    python -m mdlc_amd.tools.rocprof_summary pmc.db --counter FETCH_SIZE
    python -m mdlc_amd.tools.rocprof_summary --traffic fetch.db write.db \
        copy_fetch.db copy_write.db --copy-mib 256 --out traffic.json
    python -m mdlc_amd.tools.rocprof_summary trace.db --rates traffic.json
    python -m mdlc_amd.tools.rocprof_summary trace.db --per-launch KERNEL 8 \
        --traffic fetch.db write.db copy_fetch.db copy_write.db

The first form lists, per kernel name, the dispatch count, total and average
duration and share of device time (the ``--kernel-trace --stats`` view). The
second lists the average value of one PMC counter per dispatch of each
kernel (``--pmc`` runs). The third turns a FETCH_SIZE run and a WRITE_SIZE
run of a workload, plus the same two counters read for a plain copy of
``--copy-mib`` MiB, into HBM bytes per dispatch for every kernel: each
counter is scaled by (true copy bytes / counter reading for the copy). The
fourth divides those bytes by each kernel's average traced duration (HBM
GB/s against the 8 TB/s peak). ``--counter MfmaUtil`` (a derived counter of
``rocprofv3 --pmc MfmaUtil``) gives the matrix-core busy percentage.
"""

from __future__ import annotations

import argparse
import json
import sqlite3


def kernel_stats(path: str) -> list:
    con = sqlite3.connect(path)
    rows = con.execute(
        "select name, count(*), sum(duration), avg(duration), min(duration), max(duration) "
        "from kernels group by name order by sum(duration) desc").fetchall()
    con.close()
    return rows


def kernel_stats_by_grid(path: str) -> list:
    """Per (kernel name, grid): calls, total, average, median, min, max
    duration — kernels of one name built by separate plans for different
    shapes (the micro GEMMs) are told apart by their grids."""
    con = sqlite3.connect(path)
    by: dict = {}
    for name, gx, gy, gz, d in con.execute(
            "select name, grid_x, grid_y, grid_z, duration from kernels order by dispatch_id"):
        by.setdefault((name, gx, gy, gz), []).append(d)
    con.close()
    rows = []
    for (name, gx, gy, gz), v in by.items():
        w = sorted(v)
        k = len(w)
        med = w[k // 2] if k % 2 else 0.5 * (w[k // 2 - 1] + w[k // 2])
        rows.append((name, (gx, gy, gz), k, sum(v), sum(v) / k, med, w[0], w[-1]))
    return sorted(rows, key=lambda r: -r[3])


def kernel_medians(path: str) -> dict:
    """Median dispatch duration per kernel name."""
    con = sqlite3.connect(path)
    by: dict = {}
    for name, d in con.execute("select name, duration from kernels"):
        by.setdefault(name, []).append(d)
    con.close()
    out = {}
    for name, v in by.items():
        v.sort()
        k = len(v)
        out[name] = v[k // 2] if k % 2 else 0.5 * (v[k // 2 - 1] + v[k // 2])
    return out


def counter_stats(path: str, counter: str) -> list:
    con = sqlite3.connect(path)
    rows = con.execute(
        "select k.name, count(*), avg(p.counter_value) from pmc_events p "
        "join kernels k on k.dispatch_id = p.dispatch_id "
        "where p.counter_name = ? group by k.name order by avg(p.counter_value) desc",
        (counter,)).fetchall()
    con.close()
    return rows


def per_position(path: str, kernel: str, period: int, counter: str = "") -> list:
    """Average duration (trace db) or counter value (pmc db) of ``kernel``'s
    dispatches by position within each run of ``period`` consecutive ones
    (e.g. the 8 launches one forward makes of a shared kernel)."""
    con = sqlite3.connect(path)
    if counter:
        rows = con.execute(
            "select p.counter_value from pmc_events p join kernels k on k.dispatch_id = p.dispatch_id "
            "where k.name = ? and p.counter_name = ? order by k.dispatch_id", (kernel, counter)).fetchall()
    else:
        rows = con.execute("select duration from kernels where name = ? order by dispatch_id",
                           (kernel,)).fetchall()
    con.close()
    sums, counts = [0.0] * period, [0] * period
    for i, (v,) in enumerate(rows):
        sums[i % period] += v
        counts[i % period] += 1
    return [s / max(c, 1) for s, c in zip(sums, counts)]


def traffic(fetch_db, write_db, copy_fetch_db, copy_write_db, copy_mib) -> dict:
    true_kib = copy_mib * 1024.0
    cf = dict((n, v) for n, _, v in counter_stats(copy_fetch_db, "FETCH_SIZE"))["copy_bytes"]
    cw = dict((n, v) for n, _, v in counter_stats(copy_write_db, "WRITE_SIZE"))["copy_bytes"]
    fs, ws = true_kib / cf, true_kib / cw
    fetch = {n: v for n, _, v in counter_stats(fetch_db, "FETCH_SIZE")}
    write = {n: v for n, _, v in counter_stats(write_db, "WRITE_SIZE")}
    kernels = {n: {"fetch_bytes": fetch[n] * fs * 1024, "write_bytes": write.get(n, 0.0) * ws * 1024,
                   "traffic_bytes": (fetch[n] * fs + write.get(n, 0.0) * ws) * 1024}
               for n in fetch}
    return {"fetch_scale": fs, "write_scale": ws, "copy_mib": copy_mib, "kernels": kernels}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("db", nargs="?")
    ap.add_argument("--counter", default="")
    ap.add_argument("--by-grid", action="store_true",
                    help="one row per (kernel, grid size in work-items) instead of per kernel name")
    ap.add_argument("--traffic", nargs=4, metavar=("FETCH_DB", "WRITE_DB", "COPY_FETCH_DB", "COPY_WRITE_DB"))
    ap.add_argument("--copy-mib", type=int, default=256)
    ap.add_argument("--out", default="")
    ap.add_argument("--rates", metavar="TRAFFIC_JSON", default="",
                    help="with a kernel-trace db: HBM GB/s per kernel from a --traffic JSON")
    ap.add_argument("--per-launch", nargs=2, metavar=("KERNEL", "PERIOD"),
                    help="with a trace db and --traffic: HBM GB/s of each of a kernel's PERIOD "
                         "launches per forward")
    args = ap.parse_args(argv)
    if args.per_launch and args.traffic:
        kernel, period = args.per_launch[0], int(args.per_launch[1])
        true_kib = args.copy_mib * 1024.0
        cf = dict((n, v) for n, _, v in counter_stats(args.traffic[2], "FETCH_SIZE"))["copy_bytes"]
        cw = dict((n, v) for n, _, v in counter_stats(args.traffic[3], "WRITE_SIZE"))["copy_bytes"]
        dur = per_position(args.db, kernel, period)
        fet = per_position(args.traffic[0], kernel, period, "FETCH_SIZE")
        wri = per_position(args.traffic[1], kernel, period, "WRITE_SIZE")
        print(f"{'launch':>6s} {'avg_us':>8s} {'HBM_MB':>8s} {'GB/s':>7s} {'of 8 TB/s':>9s}")
        for i in range(period):
            b = (fet[i] * true_kib / cf + wri[i] * true_kib / cw) * 1024
            gbs = b / (dur[i] * 1e-9) / 1e9
            print(f"{i:6d} {dur[i] / 1e3:8.2f} {b / 1e6:8.2f} {gbs:7.0f} {gbs / 8000.0:9.1%}")
        return 0
    if args.rates:
        with open(args.rates) as f:
            t = json.load(f)["kernels"]
        print(f"{'kernel':64s} {'avg_us':>9s} {'HBM_MB':>9s} {'GB/s':>8s} {'of 8 TB/s':>9s}")
        for name, n, tot, avg, mn, mx in kernel_stats(args.db):
            if name in t:
                gbs = t[name]["traffic_bytes"] / (avg * 1e-9) / 1e9
                print(f"{name[:64]:64s} {avg / 1e3:9.2f} {t[name]['traffic_bytes'] / 1e6:9.2f} "
                      f"{gbs:8.0f} {gbs / 8000.0:9.1%}")
        return 0
    if args.traffic:
        t = traffic(*args.traffic, args.copy_mib)
        text = json.dumps(t, indent=1, sort_keys=True)
        if args.out:
            with open(args.out, "w") as f:
                f.write(text + "\n")
        print(f"scale: FETCH_SIZE x{t['fetch_scale']:.4f}, WRITE_SIZE x{t['write_scale']:.4f}")
        for n, d in sorted(t["kernels"].items(), key=lambda kv: -kv[1]["traffic_bytes"]):
            print(f"{n[:64]:64s} fetch {d['fetch_bytes'] / 1e6:9.2f} MB  write "
                  f"{d['write_bytes'] / 1e6:9.2f} MB")
        return 0
    if args.counter:
        print(f"{'kernel':64s} {'dispatches':>10s} {'avg ' + args.counter:>18s}")
        for name, n, avg in counter_stats(args.db, args.counter):
            print(f"{name[:64]:64s} {n:10d} {avg:18.1f}")
        return 0
    if args.by_grid:
        rows = kernel_stats_by_grid(args.db)
        total = sum(r[3] for r in rows) or 1
        print(f"{'kernel':56s} {'grid':>20s} {'calls':>6s} {'avg_us':>8s} {'med_us':>8s} "
              f"{'min_us':>8s} {'pct':>6s}")
        for name, grid, n, tot, avg, med, mn, mx in rows:
            print(f"{name[:56]:56s} {'x'.join(str(g) for g in grid):>20s} {n:6d} {avg / 1e3:8.2f} "
                  f"{med / 1e3:8.2f} {mn / 1e3:8.2f} {100.0 * tot / total:6.2f}")
        return 0
    rows = kernel_stats(args.db)
    med = kernel_medians(args.db)
    total = sum(r[2] for r in rows) or 1
    print(f"{'kernel':64s} {'calls':>6s} {'total_us':>10s} {'avg_us':>9s} {'med_us':>9s} "
          f"{'min_us':>9s} {'max_us':>9s} {'pct':>6s}")
    for name, n, tot, avg, mn, mx in rows:
        print(f"{name[:64]:64s} {n:6d} {tot / 1e3:10.1f} {avg / 1e3:9.2f} {med[name] / 1e3:9.2f} "
              f"{mn / 1e3:9.2f} {mx / 1e3:9.2f} {100.0 * tot / total:6.2f}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
