# -*- coding: utf-8 -*-
"""Summarise a rocprofv3 database (``--kernel-trace``, rocpd SQLite output)
per kernel launch shape, for the roofline figures of this backend.

``rocpd2summary`` averages per kernel symbol; one MFMA conv instantiation
serves several decoder stages and the ConvTranspose phases, so the per-symbol
average mixes shapes.  This groups dispatches by (symbol, grid, workgroup)
instead, and reports the decoder ResBlock family the benchmark's roofline
uses: every persistent ``conv1d_mfma_persist_kernel<..., 1>`` dispatch (the
instantiation reserved for launches of three stored groups: the three
ResBlocks of a stage share one launch) and every one-shot
``conv1d_mfma_kernel`` dispatch whose grid z is 3 and whose grid is at least
64 workgroups wide (a ResBlock launch spans 10P..400P samples, at least 79
workgroups at P = 1000; the enc_p / flow convs span P samples, at most 32
workgroups, and their split-K launches can also have z = 3).

    python -m rvc_hip.profsum prof/bench_results.db [--steps N]

With ``--pmc`` it also reports the ``FETCH_SIZE`` / ``WRITE_SIZE`` counter
means (KiB per dispatch) of a ``rocprofv3 --pmc`` database, grouped the same
way.

With ``--traffic`` it turns four ``--pmc`` databases into HBM bytes per
dispatch: FETCH_SIZE and WRITE_SIZE of the benchmark, each scaled by what
the same counter reads on the library's copy kernel moving a known number of
bytes (``bench.py --calibrate-copy MIB``):

    python -m rvc_hip.profsum --traffic --copy-mib 256 \
        --copy-fetch copy_fetch.db --copy-write copy_write.db bench_fetch.db bench_write.db

It prints a table per launch shape and one machine-readable line for the
ResBlock family, ``resblock_traffic_bytes_per_launch: N``, which ``bench.py``
reads from the committed summary.
"""

from __future__ import annotations

import argparse
import re
import sqlite3
import sys


def _short(name: str) -> str:
    name = name.replace("rvc::(anonymous namespace)::", "").replace("void ", "")
    name = re.sub(r"\(.*\)$", "", name)
    return name


def kernel_rows(db: str):
    con = sqlite3.connect(db)
    q = ("select name, grid_x, grid_y, grid_z, workgroup_x, lds_size, vgpr_count, accum_vgpr_count, "
         "count(*), avg(duration), sum(duration) from kernels "
         "group by name, grid_x, grid_y, grid_z, workgroup_x order by sum(duration) desc")
    rows = []
    for r in con.execute(q):
        name, gx, gy, gz, wx, lds, v, a, n, avg, tot = r
        rows.append({"kernel": _short(name), "grid": (gx // max(wx, 1), gy, gz), "wg": wx, "lds": lds,
                     "vgpr": v, "agpr": a, "calls": n, "avg_us": avg / 1e3, "total_ms": tot / 1e6})
    return rows


def pmc_rows(db: str):
    con = sqlite3.connect(db)
    q = ("select k.name, k.grid_x, k.grid_y, k.grid_z, k.workgroup_x, p.counter_name, avg(p.counter_value), count(*) "
         "from pmc_events p join kernels k on p.event_id = k.id "
         "group by k.name, k.grid_x, k.grid_y, k.grid_z, p.counter_name")
    out = []
    for name, gx, gy, gz, wx, cn, val, n in con.execute(q):
        out.append({"kernel": _short(name), "grid": (gx // max(wx, 1), gy, gz), "counter": cn, "mean": val,
                    "n": n})
    return out


def is_resblock(kernel: str, grid) -> bool:
    if kernel.startswith("conv1d_mfma_persist_kernel"):
        return kernel.replace(" ", "").endswith(",1>")   # FAM = 1: the three-group stored launches
    return kernel.startswith("conv1d_mfma_kernel") and grid[2] == 3 and grid[0] >= 64


def _counter_means(db: str, counter: str):
    """{(kernel, grid): (mean KiB per dispatch, dispatches)} for one counter."""
    return {(r["kernel"], r["grid"]): (r["mean"], r["n"]) for r in pmc_rows(db) if r["counter"] == counter}


def _copy_factor(db: str, counter: str, mib: int) -> float:
    """Known bytes / counted bytes for the copy kernel (each launch reads and
    writes ``mib`` MiB)."""
    rows = [(v, n) for (k, _), (v, n) in _counter_means(db, counter).items() if k.startswith("copy_kernel")]
    if not rows:
        raise SystemExit(f"{db}: no copy_kernel dispatch with {counter}")
    kib = sum(v * n for v, n in rows) / sum(n for _, n in rows)
    return mib * 1024.0 / kib


def traffic(fetch_db: str, write_db: str, copy_fetch: str, copy_write: str, mib: int) -> int:
    ff = _copy_factor(copy_fetch, "FETCH_SIZE", mib)
    fw = _copy_factor(copy_write, "WRITE_SIZE", mib)
    fetch = _counter_means(fetch_db, "FETCH_SIZE")
    write = _counter_means(write_db, "WRITE_SIZE")
    print(f"copy calibration ({mib} MiB copies): FETCH_SIZE x {ff:.3f}, WRITE_SIZE x {fw:.3f}\n")
    print("| kernel | grid | dispatches | read MB | write MB | HBM MB per dispatch |")
    print("|---|---|---:|---:|---:|---:|")
    keys = sorted(set(fetch) & set(write), key=lambda k: -(fetch[k][0] + write[k][0]) * fetch[k][1])
    fam_b, fam_n = 0.0, 0
    for k in keys:
        rd = fetch[k][0] * 1024 * ff
        wr = write[k][0] * 1024 * fw
        n = fetch[k][1]
        print(f"| {k[0]} | {k[1]} | {n} | {rd / 1e6:.2f} | {wr / 1e6:.2f} | {(rd + wr) / 1e6:.2f} |")
        if is_resblock(*k):
            fam_b += (rd + wr) * n
            fam_n += n
    if fam_n:
        print(f"\nResBlock family (persistent FAM 1, or one-shot grid z = 3 and >= 64 wide): {fam_n} dispatches")
        print(f"resblock_traffic_bytes_per_launch: {int(round(fam_b / fam_n))}")
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("db")
    ap.add_argument("db2", nargs="?", help="with --traffic: the WRITE_SIZE database (db is FETCH_SIZE)")
    ap.add_argument("--traffic", action="store_true")
    ap.add_argument("--copy-fetch")
    ap.add_argument("--copy-write")
    ap.add_argument("--copy-mib", type=int, default=256)
    ap.add_argument("--steps", type=int, default=0, help="timed steps in the run (per-step figures)")
    ap.add_argument("--top", type=int, default=30)
    ap.add_argument("--pmc", action="store_true")
    args = ap.parse_args(argv)
    if args.traffic:
        if not (args.db2 and args.copy_fetch and args.copy_write):
            ap.error("--traffic needs FETCH and WRITE databases and --copy-fetch / --copy-write")
        return traffic(args.db, args.db2, args.copy_fetch, args.copy_write, args.copy_mib)
    if args.pmc:
        print("| kernel | grid | counter | mean per dispatch | dispatches |")
        print("|---|---|---|---:|---:|")
        for r in pmc_rows(args.db):
            print(f"| {r['kernel']} | {r['grid']} | {r['counter']} | {r['mean']:.1f} | {r['n']} |")
        return 0
    rows = kernel_rows(args.db)
    print("| kernel | grid (workgroups) | wg | LDS B | VGPR | AGPR | calls | avg us | total ms |")
    print("|---|---|---:|---:|---:|---:|---:|---:|---:|")
    for r in rows[:args.top]:
        print(f"| {r['kernel']} | {r['grid']} | {r['wg']} | {r['lds']} | {r['vgpr']} | {r['agpr']} | "
              f"{r['calls']} | {r['avg_us']:.1f} | {r['total_ms']:.2f} |")
    rb = [r for r in rows if is_resblock(r["kernel"], r["grid"])]
    n = sum(r["calls"] for r in rb)
    tot = sum(r["total_ms"] for r in rb)
    if n:
        print(f"\nResBlock family (persistent FAM 1, or one-shot grid z = 3 and >= 64 wide): {n} dispatches, "
              f"{tot:.2f} ms total, average {tot * 1e3 / n:.1f} us per dispatch")
    allk = sum(r["total_ms"] for r in rows)
    print(f"all kernels: {allk:.2f} ms" + (f", {allk / args.steps:.3f} ms per step" if args.steps else ""))
    return 0


if __name__ == "__main__":
    sys.exit(main())
