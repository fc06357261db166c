# -*- coding: utf-8 -*-
"""Summarise a rocprofv3 database (``--kernel-trace``, rocpd SQLite output)
per kernel launch shape, for the roofline figures of this backend.

``rocpd2summary`` averages per kernel symbol; one MFMA conv instantiation
serves several decoder stages and the ConvTranspose phases, so the per-symbol
average mixes shapes.  This groups dispatches by (symbol, grid, workgroup)
instead, and reports the decoder ResBlock family the benchmark's roofline
uses: every ``conv1d_mfma_kernel`` dispatch whose grid z is 3 (the three
ResBlocks of a stage share one launch, z = 3 groups x batch 1).

    python -m rvc_hip.profsum gpurun_out/prof/bench_results.db [--steps N]

With ``--pmc`` it also reports the ``FETCH_SIZE`` / ``WRITE_SIZE`` counter
means (KiB per dispatch) of a ``rocprofv3 --pmc`` database, grouped the same
way.
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


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("db")
    ap.add_argument("--steps", type=int, default=0, help="timed steps in the run (per-step figures)")
    ap.add_argument("--top", type=int, default=30)
    ap.add_argument("--pmc", action="store_true")
    args = ap.parse_args(argv)
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
    rb = [r for r in rows if r["kernel"].startswith("conv1d_mfma_kernel") and r["grid"][2] == 3]
    n = sum(r["calls"] for r in rb)
    tot = sum(r["total_ms"] for r in rb)
    if n:
        print(f"\nResBlock family (conv1d_mfma_kernel, grid z = 3): {n} dispatches, "
              f"{tot:.2f} ms total, average {tot * 1e3 / n:.1f} us per dispatch")
    allk = sum(r["total_ms"] for r in rows)
    print(f"all kernels: {allk:.2f} ms" + (f", {allk / args.steps:.3f} ms per step" if args.steps else ""))
    return 0


if __name__ == "__main__":
    sys.exit(main())
