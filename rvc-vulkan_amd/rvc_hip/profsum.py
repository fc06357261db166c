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

With ``--sq`` it turns two ``--pmc`` databases of SQ counters into MFMA
utilisation and instruction mix per launch shape:

    pass A: SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY
            SQ_ACTIVE_INST_ANY SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_MFMA
    pass B: SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_INSTS_VALU
            SQ_INSTS_SALU SQ_INSTS_VMEM_RD (optional)

    python -m rvc_hip.profsum --sq pass_a.db [pass_b.db]

MFMA busy is SQ_VALU_MFMA_BUSY_CYCLES (summed over every SIMD) divided by
the SIMD-cycles of the dispatch: 1024 SIMDs x duration x clock, once at the
2.4 GHz peak engine clock (the basis of the published 157.3 TFLOP/s) and once
at the clock the shader engines actually ran (SQ_BUSY_CYCLES / 32 engines /
duration).
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
        # template arguments <BM, BN, WM, WN, BK, FAM[, DIRECT]>: FAM = 1 marks
        # the three-group stored launches
        args = kernel[kernel.find("<") + 1:kernel.rfind(">")].replace(" ", "").split(",")
        return len(args) >= 6 and args[5] == "1"
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


N_SIMD, N_SE, PEAK_GHZ = 1024, 32, 2.4


def _sq(db: str):
    """{(kernel, grid): {counter: mean per dispatch}}, dispatch counts and
    mean durations (ns), from the database's per-dispatch counter view."""
    con = sqlite3.connect(db)
    q = ("select dispatch_id, kernel_name, grid_size_x, grid_size_y, grid_size_z, workgroup_size_x, "
         "counter_name, value, duration from counters_collection")
    per, key = {}, {}
    for did, name, gx, gy, gz, wx, cn, v, d in con.execute(q):
        key[did] = ((_short(name), (gx // max(wx, 1), gy, gz)), d)
        per.setdefault(did, {})[cn] = v
    means, counts, dur = {}, {}, {}
    for did, cs in per.items():
        k, d = key[did]
        counts[k] = counts.get(k, 0) + 1
        dur[k] = dur.get(k, 0.0) + d
        m = means.setdefault(k, {})
        for cn, v in cs.items():
            m[cn] = m.get(cn, 0.0) + v
    for k in means:
        for cn in means[k]:
            means[k][cn] /= counts[k]
        dur[k] /= counts[k]
    return means, counts, dur


def sq_summary(db_a: str, db_b: str = None) -> int:
    a, n, dur = _sq(db_a)
    b = _sq(db_b)[0] if db_b else {}
    print("| kernel | grid | dispatches | us | clock GHz | MFMA busy at 2.4 GHz | MFMA busy at run clock | "
          "wait / waitcnt | wait / issue | VALU per MFMA | SALU per MFMA | LDS per MFMA | bank-conflict cycles |")
    print("|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|")
    fam = [0.0, 0.0, 0.0]  # busy cycles, SIMD-cycles at 2.4 GHz, at run clock
    for k in sorted(a, key=lambda k: -dur.get(k, 0) * n[k]):
        c = a[k]
        if "SQ_VALU_MFMA_BUSY_CYCLES" not in c or k not in dur:
            continue
        d = dur[k] * 1e-9
        busy = c["SQ_VALU_MFMA_BUSY_CYCLES"]
        clk = c.get("SQ_BUSY_CYCLES", 0.0) / N_SE / d / 1e9 if d > 0 else 0.0
        at_peak = busy / (N_SIMD * d * PEAK_GHZ * 1e9) if d > 0 else 0.0
        at_run = busy / (N_SIMD * d * clk * 1e9) if clk > 0 else 0.0
        w = max(c.get("SQ_WAVE_CYCLES", 0.0), 1.0)
        mf = c.get("SQ_INSTS_MFMA", 0.0)
        cb = b.get(k, {})
        mix = (f"{cb['SQ_INSTS_VALU'] / mf:.2f} | {cb['SQ_INSTS_SALU'] / mf:.2f} | {cb['SQ_INSTS_LDS'] / mf:.2f} | "
               f"{cb['SQ_LDS_BANK_CONFLICT'] / max(cb['SQ_LDS_IDX_ACTIVE'], 1.0):.2f}"
               if mf > 0 and {"SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT",
                              "SQ_LDS_IDX_ACTIVE"} <= set(cb) else "- | - | - | -")
        print(f"| {k[0]} | {k[1]} | {n[k]} | {dur[k] / 1e3:.1f} | {clk:.2f} | {at_peak:.3f} | {at_run:.3f} | "
              f"{c.get('SQ_WAIT_ANY', 0.0) / w:.2f} | {c.get('SQ_WAIT_INST_ANY', 0.0) / w:.2f} | {mix} |")
        if is_resblock(*k):
            fam[0] += busy * n[k]
            fam[1] += N_SIMD * d * PEAK_GHZ * 1e9 * n[k]
            fam[2] += N_SIMD * d * clk * 1e9 * n[k]
    if fam[1] > 0:
        print(f"\nResBlock family (persistent FAM 1, or one-shot grid z = 3 and >= 64 wide):")
        print(f"resblock_mfma_busy_at_peak_clock: {fam[0] / fam[1]:.3f}")
        print(f"resblock_mfma_busy_at_run_clock: {fam[0] / fam[2]:.3f}")
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
    ap.add_argument("--sq", action="store_true", help="SQ-counter MFMA utilisation (db = pass A, db2 = pass B)")
    args = ap.parse_args(argv)
    if args.sq:
        return sq_summary(args.db, args.db2)
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
