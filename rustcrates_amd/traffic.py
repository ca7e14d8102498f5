"""HBM bytes per launch of a kernel class, from rocprofv3 counters.

FETCH_SIZE and WRITE_SIZE (KiB per dispatch) do not read as plain bytes on
MI355X, so each is scaled by what it reads for a plain device copy of known
size (the calibration run).  Four counter runs, each in its own process
(run from the repository root on the GPU box, TMPDIR=/tmp):

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d gpurun_out/cal_f -o c -- python3 -m rustcrates_amd.traffic copy
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d gpurun_out/cal_w -o c -- python3 -m rustcrates_amd.traffic copy
    rocprofv3 --pmc FETCH_SIZE --output-format csv -d gpurun_out/wl_f -o w -- python3 bench.py --workload c3b32 \\
        --steps 1 --warmup 0 --no-cpu --no-b1 --no-classes --direct
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d gpurun_out/wl_w -o w -- python3 bench.py ... (same)

then

    python -m rustcrates_amd.traffic summarize --cal-fetch gpurun_out/cal_f --cal-write gpurun_out/cal_w \\
        --fetch gpurun_out/wl_f --write gpurun_out/wl_w --workload c3b32 --kernel-class layer_gemm \\
        --match 'k_zgemm_skinny<' --out profiles/layer_gemm_c3b32_traffic

writes <out>.json (read by bench.py for the roofline's `traffic`) and <out>.md.
`stats` writes the per-kernel table of a --kernel-trace database; `mfma` the
MFMA utilisation of a class from a SQ_VALU_MFMA_BUSY_CYCLES /
SQ_INSTS_VALU_MFMA_MOPS_F64 counter run and a kernel trace of the same workload.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
import sys

COPY_BYTES = 1 << 30  # the calibration copy: 1 GiB read + 1 GiB written, above the 256 MB last-level cache


def _copy() -> None:
    import torch

    a = torch.empty(COPY_BYTES // 8, dtype=torch.float64, device="cuda").uniform_()
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(f"copied {COPY_BYTES} bytes x 3", flush=True)


def _rows(d: str):
    """(kernel name, dispatch id, counter, value) of every counter row under d."""
    files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {d}")
    for f in files:
        with open(f) as fh:
            for r in csv.DictReader(fh):
                yield r["Kernel_Name"], r.get("Dispatch_Id", ""), r["Counter_Name"], float(r["Counter_Value"])


def _per_dispatch(d: str, counter: str):
    out = {}
    for name, disp, cname, val in _rows(d):
        if cname == counter:
            key = (name, disp)
            out[key] = out.get(key, 0.0) + val
    return out


def _short(name: str) -> str:
    return re.sub(r"\(.*", "", name).replace("void ", "")


def _summarize(a) -> None:
    cal_f = _per_dispatch(a.cal_fetch, "FETCH_SIZE")
    cal_w = _per_dispatch(a.cal_write, "WRITE_SIZE")
    # the copy: the dispatches that moved the most (3 identical copies)
    top_f = sorted(cal_f.values())[-3:]
    top_w = sorted(cal_w.values())[-3:]
    f_kib = sum(top_f) / len(top_f)
    w_kib = sum(top_w) / len(top_w)
    factor_f = COPY_BYTES / (f_kib * 1024.0)
    factor_w = COPY_BYTES / (w_kib * 1024.0)
    pat = re.compile(re.escape(a.match))
    excl = re.compile(re.escape(a.exclude)) if a.exclude else None
    fetch = {k: v for k, v in _per_dispatch(a.fetch, "FETCH_SIZE").items() if pat.search(_short(k[0]))
             and not (excl and excl.search(_short(k[0])))}
    write = {k: v for k, v in _per_dispatch(a.write, "WRITE_SIZE").items() if pat.search(_short(k[0]))
             and not (excl and excl.search(_short(k[0])))}
    if not fetch or not write:
        raise SystemExit(f"no dispatch of a kernel matching {a.match!r}")
    fb = sum(fetch.values()) / len(fetch) * 1024.0 * factor_f
    wb = sum(write.values()) / len(write) * 1024.0 * factor_w
    kernels = sorted({_short(k[0]) for k in fetch})
    from .build import source_hash

    res = {
        "workload": a.workload,
        "kernel_class": a.kernel_class,
        "csrc_sha": source_hash(),
        "kernels": kernels,
        "dispatches": len(fetch),
        "fetch_bytes_per_launch": fb,
        "write_bytes_per_launch": wb,
        "traffic_bytes_per_launch": fb + wb,
        "copy_bytes": COPY_BYTES,
        "copy_fetch_kib": f_kib,
        "copy_write_kib": w_kib,
        "factor_fetch": factor_f,
        "factor_write": factor_w,
    }
    with open(a.out + ".json", "w") as fh:
        json.dump(res, fh, indent=1)
    with open(a.out + ".md", "w") as fh:
        fh.write(f"# HBM traffic per launch: {a.kernel_class} at {a.workload}\n\n")
        fh.write("Measured with rocprofv3 counter runs and `python -m rustcrates_amd.traffic summarize` "
                 f"(`--match {a.match!r}`" + (f", `--exclude {a.exclude!r}`" if a.exclude else "") + ").\n")
        cmds = [
            f"rocprofv3 --pmc FETCH_SIZE --output-format csv -d {a.cal_fetch} -o c -- python3 -m rustcrates_amd.traffic copy",
            f"rocprofv3 --pmc WRITE_SIZE --output-format csv -d {a.cal_write} -o c -- python3 -m rustcrates_amd.traffic copy",
            f"rocprofv3 --pmc FETCH_SIZE --output-format csv -d {a.fetch} -o w -- python3 {a.run}",
            f"rocprofv3 --pmc WRITE_SIZE --output-format csv -d {a.write} -o w -- python3 {a.run}",
            f"python -m rustcrates_amd.traffic summarize --cal-fetch {a.cal_fetch} --cal-write {a.cal_write} "
            f"--fetch {a.fetch} --write {a.write} --workload {a.workload} --kernel-class {a.kernel_class} "
            f"--match '{a.match}'" + (f" --exclude '{a.exclude}'" if a.exclude else "") + f" --run '{a.run}' --out {a.out}",
        ]
        fh.write("Commands (from the repository root on the MI355X box, TMPDIR=/tmp; each counter run in its "
                 "own process):\n\n```\n" + "\n".join(cmds) + "\n```\n\n")
        fh.write("| quantity | value |\n|---|---:|\n")
        fh.write(f"| calibration copy | {COPY_BYTES} B read + {COPY_BYTES} B written |\n")
        fh.write(f"| copy FETCH_SIZE | {f_kib:.0f} KiB (factor {factor_f:.4f}) |\n")
        fh.write(f"| copy WRITE_SIZE | {w_kib:.0f} KiB (factor {factor_w:.4f}) |\n")
        fh.write(f"| dispatches of the class | {len(fetch)} |\n")
        fh.write(f"| fetched per launch (scaled) | {fb / 1e6:.3f} MB |\n")
        fh.write(f"| written per launch (scaled) | {wb / 1e6:.3f} MB |\n")
        fh.write(f"| traffic per launch | {(fb + wb) / 1e6:.3f} MB |\n\n")
        fh.write("Kernels: " + ", ".join(f"`{k}`" for k in kernels) + "\n\n")
        fh.write(f"Sources: `csrc` SHA-256 prefix `{res['csrc_sha']}` (bench.py reports this traffic only while "
                 "the sources hash the same).\n")
    print(json.dumps(res))


def _stats(a) -> None:
    """Per-kernel summary of a rocprofv3 --kernel-trace database: calls, total,
    average and share of the traced kernel time, per kernel and grid shape."""
    import sqlite3

    dbs = glob.glob(os.path.join(a.trace, "**", "*.db"), recursive=True)
    if not dbs:
        raise SystemExit(f"no rocpd database under {a.trace}")
    c = sqlite3.connect(dbs[0])
    q = ("select name, grid_x, grid_y, grid_z, workgroup_x, count(*), sum(duration), avg(duration) "
         "from kernels group by name, grid_x, grid_y, grid_z order by sum(duration) desc")
    rows = list(c.execute(q))
    total = sum(r[6] for r in rows) or 1
    with open(a.out, "w") as fh:
        fh.write(f"# {a.title}\n\n")
        fh.write("Command (from the repository root on the MI355X box, TMPDIR=/tmp):\n\n```\n" + a.command + "\n```\n\n")
        fh.write("Summary: `python -m rustcrates_amd.traffic stats`.  Durations in microseconds from the "
                 "rocpd database's `kernels` view; grid in threads.\n\n")
        fh.write("| kernel | grid | calls | total us | avg us | % |\n|---|---|---:|---:|---:|---:|\n")
        for name, gx, gy, gz, wx, n, tot, avg in rows:
            if tot / total < a.min_share:
                continue
            fh.write(f"| `{_short(name)}` | {gx}x{gy}x{gz} | {n} | {tot / 1e3:.1f} | {avg / 1e3:.3f} | "
                     f"{100.0 * tot / total:.2f} |\n")
    print(f"wrote {a.out}")


def _mfma(a) -> None:
    """MFMA utilisation per kernel of a class: SQ_VALU_MFMA_BUSY_CYCLES (summed
    over the SIMDs) against SIMDs x clock x the kernel's traced duration, and
    SQ_INSTS_VALU_MFMA_MOPS_F64 x 512 against the algorithmic flops."""
    import sqlite3

    busy = _per_dispatch(a.counters, "SQ_VALU_MFMA_BUSY_CYCLES")
    mops = _per_dispatch(a.counters, "SQ_INSTS_VALU_MFMA_MOPS_F64")
    pat = re.compile(re.escape(a.match))
    dbs = glob.glob(os.path.join(a.trace, "**", "*.db"), recursive=True)
    if not dbs:
        raise SystemExit(f"no rocpd database under {a.trace}")
    c = sqlite3.connect(dbs[0])
    # the counter rows give only the total thread count, so launches of one
    # kernel whose grids have the same total are averaged together
    acc = {}
    for name, gx, gy, gz, n, tot in c.execute("select name, grid_x, grid_y, grid_z, count(*), sum(duration) "
                                              "from kernels group by name, grid_x, grid_y, grid_z"):
        if pat.search(_short(name)):
            e = acc.setdefault((_short(name), gx * gy * gz), [0, 0.0])
            e[0] += n
            e[1] += tot
    dur = {k: tot / n * 1e-9 for k, (n, tot) in acc.items()}
    cnt = {}
    for r in csv.DictReader(open(glob.glob(os.path.join(a.counters, "**", "*counter_collection.csv"),
                                           recursive=True)[0])):
        cnt[(r["Kernel_Name"], r["Dispatch_Id"])] = int(r["Grid_Size"])
    by = {}
    for key, b in busy.items():
        k = _short(key[0])
        if not pat.search(k):
            continue
        g = cnt[key]
        e = by.setdefault((k, g), [0, 0.0, 0.0])
        e[0] += 1
        e[1] += b
        e[2] += mops.get(key, 0.0)
    with open(a.out, "w") as fh:
        fh.write(f"# {a.title}\n\n")
        fh.write("Commands (from the repository root on the MI355X box, TMPDIR=/tmp):\n\n```\n" + a.command + "\n```\n\n")
        fh.write(f"Summary: `python -m rustcrates_amd.traffic mfma`.  Utilisation = busy cycles / ({a.simds} SIMDs x "
                 f"{a.clock_ghz} GHz x traced duration); flops = MOPS_F64 x 512.\n\n")
        fh.write("| kernel | grid (threads) | dispatches | MFMA busy cycles | MOPS_F64 x 512 (GFLOP) | traced us | "
                 "MFMA busy | TFLOP/s |\n|---|---:|---:|---:|---:|---:|---:|---:|\n")
        for (k, g), (n, b, m) in sorted(by.items()):
            d = dur.get((k, g))
            bb, mm = b / n, m / n
            util = bb / (a.simds * a.clock_ghz * 1e9 * d) if d else float("nan")
            tf = mm * 512 / d / 1e12 if d else float("nan")
            fh.write(f"| `{k}` | {g} | {n} | {bb:.4g} | {mm * 512 / 1e9:.2f} | {d * 1e6 if d else float('nan'):.1f} | "
                     f"{100 * util:.1f}% | {tf:.1f} |\n")
    print(f"wrote {a.out}")


def main() -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    sub.add_parser("copy")
    st = sub.add_parser("stats")
    st.add_argument("--trace", required=True)
    st.add_argument("--title", required=True)
    st.add_argument("--command", required=True)
    st.add_argument("--out", required=True)
    st.add_argument("--min-share", type=float, default=0.001)
    s = sub.add_parser("summarize")
    for k in ("cal-fetch", "cal-write", "fetch", "write", "workload", "kernel-class", "match", "out"):
        s.add_argument("--" + k, required=True)
    s.add_argument("--exclude", default="")
    s.add_argument("--run", default="bench.py --workload c3b32 --steps 1 --warmup 0 --no-cpu --no-b1 --no-classes --direct",
                   help="the profiled program (its arguments after python3)")
    mf = sub.add_parser("mfma")
    for k in ("counters", "trace", "match", "title", "command", "out"):
        mf.add_argument("--" + k, required=True)
    mf.add_argument("--simds", type=int, default=1024)
    mf.add_argument("--clock-ghz", type=float, default=2.4)
    a = ap.parse_args()
    if a.cmd == "mfma":
        _mfma(a)
        return
    if a.cmd == "copy":
        _copy()
    elif a.cmd == "stats":
        _stats(a)
    else:
        _summarize(a)


if __name__ == "__main__":
    main()
