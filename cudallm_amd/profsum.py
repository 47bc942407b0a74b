"""Summaries of rocprofv3 output for this library's kernels (the tables under profiles/).

    python -m cudallm_amd.profsum trace DIR [--matvec-blocks WTYPE] [--decode [--skip N] [--take K]]
                                            [--bench-legs STEPS,WARMUP]
    python -m cudallm_amd.profsum trace DIR --graph-runs LABEL,LABEL,... [--steps K] [--prompt P]
    python -m cudallm_amd.profsum counters FETCH_DIR WRITE_DIR [--calib-bytes N]

``trace``: reads DIR/*kernel_trace.csv (rocprofv3 --kernel-trace).  With --matvec-blocks the matvec dispatches are
split into contiguous runs of one kernel name (cudallm_amd.kernelbench --op shapes launches qkv, wo, gate_up, down,
lm_head in that order, and consecutive shapes use different kernel instances), and each run is matched to its shape
by position; per run: calls, mean / median / min / max duration, and GB/s and the fraction of 8 TB/s from the shape's
algorithmic bytes.  With --decode: the persistent decode kernels per weight type.  With --graph-runs (the output of
cudallm_amd.graphbench): per weight type, the decode dispatches split into runs of P prompt + K timed steps, one per
label; per run the timed steps' mean duration and the gaps between consecutive dispatches (start minus the previous
end).

``counters``: two rocprofv3 --pmc runs (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch); each counter is scaled by
what it reads for the largest __amd_rocclr_copyBuffer dispatch of known size (--calib-bytes, the bench's
--copy-calib), and the decode kernels' read and write bytes per launch are printed against their algorithmic bytes.
"""
import argparse
import csv
import glob
import json
import statistics
import sys
from pathlib import Path

from .kernelbench import SHAPES, matvec_bytes

PEAK = 8.0e12
WEIGHT_BYTES = {"bf16": 2471764096, "int8": 1238037632, "int4": 637452416}
DTYPE_OF = {"WType)1": "bf16", "WType)3": "int8", "WType)4": "int4"}


def _rows(d: Path, suffix: str):
    files = sorted(glob.glob(str(d / f"**/*{suffix}"), recursive=True))
    if not files:
        raise SystemExit(f"no *{suffix} under {d}")
    with open(files[0], newline="") as f:
        return list(csv.DictReader(f))


def _dtype(name: str) -> str | None:
    for k, v in DTYPE_OF.items():
        if k in name:
            return v
    for v in ("bf16", "int8", "int4"):
        if f"<{v}" in name or f"({v}" in name:
            return v
    return None


def _stats(us):
    return {"calls": len(us), "mean_us": statistics.fmean(us), "median_us": statistics.median(us), "min_us": min(us),
            "max_us": max(us)}


STREAM_WARMUP = 5  # kernelbench's stream_read launches this many untimed reads per launch shape


def matvec_blocks(rows, wtype: str):
    """Matvec dispatches in contiguous runs of one kernel name, matched to SHAPES by position; the bandwidth kernel's
    dispatches after a shape's run (kernelbench --stream) are that shape's stream reads, per launch shape (grid size),
    of which the fastest shape's mean (warm-up dropped) is reported."""
    blocks = []
    for r in sorted(rows, key=lambda r: int(r["Start_Timestamp"])):
        name = r["Kernel_Name"]
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        if "matvec" in name:
            if blocks and blocks[-1][0] == name and not blocks[-1][2]:
                blocks[-1][1].append(us)
            else:
                blocks.append((name, [us], {}))
        elif "stream_read_kernel" in name and blocks:
            blocks[-1][2].setdefault(r.get("Grid_Size_X", "?"), []).append(us)
    out = []
    for (name, us, streams), shape in zip(blocks, SHAPES):
        sname, rws, cols, ep, norm = shape
        st = _stats(us)
        b = matvec_bytes(wtype, rws, cols)
        st.update(shape=sname, rows=rws, cols=cols, kernel=name.split("(")[0], bytes=b,
                  gbps=b / st["mean_us"] / 1e3, frac_of_8tbs=b / st["mean_us"] / 1e3 / (PEAK / 1e9))
        means = [statistics.fmean(v[STREAM_WARMUP:]) for v in streams.values() if len(v) > STREAM_WARMUP]
        if means:
            st["stream_mean_us"] = min(means)
        out.append(st)
    return out


PROBE_US = 50.0  # the engine's co-residency probe launch of the decode kernel takes a few microseconds


def _decode_launches(rows):
    """Durations (us) of the decode kernel's launches per weight type in dispatch order, and its probe launches."""
    per, probes = {}, {}
    for r in sorted(rows, key=lambda r: int(r["Start_Timestamp"])):
        if "decode_kernel" not in r["Kernel_Name"]:
            continue
        wd = _dtype(r["Kernel_Name"])
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        (probes if us < PROBE_US else per).setdefault(wd, []).append(us)
    return per, probes


def bench_legs(rows, steps: int, warmup: int, prompt: int = 16, c5_reps: int = 5, c5_warmup: int = 1, c5_gen: int = 256):
    """bench.py's decode launches per weight type, split into its legs.  The decode leg launches a warm-up sequence
    (prompt + warmup steps), the timed sequence's prompt, `steps` timed steps and one more step that returns the
    last token; the config-5 leg then runs c5_warmup + c5_reps sequences of prompt + c5_gen steps, of which the
    last c5_gen of each timed rep are timed."""
    per, _ = _decode_launches(rows)
    out = {}
    for wd, us in per.items():
        t0 = prompt + warmup + prompt
        timed = us[t0:t0 + steps]
        leg = {"decode_timed": _stats(timed)}
        # The timed steps by attention split count: step i attends over prompt + 1 + i positions, in 128-token splits.
        by = {}
        for i, v in enumerate(timed):
            by.setdefault((prompt + 1 + i + 127) // 128, []).append((prompt + 1 + i, v))
        leg["decode_timed_by_splits"] = {f"{k} ({c[0][0]}..{c[-1][0]})": _stats([v for _, v in c])
                                         for k, c in sorted(by.items())}
        c0 = t0 + steps + 1
        c5 = []
        for r in range(c5_warmup, c5_warmup + c5_reps):
            s0 = c0 + r * (prompt + c5_gen) + prompt
            c5 += us[s0:s0 + c5_gen]
        if c5:
            leg["config5_timed"] = _stats(c5)
        leg["launches"] = len(us)
        leg["expected_launches"] = c0 + (c5_warmup + c5_reps) * (prompt + c5_gen) if c5 else c0
        out[wd] = leg
    return out


def decode_stats(rows, skip: int = 0, take: int = 0):
    """Decode steps per weight type, in dispatch order; the co-residency probe launches (same kernel, under PROBE_US)
    are counted apart.  `skip` drops each weight type's first steps and `take` (when > 0) keeps the next `take`.
    bench_legs() gives the skip and take of bench.py's timed launches."""
    per, probes = _decode_launches(rows)
    per = {wd: us[skip:skip + take] if take > 0 else us[skip:] for wd, us in per.items()}
    out = {wd: _stats(us) for wd, us in per.items() if us}
    for wd, us in probes.items():
        out.setdefault(wd, {})["probe_launches"] = len(us)
    return out


def graph_runs(rows, labels: list[str], steps: int, prompt: int = 16):
    per = {}
    for r in sorted(rows, key=lambda r: int(r["Start_Timestamp"])):
        if "decode_kernel" not in r["Kernel_Name"]:
            continue
        st, en = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
        if (en - st) / 1e3 < PROBE_US:
            continue
        per.setdefault(_dtype(r["Kernel_Name"]), []).append((st, en))
    out = {}
    for wd, d in per.items():
        runs = {}
        for i, label in enumerate(labels):
            run = d[i * (prompt + steps) + prompt:(i + 1) * (prompt + steps)]
            if len(run) < 2:
                continue
            gaps = [(run[k + 1][0] - run[k][1]) / 1e3 for k in range(len(run) - 1)]
            durs = [(e - s) / 1e3 for s, e in run]
            runs[label] = {"steps": len(run), "mean_us": statistics.fmean(durs), "gap_median_us": statistics.median(gaps),
                           "gap_mean_us": statistics.fmean(gaps), "gap_max_us": max(gaps),
                           "span_us_per_step": (run[-1][1] - run[0][0]) / 1e3 / len(run)}
        out[wd] = runs
    return out


def counters(fetch_dir: Path, write_dir: Path, calib_bytes: int):
    def load(d, counter):
        rows = [r for r in _rows(d, "counter_collection.csv") if r["Counter_Name"] == counter]
        copies = [float(r["Counter_Value"]) for r in rows if r["Kernel_Name"] == "__amd_rocclr_copyBuffer"]
        dec = {}
        for r in rows:
            if "decode_kernel" in r["Kernel_Name"]:
                dec.setdefault(_dtype(r["Kernel_Name"]), []).append(float(r["Counter_Value"]))
        return (max(copies) if copies else None), dec
    fc, fd = load(fetch_dir, "FETCH_SIZE")
    wc, wdc = load(write_dir, "WRITE_SIZE")
    ffac = calib_bytes / (fc * 1024) if fc else None
    wfac = calib_bytes / (wc * 1024) if wc else None
    out = {"copy_calibration": {"bytes": calib_bytes, "fetch_kib": fc, "write_kib": wc, "fetch_factor": ffac,
                                "write_factor": wfac}, "kernels": {}}
    for wd in sorted(set(fd) | set(wdc)):
        f = statistics.median(fd.get(wd, [0])) if fd.get(wd) else None
        w = statistics.median(wdc.get(wd, [0])) if wdc.get(wd) else None
        e = {"dispatches": len(fd.get(wd, [])), "fetch_kib": f, "write_kib": w}
        if f is not None and ffac:
            e["read_bytes"] = f * 1024 * ffac
            e["read_over_weight_bytes"] = e["read_bytes"] / WEIGHT_BYTES[wd]
        if w is not None and wfac:
            e["write_bytes"] = w * 1024 * wfac
        out["kernels"][f"decode_kernel<{wd}>"] = e
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="summaries of rocprofv3 output")
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("dir", type=Path)
    t.add_argument("--matvec-blocks", metavar="WTYPE")
    t.add_argument("--decode", action="store_true")
    t.add_argument("--skip", type=int, default=0, help="decode: drop each weight type's first N steps")
    t.add_argument("--take", type=int, default=0, help="decode: then keep N steps (0 = all)")
    t.add_argument("--bench-legs", metavar="STEPS,WARMUP",
                   help="split bench.py's decode launches (run with --steps STEPS --warmup WARMUP) into its legs")
    t.add_argument("--graph-runs", help="comma-separated labels of cudallm_amd.graphbench's runs, in order")
    t.add_argument("--steps", type=int, default=256, help="graph runs: timed steps per run")
    t.add_argument("--prompt", type=int, default=16, help="graph runs: untimed prompt steps before each run")
    c = sub.add_parser("counters")
    c.add_argument("fetch_dir", type=Path)
    c.add_argument("write_dir", type=Path)
    c.add_argument("--calib-bytes", type=int, default=1 << 30)
    args = ap.parse_args(argv)
    if args.cmd == "trace":
        rows = _rows(args.dir, "kernel_trace.csv")
        res = {}
        if args.matvec_blocks:
            res["matvec"] = matvec_blocks(rows, args.matvec_blocks)
        if args.decode:
            res["decode"] = decode_stats(rows, args.skip, args.take)
        if args.bench_legs:
            k, w = (int(v) for v in args.bench_legs.split(","))
            res["bench_legs"] = bench_legs(rows, k, w)
        if args.graph_runs:
            res["graph_runs"] = graph_runs(rows, args.graph_runs.split(","), args.steps, args.prompt)
    else:
        res = counters(args.fetch_dir, args.write_dir, args.calib_bytes)
    print(json.dumps(res, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
