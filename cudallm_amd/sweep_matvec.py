"""Rows-per-block sweep of the opt matvec (the reference's bench/sweep_matvec.py:1-48) on gfx950.

    python -m cudallm_amd.sweep_matvec [--iters 200] [--out results/sweep_matvec.json]

For each weight type and rpb in 1, 2, 4, 8 (rows whose loads are in flight before the first is multiplied; on gfx950
that is R x 4 KiB bf16, 2 KiB int8 or 1 KiB int4 per 256-thread workgroup), times the five model shapes
(cudallm_amd.kernelbench --op shapes) and picks the rpb with the lowest weighted_us, ties going to the smaller rpb.
The record follows the reference's schema; it also lists each shape's fastest rpb (lowest mean kernel time) and the
library's default rpb per shape, which the library picks per weight type and shape class.
"""
import argparse
import json
import subprocess
import sys
from pathlib import Path

from .kernelbench import RPBS, SHAPES, bench_shapes, default_rpb

WTYPES = ("bf16", "int8", "int4")


def pick_winners(weighted: dict) -> dict:
    """weighted[wt][rpb] -> {wt: rpb with the lowest value}; ties go to the smaller rpb (sweep_matvec.py:29-31)."""
    return {wt: min(sorted(per), key=lambda r: per[r]) for wt, per in weighted.items()}


def shape_winners(data: dict) -> dict:
    """data[wt][str(rpb)] (bench_shapes records) -> {wt: {shape: rpb with the lowest mean kernel time}}; ties go to
    the smaller rpb."""
    out = {}
    for wt, per in data.items():
        best = {}
        for r in sorted(per, key=int):
            for row in per[r]["results"]:
                if row["name"] not in best or row["avg_us"] < best[row["name"]][1]:
                    best[row["name"]] = (int(r), row["avg_us"])
        out[wt] = {n: rb for n, (rb, _) in best.items()}
    return out


def git_commit() -> str:
    root = Path(__file__).resolve().parents[1]
    try:
        commit = subprocess.run(["git", "rev-parse", "--short", "HEAD"], check=True, capture_output=True, text=True,
                                cwd=root).stdout.strip()
        dirty = subprocess.run(["git", "status", "--porcelain"], check=True, capture_output=True, text=True,
                               cwd=root).stdout.strip()
    except (OSError, subprocess.CalledProcessError):
        return "unknown"
    return commit + ("-dirty" if dirty else "")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="rpb sweep of the opt matvec")
    ap.add_argument("--iters", type=int, default=200)
    ap.add_argument("--wtypes", default=",".join(WTYPES))
    ap.add_argument("--out", type=Path, default=Path("results/sweep_matvec.json"))
    args = ap.parse_args(argv)
    import torch
    wtypes = [w for w in args.wtypes.split(",") if w]
    data = {wt: {str(r): bench_shapes(wt, r, args.iters) for r in RPBS} for wt in wtypes}
    weighted = {wt: {r: data[wt][str(r)]["weighted_us"] for r in RPBS} for wt in wtypes}
    winners = pick_winners(weighted)
    rec = {"tool": "sweep_matvec", "results": data, "winners": winners,
           "weighted_us": {wt: {str(r): v for r, v in per.items()} for wt, per in weighted.items()},
           "shape_winners": shape_winners(data),
           "default_rpb": {wt: {n: default_rpb(wt, ep, r, c) for n, r, c, ep, _ in SHAPES} for wt in wtypes},
           "git_commit": git_commit(),
           "gpu_name": torch.cuda.get_device_name(0)}
    args.out.parent.mkdir(parents=True, exist_ok=True)
    args.out.write_text(json.dumps(rec, indent=2) + "\n")
    print(f"saved {args.out}")
    for wt in wtypes:
        per = "  ".join(f"rpb {r}: {weighted[wt][r]:8.2f}" for r in RPBS)
        print(f"winner {wt}: rpb={winners[wt]} weighted_us={weighted[wt][winners[wt]]:.2f}   ({per})", flush=True)
        for n, r, c, ep, _ in SHAPES:
            print(f"  {wt} {n}: fastest rpb {rec['shape_winners'][wt][n]}, library default rpb "
                  f"{default_rpb(wt, ep, r, c)}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
