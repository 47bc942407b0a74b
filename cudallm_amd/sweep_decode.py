"""Launch-parameter sweep of the persistent decode kernel (the reference's bench/sweep_matvec.py, retargeted at the
knobs the default path actually has).

    python -m cudallm_amd.sweep_decode build [--out-dir cudallm_amd/_sweep] [--jobs 8]
    python -m cudallm_amd.sweep_decode run [--out-dir cudallm_amd/_sweep] [--steps 128] [--json PATH] [--md PATH]

The knobs (compile-time constants of csrc/kernels/decode.hip):
  CLLM_LOADER_LINES      lines (1 KiB loads) in flight per loader wave            default 16
  CLLM_RING_SLOTS_BF16   LDS ring slots per compute wave, bf16 weights            default 24 (30 fit)
  CLLM_RING_SLOTS_QUANT  LDS ring slots per compute wave, int8 weights             default 22
  CLLM_RING_SLOTS_INT4   LDS ring slots per compute wave, int4 weights             default 20
  CLLM_LM_ROWS_BF16      lm_head rows per unit of work, bf16 weights               default 2
  CLLM_LM_ROWS_INT8      lm_head rows per unit of work, int8 weights               default 8
  CLLM_LM_ROWS_QUANT     lm_head rows per unit of work, int4 weights               default 8
(the kernel's int4 ring and int8 lm_head units fall back to the QUANT values when their own knob is not given; the
sweep always gives every knob.)
``build`` compiles one library per configuration (one knob moved from the default at a time) into OUT_DIR/NAME/;
a configuration whose LDS does not fit fails to build and is reported as such.  ``run`` (on the GPU) times each
library with bench.py's decode leg (CUDALLM_LIB selects the library) and reports the decode kernel's microseconds
per step for every weight type; the winner per weight type is the fastest.
"""
import argparse
import json
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
DEFAULTS = {"CLLM_LOADER_LINES": 16, "CLLM_RING_SLOTS_BF16": 24, "CLLM_RING_SLOTS_QUANT": 22, "CLLM_RING_SLOTS_INT4": 20,
            "CLLM_LM_ROWS_BF16": 2, "CLLM_LM_ROWS_INT8": 8, "CLLM_LM_ROWS_QUANT": 8}
# One knob at a time around the defaults.
MOVES = {"CLLM_LOADER_LINES": (12, 20), "CLLM_RING_SLOTS_BF16": (22, 26, 30), "CLLM_RING_SLOTS_QUANT": (20,),
         "CLLM_RING_SLOTS_INT4": (18, 22), "CLLM_LM_ROWS_BF16": (1, 4), "CLLM_LM_ROWS_INT8": (4,),
         "CLLM_LM_ROWS_QUANT": (4,)}


def configs() -> dict:
    out = {"default": dict(DEFAULTS)}
    for knob, values in MOVES.items():
        for v in values:
            c = dict(DEFAULTS)
            c[knob] = v
            out[f"{knob.removeprefix('CLLM_').lower()}_{v}"] = c
    return out


def build(out_dir: Path, jobs: int) -> dict:
    status = {}
    for name, cfg in configs().items():
        d = out_dir / name
        defs = " ".join(f"-D{k}={v}" for k, v in cfg.items())
        cmd = ["make", "-C", str(PKG), f"-j{jobs}", f"BUILD={d / '_build'}", f"LIB={d / 'libcudallm.so'}",
               f"EXTRA_DEFS={defs}"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        ok = r.returncode == 0 and (d / "libcudallm.so").is_file()
        status[name] = {"config": cfg, "built": ok}
        if not ok:
            status[name]["error"] = (r.stderr or r.stdout).strip().splitlines()[-3:]
        print(f"[sweep] build {name}: {'ok' if ok else 'failed'}", flush=True)
    (out_dir / "build.json").write_text(json.dumps(status, indent=1))
    return status


def run(out_dir: Path, steps: int, warmup: int) -> dict:
    status = json.loads((out_dir / "build.json").read_text())
    results = {}
    for name, st in status.items():
        if not st["built"]:
            results[name] = {"config": st["config"], "error": "does not build (LDS or registers do not fit)"}
            continue
        env = dict(os.environ, CUDALLM_LIB=str(out_dir / name / "libcudallm.so"))
        cmd = [sys.executable, "-u", str(ROOT / "bench.py"), "--no-cpu", "--no-kernels", "--no-config5", "--no-peak",
               "--steps", str(steps), "--warmup", str(warmup)]
        r = subprocess.run(cmd, capture_output=True, text=True, env=env, timeout=600)
        if r.returncode != 0:
            results[name] = {"config": st["config"], "error": r.stderr.strip().splitlines()[-3:]}
            print(f"[sweep] run {name}: failed", flush=True)
            continue
        rec = json.loads(r.stdout.strip().splitlines()[-1])
        us = {wd: v["kernel_avg_us"] for wd, v in rec["decode"].items()}
        results[name] = {"config": st["config"], "kernel_us": us}
        print(f"[sweep] run {name}: " + ", ".join(f"{wd} {u:.1f} us" for wd, u in us.items()), flush=True)
    return results


def report(results: dict) -> str:
    lines = ["| configuration | loader lines | ring slots bf16 | ring slots int8 | ring slots int4 | lm_head rows bf16 | "
             "lm_head rows int8 | lm_head rows int4 | bf16 us | int8 us | int4 us |",
             "|---|---|---|---|---|---|---|---|---|---|---|"]
    best = {}
    for name, r in results.items():
        c = r["config"]
        if "kernel_us" in r:
            u = r["kernel_us"]
            cells = [f"{u.get(wd, float('nan')):.1f}" for wd in ("bf16", "int8", "int4")]
            for wd, v in u.items():
                if wd not in best or v < best[wd][1]:
                    best[wd] = (name, v)
        else:
            cells = ["-", "-", "-"]
        lines.append(f"| {name} | {c['CLLM_LOADER_LINES']} | {c['CLLM_RING_SLOTS_BF16']} | "
                     f"{c['CLLM_RING_SLOTS_QUANT']} | {c['CLLM_RING_SLOTS_INT4']} | {c['CLLM_LM_ROWS_BF16']} | "
                     f"{c['CLLM_LM_ROWS_INT8']} | {c['CLLM_LM_ROWS_QUANT']} | " + " | ".join(cells) + " |")
    lines.append("")
    for wd, (name, v) in sorted(best.items()):
        lines.append(f"* fastest for {wd}: {name} ({v:.1f} us per step)")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="sweep of the persistent decode kernel's build-time knobs")
    ap.add_argument("cmd", choices=("build", "run"))
    ap.add_argument("--out-dir", type=Path, default=PKG / "_sweep")
    ap.add_argument("--jobs", type=int, default=min(16, os.cpu_count() or 1))
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--json", type=Path)
    ap.add_argument("--md", type=Path)
    args = ap.parse_args(argv)
    args.out_dir.mkdir(parents=True, exist_ok=True)
    if args.cmd == "build":
        build(args.out_dir, args.jobs)
        return 0
    res = run(args.out_dir, args.steps, args.warmup)
    text = report(res)
    print(text, flush=True)
    if args.json:
        args.json.write_text(json.dumps(res, indent=1))
    if args.md:
        args.md.write_text(text + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
