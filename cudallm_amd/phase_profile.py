"""Per-phase timeline of the persistent decode kernel (cudallm_step_profile), per weight type.

    python -m cudallm_amd.phase_profile [--dtypes bf16,int8,int4] [--ctx 40] [--reps 5] [--out FILE.md]

Writes a seeded synthetic Llama-3.2-1B-shaped file per weight type, decodes to context `ctx`, then records
`reps` profiled steps and keeps the last one.  Each workgroup stamps the GPU's 100 MHz clock when it
finishes each phase; a phase's time is the median (over workgroups) end of that phase minus the median
end of the phase before it, so a phase's figure includes the wait for its input.  For layer 1 the table
also splits each phase into "input arrived" (the handoff), "prologue done" (the input is in registers or in
the digit table) and the rows, and gives the spread of phase ends over workgroups (the skew the next handoff
waits for).
"""
import argparse
import sys
import tempfile
from pathlib import Path

import numpy as np

PHASES = ["qkv", "attention", "merge", "wo", "gate_up", "down"]


def max_seq_for(ctx: int) -> int:
    """The engine's context: 4096, or the next multiple of 4096 that holds ctx."""
    return max(4096, -(-(ctx + 1) // 4096) * 4096)


def profile(path, ctx: int, reps: int):
    from . import engine as E
    with E.Engine(path, max_seq_len=max_seq_for(ctx)) as eng:
        eng.step_async(128000)
        for _ in range(ctx - 2):
            eng.step_async(None)
        stamps = None
        for _ in range(reps):
            eng.reset()
            eng.step_async(128000)
            for _ in range(ctx - 2):
                eng.step_async(None)
            stamps = eng.step_profile(None).astype(np.int64)
    return stamps


ATTN_SLOT = 112  # kAttnSteps in decode.hip


def summarise(wd: str, S: np.ndarray, ctx: int) -> list[str]:
    G = S.shape[0]
    rel = (S - S[:, 0].min()) / 100.0  # microseconds
    lines = [f"### {wd}: grid {G}, context {ctx}", ""]
    total = {p: 0.0 for p in PHASES}
    prev = np.median(rel[:, 0])
    for l in range(16):
        for k, p in enumerate(PHASES):
            e = np.median(rel[:, 1 + 6 * l + k])
            total[p] += e - prev
            prev = e
    lm_end = float(np.median(rel[:, 97]))
    argmax_end = float(rel[0, 98])
    layers = prev - np.median(rel[:, 0])
    lines += ["| phase (input wait included) | sum over 16 layers, us | per layer, us |", "|---|---|---|"]
    for p in PHASES:
        lines.append(f"| {p} | {total[p]:.1f} | {total[p] / 16:.2f} |")
    lines.append(f"| layers | {layers:.1f} | {layers / 16:.2f} |")
    lines.append(f"| lm_head (final norm, argmax folded in) | {lm_end - prev:.1f} | |")
    lines.append(f"| final argmax (workgroup 0) | {argmax_end - lm_end:.1f} | |")
    lines.append(f"| **step** | **{argmax_end:.1f}** | |")
    lines += ["", "Layer 1, per phase (us after the previous phase's median end): input arrived (median over "
                  "workgroups that stamp it), phase end median, and the spread of phase ends (p10 / max - median).", "",
              "| phase | input arrived | prologue done | end (median) | end p10 | end max |", "|---|---|---|---|---|---|"]
    pe = np.median(rel[:, 6])  # layer 0 down end
    for k, p in enumerate(PHASES):
        e = rel[:, 7 + k]
        med = np.median(e)
        inp = pro = ""
        if k in (0, 1, 3, 4, 5):
            a = rel[:, 100 + 2 * k]
            a = a[S[:, 100 + 2 * k] > 0]
            if a.size:
                inp = f"+{np.median(a) - pe:.2f}"
            b = rel[:, 101 + 2 * k]
            b = b[S[:, 101 + 2 * k] > 0]
            if b.size:
                pro = f"+{np.median(b) - pe:.2f}"
        lines.append(f"| {p} | {inp} | {pro} | +{med - pe:.2f} | {np.percentile(e, 10) - med:+.2f} | "
                     f"{e.max() - med:+.2f} |")
        pe = med
    # Inside the first attention task of layer 1 (the workgroups that run one): when it started (K/V tile loads
    # issued), had q (and the current k, v), passed its barrier, had the scores, had stored its output, and left.
    steps = ["task start", "q, k, v arrived", "barrier passed", "scores, softmax", "output stored", "task end"]
    att = S[:, ATTN_SLOT:ATTN_SLOT + len(steps)]
    who = np.all(att > 0, axis=1)
    if who.any():
        qkv_end = np.median(rel[:, 7])
        lines += ["", f"Layer 1's first attention task ({int(who.sum())} workgroups), us after qkv's median end:", "",
                  "| step | median | max |", "|---|---|---|"]
        for k, name in enumerate(steps):
            t = rel[who, ATTN_SLOT + k] - qkv_end
            lines.append(f"| {name} | {np.median(t):+.2f} | {t.max():+.2f} |")
    return lines + [""]


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="per-phase timeline of the persistent decode kernel")
    ap.add_argument("--dtypes", default="bf16,int8,int4")
    ap.add_argument("--ctx", type=int, default=40)
    ap.add_argument("--reps", type=int, default=5)
    ap.add_argument("--out", type=Path)
    ap.add_argument("--raw", type=Path, help="also save each weight type's stamps as RAW/stamps_<dtype>.npy")
    args = ap.parse_args(argv)
    from . import synth
    out = []
    with tempfile.TemporaryDirectory(dir="/dev/shm" if Path("/dev/shm").is_dir() else None) as d:
        for wd in args.dtypes.split(","):
            path = Path(d) / f"profile_{wd}.cudallm"
            synth.write_model(path, wd, seed=1234, max_seq_len=max_seq_for(args.ctx))
            S = profile(path, args.ctx, args.reps)
            if args.raw:
                args.raw.mkdir(parents=True, exist_ok=True)
                np.save(args.raw / f"stamps_{wd}.npy", S)
            block = summarise(wd, S, args.ctx)
            print("\n".join(block), flush=True)
            out += block
            path.unlink()
    if args.out:
        args.out.parent.mkdir(parents=True, exist_ok=True)
        args.out.write_text("\n".join(out) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
