"""End-to-end decode benchmark suites (the reference's bench/bench_decode.py:12-26 and its C++ runner
src/tools/cudallm_bench.cpp:41-125), driven through this library's C ABI.

    python -m cudallm_amd.bench_decode --suite {ablation,quant,context,tg,long,all} [--names A0_naive,...]
                                        [--model-dir DIR] [--out DIR]
    python -m cudallm_amd.bench_decode --table DIR      # the runs saved by --out DIR, as a markdown table

Each run decodes `prompt_len` prompt tokens (the reference's prompt: 128000, then (i*7919) % 120000 + 1000),
then times `gen` greedy steps with the device drained on both sides, `warmup` + `reps` times; the record
follows cudallm_bench's JSON (decode_tok_s per rep, medians, bytes per token = weight bytes + the average
KV bytes of the timed steps, achieved GB/s) plus `pct_of_peak` against 8 TB/s.  The models are the seeded
synthetic Llama-3.2-1B-shaped files of cudallm_amd.synth (written on first use), not a checkpoint.
"""
import argparse
import json
import statistics
import time
from pathlib import Path

PEAK_GBPS = 8000.0  # MI355X HBM3E

# (name, dtype, matvec, attn, fuse, graph, prompt_len, gen, reps): bench/bench_decode.py:12-26
ABLATION = [
    ("A0_naive", "bf16", "naive", "naive", 0, 0, 128, 256, 5),
    ("A1_matvec_opt", "bf16", "opt", "naive", 0, 0, 128, 256, 5),
    ("A2_attn_opt", "bf16", "opt", "opt", 0, 0, 128, 256, 5),
    ("A3_fused", "bf16", "opt", "opt", 1, 0, 128, 256, 5),
    ("A4_graph_nofuse", "bf16", "opt", "opt", 0, 1, 128, 256, 5),
    ("A5_full", "bf16", "opt", "opt", 1, 1, 128, 256, 5),
]
QUANT = [(f"Q_{d}", d, "opt", "opt", 1, 1, 128, 256, 5) for d in ("bf16", "int8", "int4")]
CONTEXT = [run_ for c in (128, 512, 1024, 2048, 4000)
           for run_ in ((f"ctx_opt_{c}", "bf16", "opt", "opt", 1, 1, c, 32, 3),
                        (f"ctx_naiveattn_{c}", "bf16", "opt", "naive", 1, 1, c, 32, 3))]
TG = [(f"tg_{d}", d, "opt", "opt", 1, 1, 1, 256, 5) for d in ("bf16", "int8", "int4")]
# Beyond the reference's suites: context 8000 on files whose header allows 8192 positions, where the KV
# cache (262 MB per token at int4's 637 MB of weights) is a large part of each step's bytes.
LONG = [(f"long_{d}_8000", d, "opt", "opt", 1, 1, 8000, 32, 2) for d in ("bf16", "int8", "int4")]
SUITES = {"ablation": ABLATION, "quant": QUANT, "context": CONTEXT, "tg": TG, "long": LONG}
LONG_MAX_SEQ = 8192


def prompt_token(i: int) -> int:
    """src/tools/cudallm_bench.cpp:24."""
    return 128000 if i == 0 else (i * 7919) % 120000 + 1000


def model_path(model_dir: Path, dtype: str, max_seq_len: int = 4096) -> Path:
    from . import synth
    p = Path(model_dir) / f"synth_seed1_{dtype}_ctx{max_seq_len}.cudallm"
    if not p.exists():
        Path(model_dir).mkdir(parents=True, exist_ok=True)
        synth.write_model(p, dtype, seed=1, max_seq_len=max_seq_len)
    return p


def bench(path, prompt_len: int, gen: int, reps: int, warmup: int = 1, matvec: str = "opt", attn: str = "opt",
          fuse: int = 1, graph: int = 1, rpb: int = 0) -> dict:
    """One cudallm_bench run (src/tools/cudallm_bench.cpp:41-125)."""
    import torch
    from . import engine as E
    with E.Engine(path, matvec=matvec, attn=attn, fuse=bool(fuse), cuda_graph=bool(graph), matvec_rpb=rpb) as eng:
        c = eng.config
        if prompt_len + gen > c["max_seq_len"]:
            raise ValueError("prompt_len + gen exceeds max_seq_len")
        tok_s, ms = [], []
        for r in range(warmup + reps):
            eng.reset()
            for i in range(prompt_len):
                eng.step_async(prompt_token(i))
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(gen):
                eng.step_async(None)
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
            if r >= warmup:
                tok_s.append(gen / dt)
                ms.append(1e3 * dt / gen)
        weight_bytes = c["weight_bytes"]
        kv = c["n_layers"] * 2 * c["n_kv_heads"] * c["head_dim"] * 2 * (prompt_len + (gen + 1) // 2)
    bpt = weight_bytes + kv
    med = statistics.median(tok_s)
    gbps = bpt * med / 1e9
    return {"tool": "cudallm_bench", "model": str(path), "weight_dtype": {1: "bf16", 3: "int8", 4: "int4"}.get(
                c["weight_dtype"], str(c["weight_dtype"])),
            "options": {"matvec": matvec, "attn": attn, "fuse": int(fuse), "graph": int(graph), "rpb": rpb},
            "prompt_len": prompt_len, "gen": gen, "reps": reps, "decode_tok_s": tok_s, "decode_tok_s_median": med,
            "ms_per_token_median": statistics.median(ms), "weight_bytes": weight_bytes,
            "kv_bytes_per_token_avg": kv, "bytes_per_token": bpt, "achieved_gbps_median": gbps,
            "gpu_name": torch.cuda.get_device_name(0), "pct_of_peak": 100.0 * gbps / PEAK_GBPS}


def markdown_table(out_dir: Path) -> str:
    """The runs saved under out_dir (--out) as one markdown table in suite order, then the context-scaling ratios
    (long_*_8000 against tg_* of the same weight type, ctx_opt_4000 against ctx_opt_128) where both runs are there."""
    recs = {}
    for suite in SUITES:
        for name, *_ in SUITES[suite]:
            f = out_dir / suite / f"{name}.json"
            if f.exists():
                recs[name] = (suite, json.loads(f.read_text()))
    lines = ["| suite | run | weights | options | prompt | gen | tok/s | ms/token | GB/s | % of 8 TB/s |",
             "|---|---|---|---|---|---|---|---|---|---|"]
    for name, (suite, r) in recs.items():
        o = r["options"]
        lines.append(f"| {suite} | {name} | {r['weight_dtype']} | {o['matvec']}/{o['attn']} fuse={o['fuse']} "
                     f"graph={o['graph']} | {r['prompt_len']} | {r['gen']} | {r['decode_tok_s_median']:.1f} | "
                     f"{r['ms_per_token_median']:.3f} | {r['achieved_gbps_median']:.0f} | {r['pct_of_peak']:.1f} |")
    tok = {n: r["decode_tok_s_median"] for n, (_, r) in recs.items()}
    ratios = [(f"long_{w}_8000", f"tg_{w}") for w in ("bf16", "int8", "int4")] + [("ctx_opt_4000", "ctx_opt_128")]
    notes = [f"* {a}: {tok[a]:.1f} tok/s, {100 * (1 - tok[a] / tok[b]):.1f} % below {b} ({tok[b]:.1f})"
             for a, b in ratios if a in tok and b in tok]
    return "\n".join(lines) + ("\n\n" + "\n".join(notes) if notes else "") + "\n"


def main() -> None:
    ap = argparse.ArgumentParser(description="cudallm decode benchmark suites")
    ap.add_argument("--suite", choices=(*SUITES, "all"))
    ap.add_argument("--table", metavar="DIR", help="print the runs saved under DIR (an earlier --out) as markdown")
    ap.add_argument("--names", default="", help="comma-separated subset of run names (default: the whole suite)")
    ap.add_argument("--model-dir", default="/dev/shm/cudallm_models")
    ap.add_argument("--out", default="", help="directory for one JSON file per run (suite/name.json)")
    args = ap.parse_args()
    if args.table:
        print(markdown_table(Path(args.table)), end="")
        return
    if not args.suite:
        ap.error("--suite is required (or --table DIR)")
    wanted = {n for n in args.names.split(",") if n}
    suites = list(SUITES) if args.suite == "all" else [args.suite]
    known = {e[0] for s in suites for e in SUITES[s]}
    if wanted - known:
        raise SystemExit(f"unknown run names for suite {args.suite}: {sorted(wanted - known)}")
    for suite in suites:
        for name, dtype, mv, at, fuse, graph, plen, gen, reps in SUITES[suite]:
            if wanted and name not in wanted:
                continue
            ms = LONG_MAX_SEQ if plen + gen > 4096 else 4096
            rec = bench(model_path(Path(args.model_dir), dtype, ms), plen, gen, reps, 1, mv, at, fuse, graph)
            rec["name"] = name
            print(f"{suite:8s} {name:22s} {rec['weight_dtype']:5s} prompt {plen:5d} gen {gen:4d}: "
                  f"{rec['decode_tok_s_median']:8.1f} tok/s  {rec['ms_per_token_median']:7.3f} ms/token  "
                  f"{rec['achieved_gbps_median']:7.1f} GB/s  ({rec['pct_of_peak']:.1f} % of 8 TB/s)", flush=True)
            if args.out:
                d = Path(args.out) / suite
                d.mkdir(parents=True, exist_ok=True)
                (d / f"{name}.json").write_text(json.dumps(rec, indent=1) + "\n")


if __name__ == "__main__":
    main()
