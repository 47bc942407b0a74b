"""Batch-1 decode benchmark on one MI355X (the reference's headline run: 16-token prompt + 256 greedy
tokens; kernel lines for its matvec and attention cases).

    python bench.py [--gpus 1] [--steps 256] [--warmup 16] [--dtypes bf16,int8,int4] [--no-cpu]

A "step" is one batch-1 decode step (one token) of a seeded random-init Llama-3.2-1B-shaped model:
16 layers, hidden 2048, FFN 8192, vocab 128256, GQA 32/8, tied embeddings, weights N(0, 0.02)
(bf16 master; int8 per-row and int4 group-128 files quantised from it).  Per weight type: W untimed
warm-up steps on a sequence of their own, then a reset, the 16-token seeded prompt, and K greedy decode
steps timed with the device drained on both sides (positions 17 .. 16 + K: with K = 256 this is BASELINE's
full-decode configuration, 16-token prompt + 256 greedy tokens); each step is one launch of the persistent
decode kernel with the token fed back on the device (no host sync inside the timed region, as reference
src/tools/cudallm_bench.cpp:64-80).  The run fails (exit 3) if an engine is not running the persistent kernel,
so a line never names a kernel that did not run.

Printed last, on one line: the JSON record.  ``value`` is bf16 decode tok/s; ``decode`` holds all
three weight types; ``roofline`` is the dominant kernel, the persistent decode kernel (one launch
per token), timed live with HIP events recorded on the engine's stream around the K timed steps,
with bytes per launch = weight bytes + the KV bytes the step reads, and ``traffic`` from the
committed rocprofv3 counter summary (profiles/hbm_traffic.json); ``matvec_roofline`` is the
standalone fused RMSNorm + gate_up + SwiGLU matvec over rotating weight copies (> 1 GiB, so the
256 MB Infinity Cache cannot serve them), with each weight type's lm_head and, beside each, the time
the bandwidth kernel takes to read the same weight bytes; ``cpu_baseline`` is the CPU oracle (the reference's
algorithm restated, oracle/model.py) timed on this host.
"""
import argparse
import json
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from cudallm_amd.kernelbench import SHAPES, bench_matvec, weighted_us  # noqa: E402

METRIC = "batch-1 decode tok/s (bf16/int8/int4) + matvec HBM GB/s as % of peak"
PEAK_HBM = 8.0e12  # MI355X HBM3E, bytes/s
PROMPT = 16
KV_BYTES_PER_POS = 16 * 2 * 8 * 64 * 2  # layers x (K,V) x kv heads x head_dim x fp16


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def prompt_ids(n: int) -> list[int]:
    rng = np.random.default_rng(16)
    return [128000] + [int(t) for t in rng.integers(0, 128256, n - 1)]


class NotPersistent(RuntimeError):
    """An engine ran the multi-kernel step where the benchmark times the persistent decode kernel."""


def bench_decode(path, wd: str, steps: int, warmup: int, torch) -> dict:
    from cudallm_amd import engine as E
    t_load = time.perf_counter()
    with E.Engine(path) as eng:
        load_s = time.perf_counter() - t_load
        kind, grid = eng.step_kind
        if kind != "persistent":
            raise NotPersistent(f"{wd}: the engine runs the multi-kernel step, not decode_kernel<{wd}>")
        weight_bytes = eng.config["weight_bytes"]
        ids = prompt_ids(PROMPT)
        eng.reset()  # warm-up on a sequence of its own
        for t in ids:
            eng.step_async(t)
        for _ in range(warmup):
            eng.step_async(None)
        eng.reset()  # then the timed sequence: the prompt, and `steps` greedy steps from position 17 on
        for t in ids[:-1]:
            eng.step_async(t)
        eng.step(ids[-1])  # the last prompt step returns its output: the stream is drained here
        torch.cuda.synchronize()
        # HIP events on the engine's own stream, where each step is one launch of the decode kernel.
        es = torch.cuda.ExternalStream(eng.stream)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        ev0.record(es)
        for _ in range(steps):
            eng.step_async(None)
        ev1.record(es)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        ev_us = ev0.elapsed_time(ev1) * 1e3 / steps
        nxt, _ = eng.step(None)
    ctx0 = PROMPT + 1  # the first timed step attends over 17 positions
    kv = KV_BYTES_PER_POS * (PROMPT + (steps + 1) // 2)  # reference cudallm_bench.cpp:82-85 accounting
    bpt = weight_bytes + kv
    tok_s = steps / dt
    return {"tok_s": tok_s, "ms_per_token": 1e3 * dt / steps, "weight_bytes": weight_bytes, "bytes_per_token": bpt,
            "gbps": bpt * tok_s / 1e9, "frac_of_8tbs": bpt * tok_s / PEAK_HBM,
            "roofline_tok_s": PEAK_HBM / bpt, "context": [ctx0, ctx0 + steps - 1], "load_s": round(load_s, 2),
            "last_token": nxt, "kernel_avg_us": ev_us, "kernel_gbps": bpt / ev_us / 1e3,
            "step_kind": kind, "grid": grid}


def bench_config5(path, reps: int = 5, warmup: int = 1, prompt: int = PROMPT, gen: int = 256) -> dict:
    """The headline run (16-token prompt, 256 greedy tokens) timed the way reference
    src/tools/cudallm_bench.cpp:64-85 times it: per rep, reset, the prompt, a drained stream, then `gen` greedy
    steps (token -1, no host sync) timed to the drained end; the median tok/s over `reps` reps after `warmup`
    untimed reps.  Bytes per token = weight bytes + 32768 (prompt + ceil(gen/2))."""
    from cudallm_amd import engine as E
    ids = prompt_ids(prompt)
    rates = []
    with E.Engine(path, max_seq_len=4096) as eng:
        if not eng.persistent:
            raise NotPersistent("config 5: the engine runs the multi-kernel step, not the persistent kernel")
        weight_bytes = eng.config["weight_bytes"]
        for r in range(warmup + reps):
            eng.reset()
            for t in ids[:-1]:
                eng.step_async(t)
            eng.step(ids[-1])  # the last prompt step returns its output, so the stream is drained here
            t0 = time.perf_counter()
            for _ in range(gen - 1):
                eng.step_async(None)
            eng.step(None)  # the gen-th greedy step, and the drain
            dt = time.perf_counter() - t0
            if r >= warmup:
                rates.append(gen / dt)
    bpt = weight_bytes + KV_BYTES_PER_POS * (prompt + (gen + 1) // 2)
    med = float(np.median(rates))
    return {"tok_s": med, "reps": reps, "prompt": prompt, "gen": gen, "bytes_per_token": bpt,
            "gbps": bpt * med / 1e9, "frac_of_8tbs": bpt * med / PEAK_HBM, "all_tok_s": [round(r, 2) for r in rates]}


TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic.json"


def traffic_bytes(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter summary: FETCH_SIZE and
    WRITE_SIZE (KiB per dispatch), each scaled by what the same counter read for a device copy of
    known size.  None when the summary has no entry for the kernel."""
    try:
        t = json.loads(TRAFFIC_FILE.read_text())
        k, c = t["kernels"][kernel], t["copy_calibration"]
    except (OSError, KeyError, ValueError):
        return None
    f_fac = c["bytes"] / (c["fetch_kib"] * 1024.0)
    w_fac = c["bytes"] / (c["write_kib"] * 1024.0)
    return round(k["fetch_kib"] * 1024.0 * f_fac + k["write_kib"] * 1024.0 * w_fac)


def copy_calibration(mib: int, torch) -> None:
    """Three device copies of `mib` MiB, so a counter run can scale its byte counters."""
    a = torch.empty(mib << 20, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    del a, b
    torch.cuda.empty_cache()


def cpu_baseline(path, budget_s: float) -> dict:
    """The reference's CPU path (restated in oracle/model.py: fp32 dequantise per matmul, fp16 KV
    cache) decoding the same bf16 model on this host, for about `budget_s` seconds."""
    import torch
    from oracle.model import OracleModel
    cores = min(16, os.cpu_count() or 1)
    m = OracleModel(path, cache_dense=False, threads=cores)
    ids = prompt_ids(PROMPT)
    logits, _ = m.step(ids[0])  # warm-up (page cache, allocator)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s and n < 256:
        # The prompt, then greedy tokens: the same sequence shape as the GPU leg.
        tok = ids[n + 1] if n + 1 < len(ids) else int(torch.argmax(logits))
        logits, _ = m.step(tok)
        n += 1
    dt = time.perf_counter() - t0
    return {"value": n / dt, "unit": "tok/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{n} bf16 decode steps (positions 1..{n}: prompt, then greedy) of the same synthetic model by "
                      f"the oracle (torch fp32 on the host, weights dequantised per matmul), {dt:.1f} s",
            "host": host_description()}


def host_description() -> dict:
    """The host the CPU baseline ran on: core counts and the CPU model."""
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"os_cpu_count": os.cpu_count(), "sched_getaffinity": len(os.sched_getaffinity(0)), "cpu_model": model}


def cpu_matvec_config1(reps: int = 20) -> dict:
    """The reference's int8 8192x2048 matvec case on the CPU: dequantised to fp32 then W @ x (reference.py:33-37)."""
    import torch
    from oracle import quantize as Q
    rng = np.random.default_rng(1)
    w = Q.bf16_bits_to_f32(Q.bf16_round_bits(rng.normal(0, 0.02, size=(8192, 2048)).astype(np.float32)))
    q, s = Q.quantize_int8_rows(w)
    tq, ts = torch.from_numpy(q), torch.from_numpy(s)
    x = torch.from_numpy(rng.standard_normal(2048).astype(np.float32))
    times = []
    for i in range(reps + 3):
        t0 = time.perf_counter()
        _ = (tq.float() * ts[:, None]) @ x
        if i >= 3:
            times.append(time.perf_counter() - t0)
    us = float(np.median(times)) * 1e6
    return {"us": us, "gbps": 16809984 / us / 1e3, "threads": torch.get_num_threads()}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--dtypes", default="bf16,int8,int4")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-kernels", action="store_true", help="skip the per-shape matvec lines")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-config5", action="store_true", help="skip the config-5 sequence leg")
    ap.add_argument("--no-peak", action="store_true", help="skip the measured stream-read peak")
    ap.add_argument("--model-dir", default=None)
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="first run three device copies of MIB MiB (byte-counter calibration under rocprofv3)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (batch-1 decode does not shard across GPUs here); "
              "run it with --gpus 1", file=sys.stderr)
        return 2
    if PROMPT + max(args.warmup, args.steps) + 1 > 4096:
        print("bench.py: prompt + warmup and prompt + steps must fit the 4096-token context", file=sys.stderr)
        return 2

    import torch
    from cudallm_amd import synth
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    if args.copy_calib:
        copy_calibration(args.copy_calib, torch)
    dtypes = [d for d in args.dtypes.split(",") if d]
    peak = None
    if not args.no_peak:
        from cudallm_amd import engine as E
        best, med = E.measure_read_bandwidth(4 << 30, 10)
        peak = {"best_gbps": round(best, 1), "median_gbps": round(med, 1), "bytes": 4 << 30,
                "method": "stream read of a 4 GiB buffer (> the 256 MB Infinity Cache), best of 10 timed reads "
                          "over a sweep of launch shapes (cudallm_measure_read_bandwidth)"}
        log(f"[bench] measured HBM stream-read peak: best {best:.0f} GB/s, median {med:.0f} GB/s")
    base = args.model_dir or ("/dev/shm" if os.path.isdir("/dev/shm") else None)
    tmp = tempfile.TemporaryDirectory(dir=base)
    paths = {}
    decode = {}
    for wd in dtypes:
        paths[wd] = Path(tmp.name) / f"bench_{wd}.cudallm"
        t0 = time.perf_counter()
        synth.write_model(paths[wd], wd, seed=1234)
        log(f"[bench] wrote {wd} model in {time.perf_counter() - t0:.1f} s")
        try:
            decode[wd] = bench_decode(paths[wd], wd, args.steps, args.warmup, torch)
        except NotPersistent as e:
            print(f"bench.py: {e}; refusing to report it as the persistent kernel's line", file=sys.stderr)
            return 3
        log(f"[bench] decode {wd}: {decode[wd]['tok_s']:.1f} tok/s, {decode[wd]['gbps']:.0f} GB/s "
            f"({100 * decode[wd]['frac_of_8tbs']:.1f} % of 8 TB/s); kernel {decode[wd]['kernel_avg_us']:.1f} us "
            f"by events")
        if not args.no_config5:
            try:
                decode[wd]["config5"] = bench_config5(paths[wd])
            except NotPersistent as e:
                print(f"bench.py: {e}", file=sys.stderr)
                return 3
            c5 = decode[wd]["config5"]
            log(f"[bench] config 5 {wd} (16 + 256, median of {c5['reps']}): {c5['tok_s']:.1f} tok/s, "
                f"{100 * c5['frac_of_8tbs']:.1f} % of 8 TB/s")
        if wd != "bf16" or args.no_cpu:
            paths[wd].unlink()

    head_wd = "bf16" if "bf16" in dtypes else dtypes[0]
    dom = bench_matvec(head_wd, "gate_up", 16384, 2048, "swiglu", True, 400, stream=True)
    dom_gbps = dom["bytes"] / dom["avg_us"] / 1e3
    log(f"[bench] gate_up {head_wd} matvec: kernel {dom['avg_us']:.2f} us, {dom_gbps:.0f} GB/s "
        f"(wall {dom['wall_us_per_launch']:.2f} us per launch; a plain read of its weights {dom['stream_us']:.2f} us)")
    matvecs = []
    if not args.no_kernels:
        for wd in dtypes:
            per = {}
            for name, rows, cols, ep, norm in SHAPES:
                r = bench_matvec(wd, name, rows, cols, ep, norm, 200 if name != "lm_head" else 50, stream=True)
                matvecs.append(r)
                per[name] = r["avg_us"]
            weighted = weighted_us(per)
            matvecs.append({"name": "weighted_us", "wtype": wd, "us": weighted})
            log(f"[bench] {wd} matvec weighted 16*(qkv+wo+gate_up+down)+lm_head = {weighted:.1f} us")

    cpu = None
    if not args.no_cpu and "bf16" in paths and paths["bf16"].exists():
        cpu = cpu_baseline(paths["bf16"], args.cpu_seconds)
        cpu["matvec_config1_int8"] = cpu_matvec_config1()
        log(f"[bench] cpu baseline {cpu['value']:.3f} tok/s on {cpu['cores']} threads")
    tmp.cleanup()

    head = decode[head_wd]
    pk = peak["best_gbps"] if peak else None
    for r in decode.values():
        if pk:
            r["frac_of_measured_peak"] = r["gbps"] / pk
            r["kernel_frac_of_measured_peak"] = r["kernel_gbps"] / pk
            if "config5" in r:
                r["config5"]["frac_of_measured_peak"] = r["config5"]["gbps"] / pk
    for r in matvecs:
        if pk and "bytes" in r:
            r["frac_of_measured_peak"] = r["bytes"] / r["avg_us"] / 1e3 / pk
    rec = {
        "metric": METRIC, "value": round(head["tok_s"], 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(head["ms_per_token"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": head_wd,
        "data": "synthetic: seeded random-init Llama-3.2-1B-shaped weights N(0,0.02), bf16 master",
        "config": {"workload": f"batch-1 greedy decode, {head_wd} weights: 16-token prompt, then {args.steps} timed "
                               f"greedy steps at contexts {head['context'][0]}..{head['context'][1]}, one kernel "
                               f"launch per step ({args.warmup} warm-up steps on a separate sequence)"
                               + (" = BASELINE's full-decode configuration" if args.steps == 256 else
                                  "; BASELINE's full-decode configuration (256 steps) is decode.*.config5"),
                   "model": "llama-3.2-1b-shaped (random init)", "global_batch": 1,
                   "seq_len": PROMPT + args.steps, "parallelism": "none (1 GPU)",
                   "step_kind": f"{head['step_kind']} (grid {head['grid']})"},
        "roofline": {"bound": "hbm", "achieved": round(head["kernel_gbps"], 1), "peak": 8000.0, "unit": "GB/s",
                     "frac": round(head["kernel_gbps"] / 8000.0, 4), "traffic": traffic_bytes(f"decode_kernel<{head_wd}>"),
                     "kernel": f"decode_kernel<{head_wd}> (persistent: the whole decode step is this one launch)",
                     "bytes_per_launch": head["bytes_per_token"], "avg_us": round(head["kernel_avg_us"], 3),
                     "timing": "HIP events on the engine's stream around the timed steps",
                     "traffic_source": TRAFFIC_FILE.name,
                     "measured_peak": pk, "frac_of_measured_peak": round(head["kernel_gbps"] / pk, 4) if pk else None},
        "hbm_read_peak": peak,
        "matvec_roofline": {"kernel": f"matvec_fast<{head_wd}, SWIGLU, norm> gate_up 16384x2048 (standalone)",
                            "achieved": round(dom_gbps, 1), "frac": round(dom["frac_of_8tbs"], 4),
                            "frac_of_measured_peak": round(dom_gbps / pk, 4) if pk else None,
                            "bytes_per_launch": dom["bytes"], "avg_us": round(dom["avg_us"], 3),
                            "stream_read_us": round(dom["stream_us"], 3),
                            "frac_of_stream_read": round(dom["frac_of_stream"], 4),
                            "lm_head": {r["wtype"]: {"avg_us": round(r["avg_us"], 3), "frac": round(r["frac_of_8tbs"], 4),
                                                     "stream_read_us": round(r["stream_us"], 3),
                                                     "frac_of_stream_read": round(r["frac_of_stream"], 4)}
                                        for r in matvecs if r.get("name") == "lm_head"},
                            "timing": "mean kernel duration from dispatch-recorded start/end events, "
                                      "rotating over > 1.5 GiB of weight copies; stream_read_us: the bandwidth "
                                      "kernel reading the same weight bytes on the same copies"},
        "cpu_baseline": cpu,
        "decode": {wd: {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
                   for wd, r in decode.items()},
        "matvec": [{k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()} for r in matvecs],
    }
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
