"""Matvec kernel benchmark through this library's launch hook (the reference's cudallm_kernelbench
--op matvec|shapes, src/tools/cudallm_kernelbench.cpp:115-180,253-298).

    python -m cudallm_amd.kernelbench --op shapes --wtype {bf16,int8,int4} [--rpb 1|2|4|8] [--iters 200] [--json PATH]
                                      [--stream]
    python -m cudallm_amd.kernelbench --op matvec --wtype W --rows R --cols C [--epilogue store|add|swiglu]
                                      [--fuse-norm] [--rpb N] [--iters 200] [--json PATH] [--stream]

Same operands as the reference (weights N(0, 0.02) as bf16, random int8 / packed int4 with scales, x N(0, 1),
norm weights U(0.5, 1.5)), same five model shapes and epilogues, same JSON fields (median_us per launch, GB/s,
weighted_us = 16 (qkv + wo + gate_up + down) + lm_head).  One difference, for MI355X: each launch reads a different
copy of the weights, rotating over more than 1.5 GiB, so that the 256 MB Infinity Cache cannot serve a shape
that the reference's single copy would leave cache-resident.  With --stream, each shape's weight bytes are also read
by the bandwidth kernel over the same copies (stream_us): the time a plain read of those bytes takes at that size.
"""
import argparse
import json
import math
import statistics
import sys
from pathlib import Path

SHAPES = [("qkv", 3072, 2048, "store", True), ("wo", 2048, 2048, "add", False),
          ("gate_up", 16384, 2048, "swiglu", True), ("down", 2048, 8192, "add", False),
          ("lm_head", 128256, 2048, "store", True)]
RPBS = (1, 2, 4, 8)
# The library's choice when rpb = 0 (kDefaultRpb / default_rpb in csrc/kernels/small.hip), and its grid size in
# workgroups per CU (kGridPerCu; 0: as many as can be resident), per weight type and shape class: other, SwiGLU, 8192
# columns, >= 65536 rows.
DEFAULT_RPB = {"bf16": (1, 1, 2, 2), "int8": (4, 2, 4, 4), "int4": (4, 4, 8, 4)}
GRID_PER_CU = {"bf16": (1, 1, 2, 16), "int8": (0, 1, 0, 0), "int4": (0, 1, 0, 2)}


def default_rpb(wd: str, ep: str, rows: int, cols: int) -> int:
    cls = 1 if ep == "swiglu" else 2 if cols >= 8192 else 3 if rows >= 65536 else 0
    return DEFAULT_RPB[wd][cls]
PEAK_GBPS = 8000.0


def matvec_bytes(wd: str, rows: int, cols: int) -> int:
    """Algorithmic HBM bytes of one launch: weights + scales (x and y are < 0.1 %)."""
    n = rows * cols
    if wd == "bf16":
        return 2 * n
    if wd == "int8":
        return n + 4 * rows
    return n // 2 + 2 * rows * (cols // 128)


def bench_matvec(wd: str, name: str, rows: int, cols: int, ep: str, norm: bool, iters: int, rpb: int = 0,
                 rotate_bytes: float = 1.5 * (1 << 30), stream: bool = False) -> dict:
    """Time `iters` launches on torch's current stream, rotating over weight copies totalling at least `rotate_bytes`.
    Each kernel's duration comes from events its own dispatch records at the kernel's start and end.  With `stream`,
    the same copies' weight bytes are also read by the bandwidth kernel (stream_read).  Returns the
    reference's fields (median_us, gbps) plus the mean kernel time (avg_us), the wall time per launch including the
    launch gap, and the copy count."""
    import torch
    from . import engine as E
    dev = torch.device("cuda")
    nbytes = matvec_bytes(wd, rows, cols)
    copies = max(2, math.ceil(rotate_bytes / nbytes))
    g = torch.Generator(device=dev)
    g.manual_seed(rows + cols)
    ws, ss = [], []
    for _ in range(copies):
        if wd == "bf16":
            ws.append((torch.randn(rows, cols, device=dev, generator=g) * 0.02).to(torch.bfloat16))
            ss.append(None)
        elif wd == "int8":
            ws.append(torch.randint(-127, 128, (rows, cols), device=dev, dtype=torch.int8, generator=g))
            ss.append((torch.rand(rows, device=dev, generator=g) + 0.5) / 127.0)
        else:
            ws.append(torch.randint(0, 256, (rows, cols // 2), device=dev, dtype=torch.uint8, generator=g))
            ss.append(((torch.rand(rows, cols // 128, device=dev, generator=g) + 0.5) / 7.0).half())
    x = torch.randn(cols, device=dev, generator=g)
    nw = torch.rand(cols, device=dev, generator=g) + 0.5
    out_rows = rows // 2 if ep == "swiglu" else rows
    y = torch.zeros(out_rows, device=dev)
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream

    def launch(i, ev=None):
        w, s = ws[i % copies], ss[i % copies]
        args = (wd, ep, rpb, w.data_ptr(), s.data_ptr() if s is not None else None, x.data_ptr(),
                nw.data_ptr() if norm else None, 1e-5, y.data_ptr(), rows, cols, sp)
        if ev is None:
            E.launch_matvec(*args)
        else:
            E.launch_matvec_timed(*args, ev[0].cuda_event, ev[1].cuda_event)

    for i in range(min(copies, 20)):
        launch(i)
    torch.cuda.synchronize()
    # Kernel time: events recorded by each dispatch at its kernel's start and end (no launch gap), as a
    # profiler's kernel trace reports it.  Wall time: events between consecutive launches (gaps included).
    kev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for a, b in kev:  # torch creates the HIP event at its first record
        a.record(stream)
        b.record(stream)
    w0, w1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0.record(stream)
    for i in range(iters):
        launch(i, kev[i])
    w1.record(stream)
    w1.synchronize()
    per = [a.elapsed_time(b) * 1e3 for a, b in kev]
    med, avg = statistics.median(per), statistics.fmean(per)
    wall = w0.elapsed_time(w1) * 1e3 / iters
    rec = {"name": name, "rows": rows, "cols": cols, "impl": "opt", "wtype": wd, "epilogue": ep, "fuse_norm": norm,
           "rpb": rpb or default_rpb(wd, ep, rows, cols), "bytes": nbytes, "median_us": med, "gbps": nbytes / med / 1e3,
           "avg_us": avg, "gbps_avg": nbytes / avg / 1e3, "frac_of_8tbs": nbytes / avg / 1e3 / PEAK_GBPS,
           "wall_us_per_launch": wall,
           "copies": copies, "timing": "kernel start/end events recorded by the dispatch (hipExtLaunchKernel)"}
    if stream:
        rec.update(stream_read(ws, iters, sp))
        rec["frac_of_stream"] = rec["gbps_avg"] / rec["stream_gbps"]
    del ws, ss
    torch.cuda.empty_cache()
    return rec


STREAM_BLOCKS = (4, 8, 16)  # the bandwidth kernel's launch shapes (workgroups per CU)


def stream_read(tensors, iters: int, sp: int) -> dict:
    """The bandwidth kernel reading each launch's weight tensor (its bytes rounded down to 16), over the same rotation
    of copies, timed by the dispatch like the matvec; the fastest of its launch shapes (mean kernel time).  What a
    plain read of the same bytes takes bounds what the matvec can reach."""
    import torch
    from . import engine as E
    sink = torch.zeros(16 * 1024, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
    nb = (tensors[0].numel() * tensors[0].element_size()) // 16 * 16
    best = None
    for bpc in STREAM_BLOCKS:
        kev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters + 5)]
        for a, b in kev:
            a.record(stream)
            b.record(stream)
        for i, (a, b) in enumerate(kev):  # the first 5 are warm-up
            E.launch_stream_read_timed(tensors[i % len(tensors)].data_ptr(), nb, bpc, sink.data_ptr(), sink.numel(), sp,
                                       a.cuda_event, b.cuda_event)
        kev[-1][1].synchronize()
        avg = statistics.fmean(a.elapsed_time(b) * 1e3 for a, b in kev[5:])
        if best is None or avg < best[1]:
            best = (bpc, avg)
    return {"stream_bytes": nb, "stream_us": best[1], "stream_blocks_per_cu": best[0], "stream_gbps": nb / best[1] / 1e3}


def weighted_us(per_shape_us: dict) -> float:
    """cudallm_kernelbench.cpp:296: one token's matvec time, 16 layers of qkv, wo, gate_up and down plus lm_head."""
    return 16.0 * (per_shape_us["qkv"] + per_shape_us["wo"] + per_shape_us["gate_up"] + per_shape_us["down"]) + \
        per_shape_us["lm_head"]


def bench_shapes(wd: str, rpb: int = 0, iters: int = 200, stream: bool = False) -> dict:
    """--op shapes: the five model shapes with the fused engine's epilogues."""
    import torch
    results = [bench_matvec(wd, name, rows, cols, ep, norm, iters if name != "lm_head" else max(10, iters // 4), rpb,
                            stream=stream)
               for name, rows, cols, ep, norm in SHAPES]
    return {"tool": "cudallm_kernelbench", "op": "shapes", "gpu_name": torch.cuda.get_device_name(0), "iters": iters,
            "impl": "opt", "wtype": wd, "rpb": rpb or "per shape", "results": results,
            "weighted_us": weighted_us({r["name"]: r["median_us"] for r in results})}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="matvec kernel benchmark (cudallm_kernelbench)")
    ap.add_argument("--op", choices=("matvec", "shapes"), required=True)
    ap.add_argument("--wtype", choices=("bf16", "int8", "int4"), default="bf16")
    ap.add_argument("--rpb", type=int, default=0, choices=(0, *RPBS))
    ap.add_argument("--rows", type=int)
    ap.add_argument("--cols", type=int)
    ap.add_argument("--epilogue", choices=("store", "add", "swiglu"), default="store")
    ap.add_argument("--fuse-norm", action="store_true")
    ap.add_argument("--iters", type=int, default=200)
    ap.add_argument("--json", type=Path)
    ap.add_argument("--stream", action="store_true",
                    help="also time the bandwidth kernel reading the same weight bytes (stream_us, frac_of_stream)")
    args = ap.parse_args(argv)
    if args.iters < 1:
        ap.error("--iters must be >= 1")
    if args.op == "matvec":
        if not args.rows or not args.cols:
            ap.error("--rows and --cols are required for --op matvec")
        import torch
        r = bench_matvec(args.wtype, "matvec", args.rows, args.cols, args.epilogue, args.fuse_norm, args.iters,
                         args.rpb, stream=args.stream)
        rec = {"tool": "cudallm_kernelbench", "op": "matvec", "gpu_name": torch.cuda.get_device_name(0),
               "iters": args.iters, "impl": "opt", "wtype": args.wtype, "rpb": r["rpb"], "results": [r]}
    else:
        rec = bench_shapes(args.wtype, args.rpb, args.iters, stream=args.stream)
    for r in rec["results"]:
        print(f"{r['name']:8s} {r['rows']:6d}x{r['cols']:<5d} {r['wtype']:4s} {r['epilogue']:6s} norm={int(r['fuse_norm'])} "
              f"rpb={r['rpb']}: {r['median_us']:8.2f} us  {r['gbps']:7.1f} GB/s"
              + (f"  (stream read of the weights: {r['stream_us']:.2f} us, {r['stream_gbps']:.0f} GB/s)" if "stream_us" in r
                 else ""), flush=True)
    if "weighted_us" in rec:
        print(f"weighted_us = 16*(qkv+wo+gate_up+down) + lm_head = {rec['weighted_us']:.2f}", flush=True)
    if args.json:
        args.json.parent.mkdir(parents=True, exist_ok=True)
        args.json.write_text(json.dumps(rec, indent=1) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
