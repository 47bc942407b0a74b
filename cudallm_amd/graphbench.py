"""Persistent decode kernel: direct launches against hipGraph replay (the reference replays its whole step as a graph,
src/engine/engine.cpp:117-147).

    python -m cudallm_amd.graphbench [--dtypes bf16,int4] [--steps 256] [--graph-steps 16]

Per weight type, after the same 16-token prompt each time: `steps` greedy steps launched directly (cudallm_step with
no outputs), the same number as one-step graphs replayed once per step, and as graphs of `graph-steps` consecutive
steps (the token and position stay on the device, so a captured step needs no host input).  The graphs are captured on
the engine's own stream with HIP's stream capture, through ctypes.  Prints microseconds per step from the host clock
around each run (stream drained on both sides); under rocprofv3 --kernel-trace the dispatch timestamps give the gap
between consecutive kernels (cudallm_amd.profsum gaps).
"""
import argparse
import ctypes
import sys
import tempfile
import time
from pathlib import Path

from . import engine as E
from . import synth

_CAPTURE_RELAXED = 2  # hipStreamCaptureModeRelaxed


def _hip():
    import torch  # noqa: F401  (binds the HIP runtime torch loaded, as engine.lib() does)
    h = ctypes.CDLL("libamdhip64.so")
    h.hipStreamBeginCapture.argtypes = [ctypes.c_void_p, ctypes.c_int]
    h.hipStreamEndCapture.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
    h.hipGraphInstantiate.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_size_t]
    h.hipGraphLaunch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    h.hipGraphExecDestroy.argtypes = [ctypes.c_void_p]
    h.hipGraphDestroy.argtypes = [ctypes.c_void_p]
    h.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    return h


def _ok(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: HIP error {rc}")


class StepGraph:
    """`n` consecutive greedy steps of `eng` captured as one executable graph on the engine's stream."""

    def __init__(self, hip, eng, n: int):
        self.hip, stream = hip, ctypes.c_void_p(eng.stream)
        _ok(hip.hipStreamBeginCapture(stream, _CAPTURE_RELAXED), "hipStreamBeginCapture")
        try:
            for _ in range(n):
                E.call("cudallm_step", eng.handle, -1, None, None)
        finally:
            self.graph = ctypes.c_void_p()
            _ok(hip.hipStreamEndCapture(stream, ctypes.byref(self.graph)), "hipStreamEndCapture")
        self.exec = ctypes.c_void_p()
        _ok(hip.hipGraphInstantiate(ctypes.byref(self.exec), self.graph, None, None, 0), "hipGraphInstantiate")

    def launch(self, stream) -> None:
        _ok(self.hip.hipGraphLaunch(self.exec, stream), "hipGraphLaunch")

    def close(self) -> None:
        self.hip.hipGraphExecDestroy(self.exec)
        self.hip.hipGraphDestroy(self.graph)


def run(path, steps: int, graph_steps: int) -> dict:
    hip = _hip()
    out = {}
    with E.Engine(path) as eng:
        if not eng.persistent:
            raise RuntimeError("the engine does not run the persistent decode kernel")
        stream = ctypes.c_void_p(eng.stream)

        def timed(label, fn):
            eng.reset()
            for _ in range(15):
                eng.step_async(128000)
            eng.step(1)  # drains the stream
            t0 = time.perf_counter()
            fn()
            _ok(hip.hipStreamSynchronize(stream), "hipStreamSynchronize")
            out[label] = 1e6 * (time.perf_counter() - t0) / steps

        timed("direct", lambda: [eng.step_async(None) for _ in range(steps)])
        one = StepGraph(hip, eng, 1)
        many = StepGraph(hip, eng, graph_steps)
        try:
            timed("graph_1", lambda: [one.launch(stream) for _ in range(steps)])
            timed(f"graph_{graph_steps}", lambda: [many.launch(stream) for _ in range(steps // graph_steps)])
        finally:
            one.close()
            many.close()
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--dtypes", default="bf16,int4")
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--graph-steps", type=int, default=16)
    args = ap.parse_args(argv)
    if args.steps % args.graph_steps:
        ap.error("--steps must be a multiple of --graph-steps")
    with tempfile.TemporaryDirectory(dir="/dev/shm" if Path("/dev/shm").is_dir() else None) as d:
        for wd in args.dtypes.split(","):
            path = Path(d) / f"graph_{wd}.cudallm"
            synth.write_model(path, wd, seed=1234)
            r = run(path, args.steps, args.graph_steps)
            print(f"[graphbench] {wd}: " + ", ".join(f"{k} {v:.1f} us/step" for k, v in r.items()), flush=True)
            path.unlink()
    return 0


if __name__ == "__main__":
    sys.exit(main())
