"""Python view of libcudallm.so, the C ABI declared in include/cudallm/cudallm.h.

The public surface is the one the reference's Python package offers (``python/cudallm/engine.py``):
``Engine`` (``step``, ``step_debug``, ``reset``, ``pos``, ``config``), ``CudaLLMError`` carrying the
C error code, and the single-kernel hooks ``kernel_matvec`` ... ``kernel_argmax`` with the same argument
meaning, so code written against the reference runs unchanged.  Added: ``step_async``, ``step_profile``,
``step_trace``, ``stream`` and the device-pointer launches.

Every C call goes through :func:`call`, which raises ``CudaLLMError`` for a non-zero return code.  The
library is found through ``CUDALLM_LIB`` or next to this file; there is no CPU fallback: a missing
library raises.
"""
import ctypes
import os
from ctypes import POINTER, c_byte, c_char_p, c_double, c_float, c_int, c_longlong, c_ubyte, c_ulonglong, c_ushort, c_void_p
from pathlib import Path

import numpy as np

LIB_PATH = Path(os.environ.get("CUDALLM_LIB", Path(__file__).resolve().parent / "libcudallm.so"))

IMPL_CODES = {"naive": 0, "opt": 1}
WEIGHT_CODES = {"bf16": 1, "int8": 3, "int4": 4}
EPILOGUE_CODES = {"store": 0, "add": 1, "swiglu": 2}
ERR_STATE = 5
ERR_INTERNAL = 6


class CudallmOptions(ctypes.Structure):
    """``cudallm_options``: six ints (24 bytes)."""
    _fields_ = [(name, c_int) for name in
                ("matvec_impl", "attn_impl", "fuse", "cuda_graph", "max_seq_len", "matvec_rpb")]


class CudallmConfigInfo(ctypes.Structure):
    """``cudallm_config_info``: ten ints, a float, then a u64 at offset 48 (56 bytes)."""
    _fields_ = [(name, c_int) for name in ("weight_dtype", "hidden", "inter", "n_layers", "n_heads", "n_kv_heads",
                                            "head_dim", "vocab", "max_seq_len", "group_size")] + \
               [("rms_eps", c_float), ("weight_bytes", c_ulonglong)]


class CudaLLMError(RuntimeError):
    """A failed C call: ``code`` is the CUDALLM_* code, the message is ``cudallm_last_error()``."""

    def __init__(self, code: int, message: str):
        super().__init__(f"cudallm error {code}: {message}")
        self.code = code


_F32P, _I32P, _U16P = POINTER(c_float), POINTER(c_int), POINTER(c_ushort)

# name -> (argtypes, restype), in header order.
SIGNATURES = {
    "cudallm_last_error": ([], c_char_p),
    "cudallm_default_options": ([POINTER(CudallmOptions)], None),
    "cudallm_create": ([c_char_p, POINTER(CudallmOptions), POINTER(c_void_p)], c_int),
    "cudallm_destroy": ([c_void_p], None),
    "cudallm_get_config": ([c_void_p, POINTER(CudallmConfigInfo)], c_int),
    "cudallm_reset": ([c_void_p], c_int),
    "cudallm_pos": ([c_void_p], c_int),
    "cudallm_step": ([c_void_p, c_int, _F32P, _I32P], c_int),
    "cudallm_step_debug": ([c_void_p, c_int, _F32P, _F32P, _I32P], c_int),
    "cudallm_step_profile": ([c_void_p, c_int, POINTER(c_ulonglong), c_longlong, _I32P], c_int),
    "cudallm_step_trace": ([c_void_p, c_int, _F32P, c_longlong, _F32P, _I32P], c_int),
    "cudallm_get_stream": ([c_void_p, POINTER(c_void_p)], c_int),
    "cudallm_get_step_kind": ([c_void_p, _I32P, _I32P], c_int),
    "cudallm_kernel_matvec": ([c_int, c_int, c_int, c_int, c_int, c_void_p, c_ulonglong, c_void_p, c_ulonglong,
                               _F32P, _F32P, c_float, _F32P, c_int, c_int], c_int),
    "cudallm_kernel_rmsnorm": ([_F32P, _F32P, c_float, _F32P, c_int], c_int),
    "cudallm_kernel_rope_kv": ([c_int, _F32P, _F32P, c_int, _U16P, _U16P, c_int, c_int, c_int, c_int], c_int),
    "cudallm_kernel_attention": ([c_int, _F32P, _U16P, _U16P, c_int, _F32P, c_int, c_int, c_int, c_int], c_int),
    "cudallm_kernel_silu_mul": ([_F32P, _F32P, c_int], c_int),
    "cudallm_kernel_argmax": ([_F32P, c_int, _I32P], c_int),
    "cudallm_launch_matvec": ([c_int, c_int, c_int] + [c_void_p] * 4 + [c_float, c_void_p, c_int, c_int, c_void_p],
                              c_int),
    "cudallm_launch_stream_read_timed": ([c_void_p, c_ulonglong, c_int, c_void_p, c_ulonglong, c_void_p, c_void_p,
                                          c_void_p], c_int),
    "cudallm_launch_matvec_timed": ([c_int, c_int, c_int] + [c_void_p] * 4 + [c_float, c_void_p, c_int, c_int] +
                                    [c_void_p] * 3, c_int),
    "cudallm_launch_attention": ([c_void_p] * 7 + [c_int] * 4 + [c_void_p], c_int),
    "cudallm_launch_attention_static": ([c_void_p] * 5 + [c_int] * 4 + [c_void_p], c_int),
    "cudallm_measure_read_bandwidth": ([c_ulonglong, c_int, POINTER(c_double), POINTER(c_double)], c_int),
    "cudallm_quantize_int8_rows": ([_F32P, c_int, c_int, POINTER(c_byte), _F32P], c_int),
    "cudallm_quantize_int4_groups": ([_F32P, c_int, c_int, c_int, POINTER(c_ubyte), _U16P], c_int),
    "cudallm_unpack_int4": ([POINTER(c_ubyte), c_int, c_int, POINTER(c_byte)], c_int),
}

_loaded: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The library with every declared function typed.  Raises CudaLLMError when it is not built."""
    global _loaded
    if _loaded is None:
        if not LIB_PATH.is_file():
            raise CudaLLMError(ERR_INTERNAL, f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                                             f"or make -C cudallm_amd")
        # A process that also imports torch must bind our HIP runtime dependency to the copy torch already
        # loaded (same SONAME); loading ours first would start a second runtime that cannot open the GPU.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes, fn.restype = argtypes, restype
        _loaded = handle
    return _loaded


def call(name: str, *args) -> int:
    """Call ``name``; a non-zero CUDALLM_* code becomes CudaLLMError with the library's message."""
    rc = getattr(lib(), name)(*args)
    if rc:
        raw = lib().cudallm_last_error()
        raise CudaLLMError(rc, raw.decode("utf-8", "replace") if raw else "")
    return rc


def _code(table: dict, v) -> int:
    """A name from `table` or an int passed through (the hooks take either)."""
    return table[v] if isinstance(v, str) else int(v)


def _in(a, dtype) -> np.ndarray:
    """Contiguous array of `dtype` for an input operand (no copy when it already is one)."""
    return np.ascontiguousarray(a, dtype=dtype)


def _half_bits(a) -> np.ndarray:
    """A private uint16 copy of fp16 data (given as float16, or as its raw bits)."""
    a = np.asarray(a)
    return np.array(a.view(np.uint16) if a.dtype == np.float16 else a, dtype=np.uint16, order="C", copy=True)


def _p(a: np.ndarray | None, ctype=c_float):
    return None if a is None else a.ctypes.data_as(POINTER(ctype))


def _tok(token) -> int:
    return -1 if token is None else int(token)


class Engine:
    """One decode engine over a ``.cudallm`` file; single-threaded, like the C handle it owns."""

    def __init__(self, path, *, matvec: str = "opt", attn: str = "opt", fuse: bool = True, cuda_graph: bool = True,
                 max_seq_len: int = 0, matvec_rpb: int = 0):
        self._h = None
        opts = CudallmOptions(matvec_impl=IMPL_CODES[matvec], attn_impl=IMPL_CODES[attn], fuse=int(bool(fuse)),
                              cuda_graph=int(bool(cuda_graph)), max_seq_len=int(max_seq_len),
                              matvec_rpb=int(matvec_rpb))
        handle = c_void_p()
        call("cudallm_create", os.fsencode(str(path)), ctypes.byref(opts), ctypes.byref(handle))
        self._h = handle
        info = CudallmConfigInfo()
        call("cudallm_get_config", handle, ctypes.byref(info))
        self.config = {f: getattr(info, f) for f, _ in CudallmConfigInfo._fields_}

    # -- handle ------------------------------------------------------------------------------------
    @property
    def handle(self) -> c_void_p:
        if self._h is None:
            raise CudaLLMError(ERR_STATE, "engine is closed")
        return self._h

    def close(self) -> None:
        h, self._h = self._h, None
        if h is not None:
            lib().cudallm_destroy(h)

    def __enter__(self) -> "Engine":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        if getattr(self, "_h", None) is not None:
            self.close()

    # -- state -------------------------------------------------------------------------------------
    @property
    def pos(self) -> int:
        return lib().cudallm_pos(self.handle)

    @property
    def stream(self) -> int:
        """Address of the engine's HIP stream (a hipStream_t), e.g. for torch.cuda.ExternalStream."""
        s = c_void_p()
        call("cudallm_get_stream", self.handle, ctypes.byref(s))
        return s.value or 0

    @property
    def step_kind(self) -> tuple[str, int]:
        """("persistent", grid) when each step is one launch of the persistent decode kernel, ("program", 0)
        for the multi-kernel step."""
        kind, grid = c_int(), c_int()
        call("cudallm_get_step_kind", self.handle, ctypes.byref(kind), ctypes.byref(grid))
        return ("persistent" if kind.value == 1 else "program"), grid.value

    @property
    def persistent(self) -> bool:
        return self.step_kind[0] == "persistent"

    def reset(self) -> None:
        call("cudallm_reset", self.handle)

    # -- steps -------------------------------------------------------------------------------------
    def _vocab_buffer(self) -> np.ndarray:
        return np.empty(self.config["vocab"], dtype=np.float32)

    def step(self, token: int | None = None, *, want_logits: bool = False) -> tuple[int, np.ndarray | None]:
        """Decode one position; token None reuses the previous device argmax.  Returns (next token, logits)."""
        logits = self._vocab_buffer() if want_logits else None
        nxt = c_int()
        call("cudallm_step", self.handle, _tok(token), _p(logits), ctypes.byref(nxt))
        return nxt.value, logits

    def step_async(self, token: int | None = None) -> None:
        """A step that asks for no output, so it does not synchronise (pipelined decoding)."""
        call("cudallm_step", self.handle, _tok(token), None, None)

    def step_debug(self, token: int | None = None) -> tuple[int, np.ndarray, np.ndarray]:
        """Returns (next token, logits, residuals[n_layers + 1, hidden])."""
        c = self.config
        residuals = np.empty((c["n_layers"] + 1, c["hidden"]), dtype=np.float32)
        logits, nxt = self._vocab_buffer(), c_int()
        call("cudallm_step_debug", self.handle, _tok(token), _p(residuals), _p(logits), ctypes.byref(nxt))
        return nxt.value, logits, residuals

    def step_profile(self, token: int | None = None) -> np.ndarray:
        """One synchronous step of the persistent kernel; returns the uint64 stamps [grid, 128] (100 MHz clock):
        [:, 0] start, [:, 1 + 6*l + k] end of phase k of layer l, [:, 97] lm_head end."""
        cap = 4096 * 128
        stamps = np.zeros(cap, dtype=np.uint64)
        grid = c_int()
        call("cudallm_step_profile", self.handle, _tok(token), _p(stamps, c_ulonglong), cap, ctypes.byref(grid))
        return stamps[:grid.value * 128].reshape(grid.value, 128)

    def step_trace(self, token: int | None = None) -> tuple[int, np.ndarray, dict]:
        """One synchronous step of the persistent kernel that returns every phase's output:
        (next token, logits, {"residuals": [L+1, H], "qkv": [L, 3072], "att": [L, 2048], "xa": [L, H],
        "act": [L, inter]})."""
        c = self.config
        L, H = c["n_layers"], c["hidden"]
        shapes = {"residuals": (L + 1, H), "qkv": (L, (c["n_heads"] + 2 * c["n_kv_heads"]) * c["head_dim"]),
                  "att": (L, c["n_heads"] * c["head_dim"]), "xa": (L, H), "act": (L, c["inter"])}
        total = sum(a * b for a, b in shapes.values())
        flat = np.empty(total, dtype=np.float32)
        logits, nxt = self._vocab_buffer(), c_int()
        call("cudallm_step_trace", self.handle, _tok(token), _p(flat), total, _p(logits), ctypes.byref(nxt))
        out, at = {}, 0
        for name, (a, b) in shapes.items():
            out[name] = flat[at:at + a * b].reshape(a, b)
            at += a * b
        return nxt.value, logits, out


# ---- single-kernel hooks (host arrays in and out; each call is synchronous) ------------------------

def kernel_matvec(impl, wtype, epilogue, fuse_norm, rpb: int, w: np.ndarray, scales, x: np.ndarray, norm_w,
                  eps: float, y_init, rows: int, cols: int) -> np.ndarray:
    """y = W x^ (STORE), y_init + W x^ (ADD) or silu(d[:rows/2]) * d[rows/2:] (SWIGLU), x^ = rmsnorm(x) * norm_w
    when fuse_norm is set."""
    ep = _code(EPILOGUE_CODES, epilogue)
    n_out = rows // 2 if ep == EPILOGUE_CODES["swiglu"] else rows
    w = np.ascontiguousarray(w)
    s = None if scales is None else np.ascontiguousarray(scales)
    y = np.zeros(n_out, np.float32) if y_init is None else np.array(y_init, dtype=np.float32, order="C", copy=True)
    if y.shape != (n_out,):
        raise ValueError(f"y_init has shape {y.shape}, expected ({n_out},)")
    xin = _in(x, np.float32)
    nin = None if norm_w is None else _in(norm_w, np.float32)
    call("cudallm_kernel_matvec", _code(IMPL_CODES, impl), _code(WEIGHT_CODES, wtype), ep, int(bool(fuse_norm)),
         int(rpb), w.ctypes.data, w.nbytes, None if s is None else s.ctypes.data, 0 if s is None else s.nbytes,
         _p(xin), _p(nin), float(eps), _p(y), int(rows), int(cols))
    return y


def kernel_rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    xin, win = _in(x, np.float32), _in(w, np.float32)
    y = np.empty_like(xin)
    call("cudallm_kernel_rmsnorm", _p(xin), _p(win), float(eps), _p(y), xin.size)
    return y


def kernel_rope_kv(fused, qkv, inv_freq, pos: int, k_cache, v_cache, nh: int, nkv: int, hd: int, max_seq: int):
    """Returns (qkv after the kernel, k cache, v cache) as (float32, float16, float16) arrays."""
    q = np.array(qkv, dtype=np.float32, order="C", copy=True)
    k, v = _half_bits(k_cache), _half_bits(v_cache)
    call("cudallm_kernel_rope_kv", int(bool(fused)), _p(q), _p(_in(inv_freq, np.float32)), int(pos), _p(k, c_ushort),
         _p(v, c_ushort), nh, nkv, hd, max_seq)
    return q, k.view(np.float16), v.view(np.float16)


def kernel_attention(impl, q, k_cache, v_cache, ctx: int, nh: int, nkv: int, hd: int, max_seq: int) -> np.ndarray:
    qin = _in(q, np.float32)
    k, v = _half_bits(k_cache), _half_bits(v_cache)
    out = np.empty(nh * hd, dtype=np.float32)
    call("cudallm_kernel_attention", _code(IMPL_CODES, impl), _p(qin), _p(k, c_ushort), _p(v, c_ushort), int(ctx),
         _p(out), nh, nkv, hd, max_seq)
    return out


def kernel_silu_mul(gu: np.ndarray) -> np.ndarray:
    g = _in(gu, np.float32)
    act = np.empty(g.size // 2, dtype=np.float32)
    call("cudallm_kernel_silu_mul", _p(g), _p(act), act.size)
    return act


def kernel_argmax(logits: np.ndarray) -> int:
    lg = _in(logits, np.float32)
    idx = c_int(-1)
    call("cudallm_kernel_argmax", _p(lg), lg.size, ctypes.byref(idx))
    return idx.value


# ---- device-pointer launches (integer addresses, e.g. tensor.data_ptr(); stream None = null stream) --------

def launch_matvec(wtype, epilogue, rpb: int, w_ptr: int, scales_ptr: int | None, x_ptr: int, norm_ptr: int | None,
                  eps: float, y_ptr: int, rows: int, cols: int, stream: int | None = None) -> None:
    call("cudallm_launch_matvec", _code(WEIGHT_CODES, wtype), _code(EPILOGUE_CODES, epilogue), int(rpb), w_ptr,
         scales_ptr, x_ptr, norm_ptr, float(eps), y_ptr, int(rows), int(cols), stream)


def launch_matvec_timed(wtype, epilogue, rpb: int, w_ptr: int, scales_ptr: int | None, x_ptr: int,
                        norm_ptr: int | None, eps: float, y_ptr: int, rows: int, cols: int, stream: int | None,
                        start_event: int, stop_event: int) -> None:
    """launch_matvec whose kernel records the two hipEvent_t handles at its own start and end."""
    call("cudallm_launch_matvec_timed", _code(WEIGHT_CODES, wtype), _code(EPILOGUE_CODES, epilogue), int(rpb), w_ptr,
         scales_ptr, x_ptr, norm_ptr, float(eps), y_ptr, int(rows), int(cols), stream, start_event, stop_event)


def launch_stream_read_timed(src_ptr: int, nbytes: int, blocks_per_cu: int, sink_ptr: int, sink_words: int,
                             stream: int | None, start_event: int, stop_event: int) -> None:
    """One stream read of nbytes at src_ptr whose kernel records the two hipEvent_t handles at its start and end."""
    call("cudallm_launch_stream_read_timed", src_ptr, int(nbytes), int(blocks_per_cu), sink_ptr, int(sink_words), stream,
         start_event, stop_event)


def launch_attention(q_ptr: int, k_ptr: int, v_ptr: int, pos_ptr: int, part_o_ptr: int, part_ml_ptr: int, out_ptr: int,
                     nh: int, nkv: int, hd: int, max_seq: int, stream: int | None = None) -> None:
    """Split-K attention over ctx = *pos + 1 tokens; part_o / part_ml are the caller's scratch."""
    call("cudallm_launch_attention", q_ptr, k_ptr, v_ptr, pos_ptr, part_o_ptr, part_ml_ptr, out_ptr, nh, nkv, hd,
         max_seq, stream)


def launch_attention_static(q_ptr: int, k_ptr: int, v_ptr: int, pos_ptr: int, out_ptr: int, nh: int, nkv: int,
                            hd: int, max_seq: int, stream: int | None = None) -> None:
    """launch_attention with its split partials in the library's static device scratch (allocates nothing)."""
    call("cudallm_launch_attention_static", q_ptr, k_ptr, v_ptr, pos_ptr, out_ptr, nh, nkv, hd, max_seq, stream)


def measure_read_bandwidth(nbytes: int = 4 << 30, reps: int = 10) -> tuple[float, float]:
    """(best, median) stream-read GB/s of device memory over an `nbytes` buffer."""
    best, med = c_double(), c_double()
    call("cudallm_measure_read_bandwidth", int(nbytes), int(reps), ctypes.byref(best), ctypes.byref(med))
    return best.value, med.value
