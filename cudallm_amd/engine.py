"""ctypes binding of libcudallm.so (the C ABI in include/cudallm/cudallm.h).

Same public surface as the reference's ``python/cudallm/engine.py:16-214`` - ``Engine``,
``CudaLLMError`` and the ``kernel_*`` hooks with the same argument meaning - plus the GPU
quantiser entry points.  The library is located by ``CUDALLM_LIB`` or next to this file.
Nothing here falls back to a CPU implementation: a missing library raises.
"""
import ctypes
import functools
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_ubyte, c_ulonglong, c_ushort, c_void_p, c_byte
from pathlib import Path

import numpy as np

LIB_PATH = Path(os.environ.get("CUDALLM_LIB", Path(__file__).resolve().parent / "libcudallm.so"))

_IMPL = {"naive": 0, "opt": 1}
_WTYPE = {"bf16": 1, "int8": 3, "int4": 4}
_EPILOGUE = {"store": 0, "add": 1, "swiglu": 2}


class CudallmOptions(ctypes.Structure):
    _fields_ = [("matvec_impl", c_int), ("attn_impl", c_int), ("fuse", c_int), ("cuda_graph", c_int),
                ("max_seq_len", c_int), ("matvec_rpb", c_int)]


class CudallmConfigInfo(ctypes.Structure):
    _fields_ = [("weight_dtype", c_int), ("hidden", c_int), ("inter", c_int), ("n_layers", c_int),
                ("n_heads", c_int), ("n_kv_heads", c_int), ("head_dim", c_int), ("vocab", c_int),
                ("max_seq_len", c_int), ("group_size", c_int), ("rms_eps", c_float),
                ("weight_bytes", c_ulonglong)]


class CudaLLMError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"cudallm error {code}: {message}")
        self.code = code


_FP = POINTER(c_float)
_IP = POINTER(c_int)
_U16P = POINTER(c_ushort)

# The ABI as ctypes sees it: name -> (argtypes, restype).
SIGNATURES = {
    "cudallm_last_error": ([], c_char_p),
    "cudallm_default_options": ([POINTER(CudallmOptions)], None),
    "cudallm_create": ([c_char_p, POINTER(CudallmOptions), POINTER(c_void_p)], c_int),
    "cudallm_destroy": ([c_void_p], None),
    "cudallm_get_config": ([c_void_p, POINTER(CudallmConfigInfo)], c_int),
    "cudallm_reset": ([c_void_p], c_int),
    "cudallm_pos": ([c_void_p], c_int),
    "cudallm_get_stream": ([c_void_p, POINTER(c_void_p)], c_int),
    "cudallm_step": ([c_void_p, c_int, _FP, _IP], c_int),
    "cudallm_step_debug": ([c_void_p, c_int, _FP, _FP, _IP], c_int),
    "cudallm_step_profile": ([c_void_p, c_int, POINTER(c_ulonglong), ctypes.c_longlong, _IP], c_int),
    "cudallm_kernel_matvec": ([c_int, c_int, c_int, c_int, c_int, c_void_p, c_ulonglong, c_void_p, c_ulonglong,
                               _FP, _FP, c_float, _FP, c_int, c_int], c_int),
    "cudallm_kernel_rmsnorm": ([_FP, _FP, c_float, _FP, c_int], c_int),
    "cudallm_kernel_rope_kv": ([c_int, _FP, _FP, c_int, _U16P, _U16P, c_int, c_int, c_int, c_int], c_int),
    "cudallm_kernel_attention": ([c_int, _FP, _U16P, _U16P, c_int, _FP, c_int, c_int, c_int, c_int], c_int),
    "cudallm_kernel_silu_mul": ([_FP, _FP, c_int], c_int),
    "cudallm_kernel_argmax": ([_FP, c_int, _IP], c_int),
    "cudallm_launch_matvec": ([c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_void_p, c_int,
                               c_int, c_void_p], c_int),
    "cudallm_launch_attention": ([c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                  c_int, c_int, c_void_p], c_int),
    "cudallm_quantize_int8_rows": ([_FP, c_int, c_int, POINTER(c_byte), _FP], c_int),
    "cudallm_quantize_int4_groups": ([_FP, c_int, c_int, c_int, POINTER(c_ubyte), _U16P], c_int),
    "cudallm_unpack_int4": ([POINTER(c_ubyte), c_int, c_int, POINTER(c_byte)], c_int),
}


@functools.cache
def _lib() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise CudaLLMError(6, f"{LIB_PATH} is not built (run __graft_entry__.build() or make -C cudallm_amd)")
    # One HIP runtime per process: a process that also uses torch must resolve libamdhip64.so.7 to
    # the copy torch already loaded (same SONAME).  Loading ours first would bring a second HSA
    # runtime, and whichever initialises second cannot open the GPU.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (argtypes, restype) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    return lib


def lib() -> ctypes.CDLL:
    """The loaded library (raises CudaLLMError if it is not built)."""
    return _lib()


def _check(rc: int) -> None:
    if rc != 0:
        msg = _lib().cudallm_last_error()
        raise CudaLLMError(rc, msg.decode("utf-8", "replace") if msg else "")


def _fp(a: np.ndarray):
    return a.ctypes.data_as(_FP)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _fp16_bits(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype == np.float16:
        return np.ascontiguousarray(a).view(np.uint16).copy()
    return np.ascontiguousarray(a, dtype=np.uint16).copy()


def _code(table: dict, v) -> int:
    return table[v] if isinstance(v, str) else int(v)


class Engine:
    """One decode engine (``python/cudallm/engine.py:94-151``)."""

    def __init__(self, path, *, matvec: str = "opt", attn: str = "opt", fuse: bool = True, cuda_graph: bool = True,
                 max_seq_len: int = 0, matvec_rpb: int = 0):
        self._h = None
        lib = _lib()
        opts = CudallmOptions(_IMPL[matvec], _IMPL[attn], int(bool(fuse)), int(bool(cuda_graph)), int(max_seq_len),
                              int(matvec_rpb))
        h = c_void_p()
        _check(lib.cudallm_create(str(path).encode(), ctypes.byref(opts), ctypes.byref(h)))
        self._h = h
        info = CudallmConfigInfo()
        _check(lib.cudallm_get_config(self._h, ctypes.byref(info)))
        self.config = {name: getattr(info, name) for name, _ in CudallmConfigInfo._fields_}
        self._vocab, self._rows, self._hidden = info.vocab, info.n_layers + 1, info.hidden

    def _handle(self) -> c_void_p:
        if self._h is None:
            raise CudaLLMError(5, "engine is closed")
        return self._h

    @property
    def pos(self) -> int:
        return _lib().cudallm_pos(self._handle())

    def reset(self) -> None:
        _check(_lib().cudallm_reset(self._handle()))

    def step(self, token: int | None = None, *, want_logits: bool = False) -> tuple[int, np.ndarray | None]:
        nxt = c_int(0)
        logits = np.empty(self._vocab, dtype=np.float32) if want_logits else None
        _check(_lib().cudallm_step(self._handle(), -1 if token is None else int(token),
                                   _fp(logits) if logits is not None else None, ctypes.byref(nxt)))
        return nxt.value, logits

    def step_async(self, token: int | None = None) -> None:
        """A step that requests no outputs, so it does not synchronise (pipelined decoding)."""
        _check(_lib().cudallm_step(self._handle(), -1 if token is None else int(token), None, None))

    def step_debug(self, token: int | None = None) -> tuple[int, np.ndarray, np.ndarray]:
        nxt = c_int(0)
        logits = np.empty(self._vocab, dtype=np.float32)
        residuals = np.empty((self._rows, self._hidden), dtype=np.float32)
        _check(_lib().cudallm_step_debug(self._handle(), -1 if token is None else int(token), _fp(residuals),
                                         _fp(logits), ctypes.byref(nxt)))
        return nxt.value, logits, residuals

    def step_profile(self, token: int | None = None) -> np.ndarray:
        """One synchronous step of the persistent kernel; returns uint64 stamps [grid, 128]
        (100 MHz clock): [:, 0] start, [:, 1 + 6*l + k] end of phase k of layer l, [:, 97] lm_head."""
        cap = 4096 * 128
        buf = np.zeros(cap, dtype=np.uint64)
        grid = c_int(0)
        _check(_lib().cudallm_step_profile(self._handle(), -1 if token is None else int(token),
                                           buf.ctypes.data_as(POINTER(c_ulonglong)), cap, ctypes.byref(grid)))
        return buf[:grid.value * 128].reshape(grid.value, 128)

    @property
    def stream(self) -> int:
        """Address of the engine's HIP stream (hipStream_t), e.g. for torch.cuda.ExternalStream."""
        s = c_void_p(0)
        _check(_lib().cudallm_get_stream(self._handle(), ctypes.byref(s)))
        return s.value or 0

    def close(self) -> None:
        if self._h is not None:
            _lib().cudallm_destroy(self._h)
            self._h = None

    def __enter__(self) -> "Engine":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        if getattr(self, "_h", None) is not None:
            self.close()


def kernel_matvec(impl, wtype, epilogue, fuse_norm, rpb: int, w: np.ndarray, scales, x: np.ndarray, norm_w,
                  eps: float, y_init, rows: int, cols: int) -> np.ndarray:
    """``python/cudallm/engine.py:154-169``."""
    ep = _code(_EPILOGUE, epilogue)
    out_rows = rows // 2 if ep == 2 else rows
    w = np.ascontiguousarray(w)
    s = np.ascontiguousarray(scales) if scales is not None else None
    x = _f32(x)
    n = _f32(norm_w) if norm_w is not None else None
    y = _f32(y_init).copy() if y_init is not None else np.zeros(out_rows, dtype=np.float32)
    if y.shape != (out_rows,):
        raise ValueError(f"y_init must have shape ({out_rows},)")
    _check(_lib().cudallm_kernel_matvec(_code(_IMPL, impl), _code(_WTYPE, wtype), ep, int(bool(fuse_norm)), int(rpb),
                                        w.ctypes.data, w.nbytes, s.ctypes.data if s is not None else None,
                                        s.nbytes if s is not None else 0, _fp(x), _fp(n) if n is not None else None,
                                        float(eps), _fp(y), int(rows), int(cols)))
    return y


def launch_matvec(wtype, epilogue, rpb: int, w_ptr: int, scales_ptr: int | None, x_ptr: int, norm_ptr: int | None,
                  eps: float, y_ptr: int, rows: int, cols: int, stream: int | None = None) -> None:
    """Enqueue the opt matvec on device pointers (e.g. ``tensor.data_ptr()``) and a HIP stream handle."""
    _check(_lib().cudallm_launch_matvec(_code(_WTYPE, wtype), _code(_EPILOGUE, epilogue), int(rpb), w_ptr, scales_ptr,
                                        x_ptr, norm_ptr, float(eps), y_ptr, int(rows), int(cols), stream))


def launch_attention(q_ptr: int, k_ptr: int, v_ptr: int, pos_ptr: int, part_o_ptr: int, part_ml_ptr: int, out_ptr: int,
                     nh: int, nkv: int, hd: int, max_seq: int, stream: int | None = None) -> None:
    """Enqueue split-K attention on device pointers over ctx = *pos + 1 tokens."""
    _check(_lib().cudallm_launch_attention(q_ptr, k_ptr, v_ptr, pos_ptr, part_o_ptr, part_ml_ptr, out_ptr, nh, nkv, hd,
                                           max_seq, stream))


def kernel_rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    y = np.empty_like(x)
    _check(_lib().cudallm_kernel_rmsnorm(_fp(x), _fp(w), float(eps), _fp(y), x.size))
    return y


def kernel_rope_kv(fused, qkv, inv_freq, pos: int, k_cache, v_cache, nh: int, nkv: int, hd: int, max_seq: int):
    qkv = _f32(qkv).copy()
    inv = _f32(inv_freq)
    k, v = _fp16_bits(k_cache), _fp16_bits(v_cache)
    _check(_lib().cudallm_kernel_rope_kv(int(bool(fused)), _fp(qkv), _fp(inv), int(pos), k.ctypes.data_as(_U16P),
                                         v.ctypes.data_as(_U16P), nh, nkv, hd, max_seq))
    return qkv, k.view(np.float16), v.view(np.float16)


def kernel_attention(impl, q, k_cache, v_cache, ctx: int, nh: int, nkv: int, hd: int, max_seq: int) -> np.ndarray:
    q = _f32(q)
    k, v = _fp16_bits(k_cache), _fp16_bits(v_cache)
    out = np.empty(nh * hd, dtype=np.float32)
    _check(_lib().cudallm_kernel_attention(_code(_IMPL, impl), _fp(q), k.ctypes.data_as(_U16P), v.ctypes.data_as(_U16P),
                                           int(ctx), _fp(out), nh, nkv, hd, max_seq))
    return out


def kernel_silu_mul(gu: np.ndarray) -> np.ndarray:
    gu = _f32(gu)
    act = np.empty(gu.size // 2, dtype=np.float32)
    _check(_lib().cudallm_kernel_silu_mul(_fp(gu), _fp(act), gu.size // 2))
    return act


def kernel_argmax(logits: np.ndarray) -> int:
    logits = _f32(logits)
    idx = c_int(-1)
    _check(_lib().cudallm_kernel_argmax(_fp(logits), logits.size, ctypes.byref(idx)))
    return idx.value
