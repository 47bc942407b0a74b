"""Weight quantisers, computed on the GPU through the C ABI.

Same names and results as the reference's ``python/cudallm/quantize.py:5-47`` (bit-identical
int8 codes and fp32 scales; bit-identical packed int4 nibbles and fp16 scales).  Dequantisation is
plain arithmetic on the stored values and stays in numpy.
"""
import ctypes

import numpy as np

from .engine import call


def _ptr(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def quantize_int8_rows(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), dtype=np.int8)
    s = np.empty(rows, dtype=np.float32)
    call("cudallm_quantize_int8_rows", _ptr(w, ctypes.c_float), rows, cols, _ptr(q, ctypes.c_byte),
         _ptr(s, ctypes.c_float))
    return q, s


def dequantize_int8_rows(q: np.ndarray, scales: np.ndarray) -> np.ndarray:
    return q.astype(np.float32) * scales.astype(np.float32)[:, None]


def quantize_int4_groups(w: np.ndarray, group: int = 128) -> tuple[np.ndarray, np.ndarray]:
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    packed = np.empty((rows, cols // 2), dtype=np.uint8)
    s = np.empty((rows, cols // group), dtype=np.uint16)
    call("cudallm_quantize_int4_groups", _ptr(w, ctypes.c_float), rows, cols, group, _ptr(packed, ctypes.c_ubyte),
         _ptr(s, ctypes.c_ushort))
    return packed, s.view(np.float16)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    rows, half = packed.shape
    q = np.empty((rows, half * 2), dtype=np.int8)
    call("cudallm_unpack_int4", _ptr(packed, ctypes.c_ubyte), rows, half * 2, _ptr(q, ctypes.c_byte))
    return q


def dequantize_int4_groups(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    q = unpack_int4(packed).astype(np.float32)
    rows, cols = q.shape
    ng = scales.shape[1]
    return (q.reshape(rows, ng, cols // ng) * scales.astype(np.float32)[:, :, None]).reshape(rows, cols)
