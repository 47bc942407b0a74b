"""Weight quantisers, restated from the reference (test infrastructure only).

Reference: ``python/cudallm/quantize.py:5-47``; the exporter applies them to the bf16
master weight upcast to fp32 (``python/cudallm/export.py:85-97``).

All arithmetic is numpy float32 with IEEE round-to-nearest-even: ``max|row| / 127`` and
``w / s`` are single-precision divisions and ``np.rint`` rounds half to even.
"""
import numpy as np


def bf16_round_bits(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits with round-to-nearest-even (``tests/test_kernels.py:19-22``)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bits -> fp32 (``python/cudallm/format.py:146-147``)."""
    return (np.asarray(bits).astype(np.uint32) << 16).view(np.float32)


def quantize_int8_rows(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """One fp32 scale per row: s = max|row|/127 (1 for an all-zero row), q = clip(rint(w/s)).

    Follows ``python/cudallm/quantize.py:5-10``.
    """
    w = np.asarray(w, dtype=np.float32)
    s = (np.abs(w).max(axis=1) / np.float32(127)).astype(np.float32)
    s[s == 0] = np.float32(1.0)
    q = np.clip(np.rint(w / s[:, None]), -127, 127).astype(np.int8)
    return q, s


def dequantize_int8_rows(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """``python/cudallm/quantize.py:13-14``."""
    return q.astype(np.float32) * np.asarray(s, dtype=np.float32)[:, None]


def quantize_int4_groups(w: np.ndarray, group: int = 128) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric int4 with one fp16 scale per ``group`` columns, two nibbles per byte.

    Follows ``python/cudallm/quantize.py:17-29``: s = max|group|/7 (1 if zero), rounded to
    fp16; q = clip(rint(w / fp32(s16)), -8, 7); u = q + 8; byte b = u[2b] | u[2b+1] << 4
    (even column in the low nibble).
    """
    w = np.asarray(w, dtype=np.float32)
    rows, cols = w.shape
    if cols % group or cols % 2:
        raise ValueError("cols must be a multiple of the group size and even")
    g = w.reshape(rows, cols // group, group)
    s = (np.abs(g).max(axis=2) / np.float32(7)).astype(np.float32)
    s[s == 0] = np.float32(1.0)
    s16 = s.astype(np.float16)
    q = np.clip(np.rint(g / s16.astype(np.float32)[:, :, None]), -8, 7).astype(np.int8).reshape(rows, cols)
    u = (q + 8).astype(np.uint8)
    packed = (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)
    return packed, s16


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """Inverse of the nibble packing (``python/cudallm/quantize.py:32-38``)."""
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty((p.shape[0], p.shape[1] * 2), dtype=np.int8)
    out[:, 0::2] = (p & 0x0F).astype(np.int8) - 8
    out[:, 1::2] = (p >> 4).astype(np.int8) - 8
    return out


def dequantize_int4_groups(packed: np.ndarray, s16: np.ndarray) -> np.ndarray:
    """``python/cudallm/quantize.py:41-47``."""
    q = unpack_int4(packed).astype(np.float32)
    rows, cols = q.shape
    ng = s16.shape[1]
    return (q.reshape(rows, ng, cols // ng) * s16.astype(np.float32)[:, :, None]).reshape(rows, cols)
