"""Reader/writer for the ``.cudallm`` weight-file format.

The format is the reference's (``src/model/cudallm_format.h:12-41``, ``python/cudallm/format.py:7-147``): a 256-byte
header, 80-byte tensor entries, 256-byte aligned tensor data with zero padding only before each tensor; the constants
below are that format.  The function names are those the reference's Python tools call; the parsing is numpy
record types, and the writer streams one tensor at a time.
"""
import struct
from pathlib import Path

import numpy as np

MAGIC = b"CLLM"
VERSION = 1

F32, BF16, F16, I8, I4X2 = 0, 1, 2, 3, 4
WEIGHT_BF16, WEIGHT_INT8, WEIGHT_INT4 = 1, 3, 4

HEADER_FMT = "<4s10I2f3IQ"
HEADER_SIZE = 256
ENTRY_FMT = "<48s4I2Q"
ENTRY_SIZE = 80
ALIGN = 256

HEADER_FIELDS = ("magic", "version", "weight_dtype", "hidden_size", "intermediate_size", "n_layers",
                 "n_heads", "n_kv_heads", "head_dim", "vocab_size", "max_seq_len", "rms_eps",
                 "rope_theta", "group_size", "n_tensors", "reserved0", "table_offset")

assert struct.calcsize(HEADER_FMT) == 72 and struct.calcsize(ENTRY_FMT) == ENTRY_SIZE


def _align(n: int) -> int:
    return (n + ALIGN - 1) // ALIGN * ALIGN


# Storage of each tensor dtype code: (numpy dtype of one stored element, logical columns per stored element).
_STORAGE = {F32: (np.dtype("<f4"), 1), BF16: (np.dtype("<u2"), 1), F16: (np.dtype("<f2"), 1), I8: (np.dtype("i1"), 1),
            I4X2: (np.dtype("u1"), 2)}


def expected_nbytes(dtype: int, rows: int, cols: int) -> int:
    """Bytes of a rows x cols tensor of `dtype` (I4X2 packs two columns per byte, so cols must be even)."""
    if dtype not in _STORAGE:
        raise ValueError(f"tensor dtype code {dtype} is not one of F32, BF16, F16, I8, I4X2")
    np_dt, per = _STORAGE[dtype]
    if cols % per:
        raise ValueError(f"dtype code {dtype} stores {per} columns per byte; {cols} columns do not divide")
    return rows * (cols // per) * np_dt.itemsize


def expected_names(n_layers: int, quant: bool) -> list[str]:
    """The fixed tensor sequence (src/model/weights.cpp:66-81): every linear is `.weight`, plus `.scales` when the
    file is quantised."""
    def linear(name):
        return [name + ".weight", name + ".scales"] if quant else [name + ".weight"]
    names = ["rope.inv_freq", *linear("tok_embeddings"), "norm.weight"]
    for i in range(n_layers):
        p = f"layers.{i}."
        names += [p + "attn_norm.weight", *linear(p + "wqkv"), *linear(p + "wo"), p + "ffn_norm.weight",
                  *linear(p + "w_gate_up"), *linear(p + "w_down")]
    return names


class Writer:
    """Streams a ``.cudallm`` file: header and table first, then tensor data as it is produced.

    ``specs`` = [(name, dtype, rows, cols)] fixes the table; ``write(data)`` must then be called
    once per tensor in that order.  Memory stays bounded by one tensor.
    """

    def __init__(self, path, header: dict, specs: list[tuple[str, int, int, int]]):
        self._f = open(path, "wb")
        self._specs, self._next = specs, 0
        entries, off = [], _align(HEADER_SIZE + ENTRY_SIZE * len(specs))
        for name, dtype, rows, cols in specs:
            nb = expected_nbytes(dtype, rows, cols)
            name_b = name.encode("ascii")
            if len(name_b) >= 48:
                raise ValueError(f"name too long: {name}")
            entries.append(struct.pack(ENTRY_FMT, name_b, dtype, rows, cols, 0, off, nb))
            off = _align(off + nb)
        hdr = struct.pack(HEADER_FMT, MAGIC, VERSION, header["weight_dtype"], header["hidden_size"],
                          header["intermediate_size"], header["n_layers"], header["n_heads"], header["n_kv_heads"],
                          header["head_dim"], header["vocab_size"], header["max_seq_len"], header["rms_eps"],
                          header["rope_theta"], header["group_size"], len(specs), 0, HEADER_SIZE)
        self._f.write(hdr + b"\0" * (HEADER_SIZE - len(hdr)))
        for e in entries:
            self._f.write(e)

    def write(self, data) -> None:
        name, dtype, rows, cols = self._specs[self._next]
        mv = memoryview(data).cast("B")
        if mv.nbytes != expected_nbytes(dtype, rows, cols):
            raise ValueError(f"{name}: {mv.nbytes} bytes, expected {expected_nbytes(dtype, rows, cols)}")
        pos = self._f.tell()
        self._f.write(b"\0" * (_align(pos) - pos))
        self._f.write(mv)
        self._next += 1

    def close(self) -> None:
        if self._next != len(self._specs):
            self._f.close()
            raise ValueError(f"only {self._next} of {len(self._specs)} tensors written")
        self._f.close()


def write_cudallm(path, header: dict, tensors: list[tuple[str, int, int, int, bytes]]) -> None:
    """Write a whole file (``python/cudallm/format.py:70-101``)."""
    w = Writer(path, header, [t[:4] for t in tensors])
    for t in tensors:
        w.write(t[4])
    w.close()


# The header and table entries as numpy record types (little-endian, packed), the same layout as HEADER_FMT /
# ENTRY_FMT: one np.frombuffer / np.fromfile call parses them.
_HEADER_DT = np.dtype([("magic", "S4"), ("version", "<u4"), ("weight_dtype", "<u4"), ("hidden_size", "<u4"),
                       ("intermediate_size", "<u4"), ("n_layers", "<u4"), ("n_heads", "<u4"), ("n_kv_heads", "<u4"),
                       ("head_dim", "<u4"), ("vocab_size", "<u4"), ("max_seq_len", "<u4"), ("rms_eps", "<f4"),
                       ("rope_theta", "<f4"), ("group_size", "<u4"), ("n_tensors", "<u4"), ("reserved0", "<u4"),
                       ("table_offset", "<u8")])
_ENTRY_DT = np.dtype([("name", "S48"), ("dtype", "<u4"), ("rows", "<u4"), ("cols", "<u4"), ("reserved", "<u4"),
                      ("offset", "<u8"), ("nbytes", "<u8")])
assert _HEADER_DT.itemsize == struct.calcsize(HEADER_FMT) and _ENTRY_DT.itemsize == ENTRY_SIZE


def _python(v):
    return v.item() if hasattr(v, "item") else v


def read_header(path) -> dict:
    """The header's fields by name (HEADER_FIELDS), as Python numbers (magic stays bytes)."""
    with open(path, "rb") as f:
        raw = f.read(HEADER_SIZE)
    if len(raw) < HEADER_SIZE:
        raise ValueError(f"{path}: file ends inside the {HEADER_SIZE}-byte header ({len(raw)} bytes)")
    rec = np.frombuffer(raw, dtype=_HEADER_DT, count=1)[0]
    return {name: _python(rec[name]) for name in HEADER_FIELDS}


def read_table(path) -> list[dict]:
    """The tensor entries in file order, each a dict with name, dtype, rows, cols, reserved, offset, nbytes."""
    hdr = read_header(path)
    n = hdr["n_tensors"]
    recs = np.fromfile(path, dtype=_ENTRY_DT, count=n, offset=hdr["table_offset"])
    if len(recs) != n:
        raise ValueError(f"{path}: the table should hold {n} entries but the file ends after {len(recs)}")
    table = []
    for rec in recs:
        e = {f: _python(rec[f]) for f in _ENTRY_DT.names}
        e["name"] = rec["name"].split(b"\0", 1)[0].decode("ascii")
        table.append(e)
    return table


def load_tensor(path, entry: dict) -> np.ndarray:
    """One tensor as stored: F32 [rows, cols] (a vector when cols == 1), BF16 as uint16 bits, F16, I8, and I4X2
    as uint8 [rows, cols / 2]."""
    np_dt, per = _STORAGE[entry["dtype"]]
    rows, cols = entry["rows"], entry["cols"]
    out = np.empty((rows, cols // per), dtype=np_dt)
    with open(path, "rb") as f:
        f.seek(entry["offset"])
        got = f.readinto(memoryview(out).cast("B"))
    if got != out.nbytes:
        raise ValueError(f"{path}: {entry['name']} needs {out.nbytes} bytes at offset {entry['offset']}, "
                         f"the file holds {got}")
    return out.reshape(rows) if entry["dtype"] == F32 and cols == 1 else out
