"""Reader/writer for the ``.cudallm`` weight-file format.

Same format and function names as the reference's ``python/cudallm/format.py:7-147``
(``src/model/cudallm_format.h:12-41``): a 256-byte header, 80-byte tensor entries, 256-byte
aligned tensor data with zero padding only before each tensor.
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


def expected_nbytes(dtype: int, rows: int, cols: int) -> int:
    if dtype == F32:
        return rows * cols * 4
    if dtype in (BF16, F16):
        return rows * cols * 2
    if dtype == I8:
        return rows * cols
    if dtype == I4X2:
        if cols % 2:
            raise ValueError("I4X2 needs an even column count")
        return rows * cols // 2
    raise ValueError(f"unknown dtype code {dtype}")


def expected_names(n_layers: int, quant: bool) -> list[str]:
    names = ["rope.inv_freq", "tok_embeddings.weight"] + (["tok_embeddings.scales"] if quant else []) + ["norm.weight"]
    for i in range(n_layers):
        p = f"layers.{i}."
        names.append(p + "attn_norm.weight")
        for lin in ("wqkv", "wo"):
            names += [p + lin + ".weight"] + ([p + lin + ".scales"] if quant else [])
        names.append(p + "ffn_norm.weight")
        for lin in ("w_gate_up", "w_down"):
            names += [p + lin + ".weight"] + ([p + lin + ".scales"] if quant else [])
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


def read_header(path) -> dict:
    with open(path, "rb") as f:
        raw = f.read(HEADER_SIZE)
    if len(raw) != HEADER_SIZE:
        raise ValueError(f"{path}: truncated header")
    return dict(zip(HEADER_FIELDS, struct.unpack(HEADER_FMT, raw[:struct.calcsize(HEADER_FMT)])))


def read_table(path) -> list[dict]:
    hdr = read_header(path)
    with open(path, "rb") as f:
        f.seek(hdr["table_offset"])
        raw = f.read(ENTRY_SIZE * hdr["n_tensors"])
    out = []
    for k in range(hdr["n_tensors"]):
        name, dtype, rows, cols, reserved, offset, nbytes = struct.unpack_from(ENTRY_FMT, raw, k * ENTRY_SIZE)
        out.append({"name": name.rstrip(b"\0").decode("ascii"), "dtype": dtype, "rows": rows, "cols": cols,
                    "reserved": reserved, "offset": offset, "nbytes": nbytes})
    return out


def load_tensor(path, entry: dict) -> np.ndarray:
    rows, cols, dtype = entry["rows"], entry["cols"], entry["dtype"]
    np_dtype, shape = {F32: (np.float32, (rows, cols)), BF16: (np.uint16, (rows, cols)),
                       F16: (np.float16, (rows, cols)), I8: (np.int8, (rows, cols)),
                       I4X2: (np.uint8, (rows, cols // 2))}[dtype]
    count = shape[0] * shape[1]
    arr = np.fromfile(path, dtype=np_dtype, count=count, offset=entry["offset"])
    if arr.size != count:
        raise ValueError(f"{path}: truncated tensor {entry['name']}")
    arr = arr.reshape(shape)
    return arr.reshape(rows) if dtype == F32 and cols == 1 else arr


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)
