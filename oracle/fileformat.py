"""``.cudallm`` weight-file reader/writer, restated from the reference (test infrastructure only).

Layout (``src/model/cudallm_format.h:12-41``, ``python/cudallm/format.py:22-30``):

* 256-byte little-endian header: ``"CLLM"``, u32 version (1), u32 weight_dtype {1,3,4},
  u32 hidden, inter, layers, heads, kv_heads, head_dim, vocab, max_seq; f32 rms_eps,
  f32 rope_theta; u32 group_size, n_tensors, reserved; u64 table_offset (256); zero padding.
* n_tensors 80-byte entries: name[48] (NUL padded), u32 dtype {0 F32, 1 BF16, 2 F16, 3 I8,
  4 I4X2}, u32 rows, u32 cols (logical), u32 reserved, u64 offset (256-aligned), u64 nbytes.
* tensor data; zero padding only before each tensor; the file ends at the last tensor's end
  (``python/cudallm/format.py:94-101``).
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


def _align(n: int) -> int:
    return -(-n // ALIGN) * ALIGN


def nbytes_of(dtype: int, rows: int, cols: int) -> int:
    """``python/cudallm/format.py:37-47``; ``src/model/weights.cpp:37-46``."""
    per = {F32: 4.0, BF16: 2.0, F16: 2.0, I8: 1.0, I4X2: 0.5}[dtype]
    return int(rows * cols * per)


def tensor_names(n_layers: int, quant: bool) -> list[str]:
    """The fixed tensor order (``python/cudallm/format.py:50-67``; ``src/model/weights.cpp:66-81``)."""
    out = ["rope.inv_freq", "tok_embeddings.weight"] + (["tok_embeddings.scales"] if quant else [])
    out.append("norm.weight")
    for i in range(n_layers):
        p = f"layers.{i}."
        out.append(p + "attn_norm.weight")
        for lin in ("wqkv", "wo"):
            out += [p + lin + ".weight"] + ([p + lin + ".scales"] if quant else [])
        out.append(p + "ffn_norm.weight")
        for lin in ("w_gate_up", "w_down"):
            out += [p + lin + ".weight"] + ([p + lin + ".scales"] if quant else [])
    return out


def write(path, header: dict, tensors: list) -> None:
    """Write ``tensors`` = [(name, dtype, rows, cols, bytes)] (``python/cudallm/format.py:70-101``)."""
    entries = []
    off = _align(HEADER_SIZE + ENTRY_SIZE * len(tensors))
    for name, dt, rows, cols, data in tensors:
        nb = nbytes_of(dt, rows, cols)
        if len(data) != nb:
            raise ValueError(f"{name}: {len(data)} bytes, expected {nb}")
        entries.append(struct.pack(ENTRY_FMT, name.encode("ascii"), dt, rows, cols, 0, off, nb))
        off = _align(off + nb)
    hdr = struct.pack(HEADER_FMT, MAGIC, VERSION, header["weight_dtype"], header["hidden_size"],
                      header["intermediate_size"], header["n_layers"], header["n_heads"], header["n_kv_heads"],
                      header["head_dim"], header["vocab_size"], header["max_seq_len"], header["rms_eps"],
                      header["rope_theta"], header["group_size"], len(tensors), 0, HEADER_SIZE)
    with open(path, "wb") as f:
        f.write(hdr.ljust(HEADER_SIZE, b"\0"))
        for e in entries:
            f.write(e)
        for *_, data in tensors:
            f.write(b"\0" * (_align(f.tell()) - f.tell()))
            f.write(data)


def read_header(path) -> dict:
    raw = Path(path).open("rb").read(HEADER_SIZE)
    if len(raw) != HEADER_SIZE:
        raise ValueError(f"{path}: truncated header")
    return dict(zip(HEADER_FIELDS, struct.unpack_from(HEADER_FMT, raw)))


def read_table(path) -> list[dict]:
    hdr = read_header(path)
    with open(path, "rb") as f:
        f.seek(hdr["table_offset"])
        raw = f.read(ENTRY_SIZE * hdr["n_tensors"])
    out = []
    for k in range(hdr["n_tensors"]):
        name, dt, rows, cols, res, off, nb = struct.unpack_from(ENTRY_FMT, raw, k * ENTRY_SIZE)
        out.append(dict(name=name.rstrip(b"\0").decode("ascii"), dtype=dt, rows=rows, cols=cols, reserved=res,
                        offset=off, nbytes=nb))
    return out


def load(path, e: dict) -> np.ndarray:
    """Memory-map one tensor as stored (``python/cudallm/format.py:124-140``)."""
    np_dt, shape = {F32: (np.float32, (e["rows"], e["cols"])), BF16: (np.uint16, (e["rows"], e["cols"])),
                    F16: (np.float16, (e["rows"], e["cols"])), I8: (np.int8, (e["rows"], e["cols"])),
                    I4X2: (np.uint8, (e["rows"], e["cols"] // 2))}[e["dtype"]]
    a = np.memmap(path, dtype=np_dt, mode="r", offset=e["offset"], shape=shape)
    if e["dtype"] == F32 and e["cols"] == 1:
        a = a.reshape(e["rows"])
    return a
