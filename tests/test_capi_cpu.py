"""CPU lane for the C ABI: the library loads, exports every declared symbol with the reference's
struct layouts, and rejects bad files and bad arguments with the reference's error codes before it
touches a device (reference src/capi/cudallm_capi.cpp:24-316, src/model/weights.cpp:99-157)."""
import ctypes
import re
import struct
import threading
from pathlib import Path

import numpy as np
import pytest

from cudallm_amd import engine as E
from cudallm_amd import format as pf

HEADER_H = Path(__file__).resolve().parents[1] / "include" / "cudallm" / "cudallm.h"
OK, INVALID_ARG, IO, FORMAT, DEVICE, STATE, INTERNAL = range(7)


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER_H.read_text(), flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(cudallm_\w+)\s*\(", text, flags=re.M)


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 18
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(E.SIGNATURES)


def test_struct_layouts():
    assert ctypes.sizeof(E.CudallmOptions) == 24
    assert ctypes.sizeof(E.CudallmConfigInfo) == 56 and E.CudallmConfigInfo.weight_bytes.offset == 48
    assert E.CudallmConfigInfo.rms_eps.offset == 40


def test_default_options(lib):
    o = E.CudallmOptions(9, 9, 9, 9, 9, 9)
    lib.cudallm_default_options(ctypes.byref(o))
    assert [getattr(o, f) for f, _ in o._fields_] == [1, 1, 1, 1, 0, 0]
    lib.cudallm_default_options(None)  # NULL-safe


def _create(lib, path, **kw):
    o = E.CudallmOptions()
    lib.cudallm_default_options(ctypes.byref(o))
    for k, v in kw.items():
        setattr(o, k, v)
    h = ctypes.c_void_p(123)
    rc = lib.cudallm_create(str(path).encode(), ctypes.byref(o), ctypes.byref(h))
    return rc, h.value, lib.cudallm_last_error().decode()


def test_create_missing_file_is_io(lib, tmp_path):
    rc, h, msg = _create(lib, tmp_path / "none.cudallm")
    assert rc == IO and h is None and "cannot open" in msg


def test_null_arguments(lib):
    assert lib.cudallm_create(None, None, None) == INVALID_ARG
    assert lib.cudallm_pos(None) == -1 and "null engine" in lib.cudallm_last_error().decode()
    assert lib.cudallm_reset(None) == INVALID_ARG
    assert lib.cudallm_step(None, 0, None, None) == INVALID_ARG
    assert lib.cudallm_get_config(None, None) == INVALID_ARG
    s = ctypes.c_void_p(0)
    assert lib.cudallm_get_stream(None, ctypes.byref(s)) == INVALID_ARG and s.value is None
    kind, grid = ctypes.c_int(7), ctypes.c_int(7)
    assert lib.cudallm_get_step_kind(None, ctypes.byref(kind), ctypes.byref(grid)) == INVALID_ARG
    assert kind.value == -1 and grid.value == 0
    lib.cudallm_destroy(None)


def test_last_error_is_thread_local(lib, tmp_path):
    _create(lib, tmp_path / "main.cudallm")
    seen = {}

    def other():
        seen["before"] = lib.cudallm_last_error().decode()
        _create(lib, tmp_path / "thread.cudallm")
        seen["after"] = lib.cudallm_last_error().decode()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["before"] == "" and "thread.cudallm" in seen["after"]
    assert "main.cudallm" in lib.cudallm_last_error().decode()


# ---- loader validation: a header + table with every field right, then one field wrong ------

def _llama_specs(wd):
    from cudallm_amd import synth
    return synth._specs(wd, synth.LLAMA_1B)


def write_header_table(path, wd="bf16", header_edit=None, entry_edit=None, data_bytes=0):
    """Header and table of a valid Llama-3.2-1B file; tensor data truncated to data_bytes."""
    specs = _llama_specs(wd)
    h = dict(weight_dtype={"bf16": 1, "int8": 3, "int4": 4}[wd], hidden_size=2048, intermediate_size=8192,
             n_layers=16, n_heads=32, n_kv_heads=8, head_dim=64, vocab_size=128256, max_seq_len=4096, rms_eps=1e-5,
             rope_theta=500000.0, group_size=128 if wd == "int4" else 0, n_tensors=len(specs), table_offset=256,
             magic=b"CLLM", version=1)
    if header_edit:
        header_edit(h)
    raw = struct.pack(pf.HEADER_FMT, h["magic"], h["version"], h["weight_dtype"], h["hidden_size"],
                      h["intermediate_size"], h["n_layers"], h["n_heads"], h["n_kv_heads"], h["head_dim"],
                      h["vocab_size"], h["max_seq_len"], h["rms_eps"], h["rope_theta"], h["group_size"],
                      h["n_tensors"], 0, h["table_offset"])
    raw = raw.ljust(256, b"\0")
    off = (256 + 80 * len(specs) + 255) // 256 * 256
    entries = []
    for i, (name, dt, rows, cols) in enumerate(specs):
        e = dict(name=name, dtype=dt, rows=rows, cols=cols, offset=off, nbytes=pf.expected_nbytes(dt, rows, cols))
        if entry_edit:
            entry_edit(i, e)
        entries.append(struct.pack(pf.ENTRY_FMT, e["name"].encode(), e["dtype"], e["rows"], e["cols"], 0,
                                   e["offset"], e["nbytes"]))
        off = (off + pf.expected_nbytes(dt, rows, cols) + 255) // 256 * 256
    with open(path, "wb") as f:
        f.write(raw + b"".join(entries))
        f.write(b"\0" * data_bytes)


def _set(key, val):
    def edit(h):
        h[key] = val
    return edit


@pytest.mark.parametrize("edit,needle", [
    (_set("magic", b"GGUF"), "bad magic"),
    (_set("version", 2), "version"),
    (_set("weight_dtype", 2), "weight_dtype"),
    (_set("hidden_size", 4096), "hidden_size"),
    (_set("intermediate_size", 14336), "intermediate_size"),
    (_set("n_layers", 32), "n_layers"),
    (_set("n_heads", 64), "n_heads"),
    (_set("n_kv_heads", 4), "n_kv_heads"),
    (_set("head_dim", 128), "head_dim"),
    (_set("vocab_size", 32000), "vocab_size"),
    (_set("max_seq_len", 100), "max_seq_len"),
    (_set("max_seq_len", 0), "max_seq_len"),
    (_set("n_tensors", 98), "n_tensors"),
    (_set("table_offset", 512), "table_offset"),
    (_set("group_size", 64), "group_size"),
])
def test_header_errors_are_format(lib, tmp_path, edit, needle):
    p = tmp_path / "bad.cudallm"
    write_header_table(p, header_edit=edit)
    rc, h, msg = _create(lib, p)
    assert rc == FORMAT and h is None and needle in msg, msg


def _entry(index, key, val):
    def edit(i, e):
        if i == index:
            e[key] = val
    return edit


def _shift(index, delta):
    def edit(i, e):
        if i == index:
            e["offset"] += delta
    return edit


@pytest.mark.parametrize("wd,edit,needle", [
    ("bf16", _entry(1, "name", "tok_embeddings.scales"), "expected 'tok_embeddings.weight'"),
    ("int8", _entry(2, "dtype", 2), "dtype or shape"),
    ("int4", _entry(3, "cols", 16), "dtype or shape"),
    ("bf16", _shift(4, 8), "aligned"),
    ("bf16", _entry(5, "offset", 256), "overlaps"),
    ("int8", _entry(6, "nbytes", 1), "nbytes"),
])
def test_table_errors_are_format(lib, tmp_path, wd, edit, needle):
    p = tmp_path / "bad.cudallm"
    write_header_table(p, wd, entry_edit=edit)
    rc, _, msg = _create(lib, p)
    assert rc == FORMAT and needle in msg, msg


@pytest.mark.parametrize("wd", ["bf16", "int8", "int4"])
def test_truncated_data_is_format(lib, tmp_path, wd):
    p = tmp_path / "trunc.cudallm"
    write_header_table(p, wd, data_bytes=1000)
    rc, _, msg = _create(lib, p)
    assert rc == FORMAT and "truncated" in msg, msg


def test_short_files(lib, tmp_path):
    p = tmp_path / "short.cudallm"
    p.write_bytes(b"CLLM")
    assert _create(lib, p)[0] == FORMAT
    write_header_table(p)
    p.write_bytes(p.read_bytes()[:1000])
    rc, _, msg = _create(lib, p)
    assert rc == FORMAT and "table" in msg


@pytest.mark.parametrize("opts,needle", [
    (dict(matvec_impl=2), "matvec_impl"),
    (dict(attn_impl=-1), "attn_impl"),
    (dict(matvec_impl=0, fuse=1), "naive"),
    (dict(matvec_rpb=3), "matvec_rpb"),
    (dict(max_seq_len=100), "max_seq_len"),
    (dict(max_seq_len=8192), "exceeds"),
])
def test_option_errors_are_invalid_arg(lib, tmp_path, opts, needle):
    """Options are validated after the file, before any device work (a truncated-but-valid table
    would otherwise report FORMAT; so the data region here is complete for a header-only check)."""
    p = tmp_path / "ok_header.cudallm"
    write_header_table(p)
    # Make the data region present (sparse file) so file validation passes.
    table = pf.read_table(p)
    with open(p, "r+b") as f:
        f.truncate(table[-1]["offset"] + table[-1]["nbytes"])
    rc, _, msg = _create(lib, p, **opts)
    assert rc == INVALID_ARG and needle in msg, msg


def test_naive_matvec_needs_bf16(lib, tmp_path):
    p = tmp_path / "int8.cudallm"
    write_header_table(p, "int8")
    table = pf.read_table(p)
    with open(p, "r+b") as f:
        f.truncate(table[-1]["offset"] + table[-1]["nbytes"])
    rc, _, msg = _create(lib, p, matvec_impl=0, fuse=0)
    assert rc == INVALID_ARG and "bf16" in msg


# ---- kernel hooks: argument checks happen before any device call --------------------------

def test_matvec_hook_argument_errors(lib):
    w = np.zeros((4, 1024), dtype=np.uint16)
    x = np.zeros(1024, dtype=np.float32)
    with pytest.raises(E.CudaLLMError) as ei:
        E.kernel_matvec("naive", "int8", "store", 0, 0, w, np.ones(4, np.float32), x, None, 1e-5, None, 4, 1024)
    assert ei.value.code == INVALID_ARG
    with pytest.raises(E.CudaLLMError) as ei:
        E.kernel_matvec("opt", 2, "store", 0, 0, w, None, x, None, 1e-5, None, 4, 1024)
    assert ei.value.code == INVALID_ARG and "weight_dtype" in str(ei.value)
    with pytest.raises(E.CudaLLMError) as ei:
        E.kernel_matvec("opt", "int8", "store", 0, 0, w, None, x, None, 1e-5, None, 4, 1024)
    assert ei.value.code == INVALID_ARG and "scales" in str(ei.value)
    with pytest.raises(E.CudaLLMError) as ei:
        E.kernel_matvec("opt", "bf16", 3, 0, 0, w, None, x, None, 1e-5, None, 4, 1024)
    assert ei.value.code == INVALID_ARG
    with pytest.raises(E.CudaLLMError) as ei:  # buffer smaller than the shape
        E.kernel_matvec("opt", "bf16", "store", 0, 0, w, None, x, None, 1e-5, None, 8, 1024)
    assert ei.value.code == INVALID_ARG and "w_bytes" in str(ei.value)
    with pytest.raises(E.CudaLLMError) as ei:
        E.kernel_matvec("opt", "bf16", "store", 1, 0, w, None, x, None, 1e-5, None, 4, 1024)
    assert ei.value.code == INVALID_ARG and "norm_w" in str(ei.value)


def test_stream_read_hook_argument_errors(lib):
    ev = ctypes.c_void_p(1)
    assert lib.cudallm_launch_stream_read_timed(None, 1 << 20, 8, ctypes.c_void_p(1), 4096, None, ev, ev) == INVALID_ARG
    assert lib.cudallm_launch_stream_read_timed(ctypes.c_void_p(1), 1000, 8, ctypes.c_void_p(1), 4096, None, ev,
                                                ev) == INVALID_ARG
    assert lib.cudallm_launch_stream_read_timed(ctypes.c_void_p(1), 1 << 20, 3, ctypes.c_void_p(1), 4096, None, ev,
                                                ev) == INVALID_ARG
    assert "blocks_per_cu" in lib.cudallm_last_error().decode()
    assert lib.cudallm_launch_stream_read_timed(ctypes.c_void_p(1), 1 << 20, 8, ctypes.c_void_p(1), 4096, None, None,
                                                ev) == INVALID_ARG
    assert "start_event" in lib.cudallm_last_error().decode()


def test_other_hook_argument_errors(lib):
    q = np.zeros(32 * 64, np.float32)
    kc = np.zeros((8, 128, 64), np.float16)
    with pytest.raises(E.CudaLLMError) as ei:
        E.kernel_attention("opt", q, kc, kc, 0, 32, 8, 64, 128)
    assert ei.value.code == INVALID_ARG
    with pytest.raises(E.CudaLLMError) as ei:
        E.kernel_attention(2, q, kc, kc, 1, 32, 8, 64, 128)
    assert ei.value.code == INVALID_ARG
    qkv = np.zeros(48 * 64, np.float32)
    with pytest.raises(E.CudaLLMError) as ei:
        E.kernel_rope_kv(1, qkv, np.ones(32, np.float32), 128, kc, kc, 32, 8, 64, 128)
    assert ei.value.code == INVALID_ARG
    with pytest.raises(E.CudaLLMError) as ei:
        E.kernel_argmax(np.zeros(0, np.float32))
    assert ei.value.code == INVALID_ARG


def test_bench_suites_mirror_the_reference():
    """The decode suites follow the reference's bench/bench_decode.py:12-26 (names, options, lengths) and its
    prompt (src/tools/cudallm_bench.cpp:24)."""
    from cudallm_amd import bench_decode as B
    assert [e[0] for e in B.ABLATION] == ["A0_naive", "A1_matvec_opt", "A2_attn_opt", "A3_fused", "A4_graph_nofuse",
                                          "A5_full"]
    assert B.ABLATION[0][1:] == ("bf16", "naive", "naive", 0, 0, 128, 256, 5)
    assert B.ABLATION[-1][1:] == ("bf16", "opt", "opt", 1, 1, 128, 256, 5)
    assert [e[0] for e in B.QUANT] == ["Q_bf16", "Q_int8", "Q_int4"]
    assert [e[6] for e in B.CONTEXT] == [128, 128, 512, 512, 1024, 1024, 2048, 2048, 4000, 4000]
    assert all(e[7] == 32 and e[8] == 3 for e in B.CONTEXT)
    assert [e[6:8] for e in B.TG] == [(1, 256)] * 3
    assert all(e[6] + e[7] <= B.LONG_MAX_SEQ for e in B.LONG)
    assert [B.prompt_token(i) for i in (0, 1, 2, 15152)] == [128000, 8919, 16838, 1000 + (15152 * 7919) % 120000]
