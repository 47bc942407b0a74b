"""Seeded synthetic ``.cudallm`` files for the parity tests (test infrastructure only).

The tensors are those ``python/cudallm/export.py:85-159`` writes (fused ``wqkv`` = q|k|v rows and
``w_gate_up`` = gate|up rows, tied embeddings, Llama-3 ``rope.inv_freq``), drawn from a seeded
generator instead of a checkpoint: every linear and the embedding is N(0, 0.02) rounded to bf16
(the bf16 master); int8/int4 files quantise that master upcast to fp32 as ``export.py:90`` does.
Norm weights are 1.0 (HF initialisation) or, with ``norm="random"``, U(0.5, 1.5).
"""
import numpy as np

from . import fileformat as ff
from . import quantize as qz
from .kernels import llama3_inv_freq

LLAMA_1B = dict(hidden_size=2048, intermediate_size=8192, n_layers=16, n_heads=32, n_kv_heads=8, head_dim=64,
                vocab_size=128256, max_seq_len=4096, rms_eps=1e-5, rope_theta=500000.0)
TINY = dict(hidden_size=256, intermediate_size=512, n_layers=2, n_heads=4, n_kv_heads=1, head_dim=64,
            vocab_size=1000, max_seq_len=128, rms_eps=1e-5, rope_theta=500000.0)


def _master(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    return qz.bf16_round_bits(rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02))


def _linear(name: str, bits: np.ndarray, wdtype: str) -> list:
    rows, cols = bits.shape
    if wdtype == "bf16":
        return [(name + ".weight", ff.BF16, rows, cols, bits.tobytes())]
    w = qz.bf16_bits_to_f32(bits)
    if wdtype == "int8":
        q, s = qz.quantize_int8_rows(w)
        return [(name + ".weight", ff.I8, rows, cols, q.tobytes()), (name + ".scales", ff.F32, rows, 1, s.tobytes())]
    p, s = qz.quantize_int4_groups(w, 128)
    return [(name + ".weight", ff.I4X2, rows, cols, p.tobytes()),
            (name + ".scales", ff.F16, rows, cols // 128, s.tobytes())]


def write_model(path, wdtype: str, seed: int = 0, dims: dict | None = None, norm: str = "ones") -> None:
    """Write a seeded model; the bf16 master depends only on (seed, dims), not on ``wdtype``."""
    d = dict(LLAMA_1B if dims is None else dims)
    H, I, L = d["hidden_size"], d["intermediate_size"], d["n_layers"]
    NH, KV, D, V = d["n_heads"], d["n_kv_heads"], d["head_dim"], d["vocab_size"]
    ss = np.random.SeedSequence(seed)
    streams = iter(ss.spawn(2 + 6 * L))

    def normw(n):
        r = np.random.default_rng(next(streams))
        return np.ones(n, dtype=np.float32) if norm == "ones" else r.uniform(0.5, 1.5, n).astype(np.float32)

    def vec(name, a):
        return (name, ff.F32, a.shape[0], 1, a.astype(np.float32).tobytes())

    t = [vec("rope.inv_freq", llama3_inv_freq(D, d["rope_theta"]))]
    t += _linear("tok_embeddings", _master(np.random.default_rng(next(streams)), V, H), wdtype)
    t.append(vec("norm.weight", normw(H)))
    for i in range(L):
        p = f"layers.{i}."
        t.append(vec(p + "attn_norm.weight", normw(H)))
        t += _linear(p + "wqkv", _master(np.random.default_rng(next(streams)), (NH + 2 * KV) * D, H), wdtype)
        t += _linear(p + "wo", _master(np.random.default_rng(next(streams)), H, NH * D), wdtype)
        t.append(vec(p + "ffn_norm.weight", normw(H)))
        t += _linear(p + "w_gate_up", _master(np.random.default_rng(next(streams)), 2 * I, H), wdtype)
        t += _linear(p + "w_down", _master(np.random.default_rng(next(streams)), H, I), wdtype)
    hdr = dict(d, weight_dtype={"bf16": ff.WEIGHT_BF16, "int8": ff.WEIGHT_INT8, "int4": ff.WEIGHT_INT4}[wdtype],
               group_size=128 if wdtype == "int4" else 0)
    ff.write(path, hdr, t)
