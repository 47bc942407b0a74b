"""Seeded synthetic Llama-3.2-1B-shaped ``.cudallm`` files (random init, no checkpoint needed).

The tensor list is the one the reference's exporter writes (``python/cudallm/export.py:85-159``):
fused ``wqkv`` (q|k|v rows) and ``w_gate_up`` (gate|up rows), tied embeddings, Llama-3 scaled
``rope.inv_freq``.  Every linear and the embedding is a bf16 master drawn N(0, 0.02) with torch's
generator on the GPU; int8 / int4 files quantise that master (upcast to fp32, as ``export.py:90``
does) with the GPU quantisers of this package.  Norm weights are 1.0 (HF initialisation) or seeded U(0.5, 1.5).
The file is streamed tensor by tensor, so host memory stays bounded by the largest tensor.
"""
import math

import numpy as np
import torch

from . import format as fmt
from . import quantize as qz

LLAMA_1B = dict(hidden_size=2048, intermediate_size=8192, n_layers=16, n_heads=32, n_kv_heads=8, head_dim=64,
                vocab_size=128256, max_seq_len=4096, rms_eps=1e-5, rope_theta=500000.0)


def llama3_inv_freq(head_dim: int = 64, theta: float = 500000.0, factor: float = 32.0, low: float = 1.0,
                    high: float = 4.0, orig: int = 8192) -> np.ndarray:
    """Llama-3 RoPE frequency scaling (the rope_scaling of Llama-3.2: factor 32, low 1, high 4,
    original context 8192), evaluated in float64 and stored as fp32."""
    out = np.empty(head_dim // 2, dtype=np.float64)
    for i in range(head_dim // 2):
        f = 1.0 / theta ** (2 * i / head_dim)
        wl = 2 * math.pi / f
        if wl < orig / high:
            out[i] = f
        elif wl > orig / low:
            out[i] = f / factor
        else:
            t = (orig / wl - low) / (high - low)
            out[i] = (1 - t) * f / factor + t * f
    return out.astype(np.float32)


def _specs(wdtype: str, d: dict) -> list[tuple[str, int, int, int]]:
    H, I, L = d["hidden_size"], d["intermediate_size"], d["n_layers"]
    QKV = (d["n_heads"] + 2 * d["n_kv_heads"]) * d["head_dim"]

    def lin(name, rows, cols):
        if wdtype == "bf16":
            return [(name + ".weight", fmt.BF16, rows, cols)]
        if wdtype == "int8":
            return [(name + ".weight", fmt.I8, rows, cols), (name + ".scales", fmt.F32, rows, 1)]
        return [(name + ".weight", fmt.I4X2, rows, cols), (name + ".scales", fmt.F16, rows, cols // 128)]

    s = [("rope.inv_freq", fmt.F32, d["head_dim"] // 2, 1)] + lin("tok_embeddings", d["vocab_size"], H)
    s.append(("norm.weight", fmt.F32, H, 1))
    for i in range(L):
        p = f"layers.{i}."
        s.append((p + "attn_norm.weight", fmt.F32, H, 1))
        s += lin(p + "wqkv", QKV, H) + lin(p + "wo", H, d["n_heads"] * d["head_dim"])
        s.append((p + "ffn_norm.weight", fmt.F32, H, 1))
        s += lin(p + "w_gate_up", 2 * I, H) + lin(p + "w_down", H, I)
    return s


def write_model(path, wdtype: str, seed: int = 0, device: str | None = None, max_seq_len: int | None = None,
                norm: str = "ones") -> int:
    """Write a seeded Llama-3.2-1B-shaped model; returns the file's weight bytes (sum of nbytes).

    The bf16 master depends only on ``seed`` (and the device's generator), not on ``wdtype``.
    ``max_seq_len`` (default 4096) is the header's context limit; the weights do not depend on it.
    ``norm``: "ones" (HF initialisation) or "random" (U(0.5, 1.5) from a numpy generator seeded with ``seed``,
    so that a test can tell the norm weights of different layers apart).
    """
    if norm not in ("ones", "random"):
        raise ValueError("norm must be 'ones' or 'random'")
    norm_rng = np.random.default_rng(seed)
    if wdtype not in ("bf16", "int8", "int4"):
        raise ValueError("wdtype must be bf16, int8 or int4")
    d = dict(LLAMA_1B)
    if max_seq_len is not None:
        if max_seq_len <= 0 or max_seq_len % 128:
            raise ValueError("max_seq_len must be a positive multiple of 128")
        d["max_seq_len"] = int(max_seq_len)
    dev = torch.device(device or ("cuda" if torch.cuda.is_available() else "cpu"))
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    specs = _specs(wdtype, d)
    header = dict(d, weight_dtype={"bf16": fmt.WEIGHT_BF16, "int8": fmt.WEIGHT_INT8, "int4": fmt.WEIGHT_INT4}[wdtype],
                  group_size=128 if wdtype == "int4" else 0)
    w = fmt.Writer(path, header, specs)
    total = 0
    i = 0
    while i < len(specs):
        name, dtype, rows, cols = specs[i]
        if dtype == fmt.F32:
            if name == "rope.inv_freq":
                a = llama3_inv_freq(d["head_dim"], d["rope_theta"])
            elif norm == "random":
                a = norm_rng.uniform(0.5, 1.5, rows).astype(np.float32)
            else:
                a = np.ones(rows, np.float32)
            w.write(a.tobytes())
            total += a.nbytes
            i += 1
            continue
        master = (torch.randn(rows, cols, generator=gen, device=dev, dtype=torch.float32) * 0.02).to(torch.bfloat16)
        if wdtype == "bf16":
            bits = master.view(torch.int16).cpu().numpy()
            w.write(bits.tobytes())
            total += bits.nbytes
            i += 1
            continue
        w32 = master.float().cpu().numpy()
        del master
        if wdtype == "int8":
            q, s = qz.quantize_int8_rows(w32)
        else:
            q, s = qz.quantize_int4_groups(w32, 128)
        del w32
        w.write(q.tobytes())
        w.write(s.tobytes())
        total += q.nbytes + s.nbytes
        i += 2
    w.close()
    return total
