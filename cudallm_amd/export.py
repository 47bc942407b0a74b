"""Convert a Hugging Face Llama-3.2-1B(-Instruct) checkpoint to a .cudallm file.

    python -m cudallm_amd.export --hf-dir DIR --out FILE --dtype {bf16,int8,int4}

Same command line, checks, tensor list and tensor order as the reference's exporter
(``python/cudallm/export.py:22-175``): q|k|v rows fused into ``wqkv``, gate|up rows into ``w_gate_up``,
norm weights as fp32 columns, tied embeddings (no ``lm_head.weight``), ``rope.inv_freq`` from
transformers' own Llama-3 rope initialisation (``ROPE_INIT_FUNCTIONS["llama3"]``), ``max_seq_len`` 4096.
Quantised files use this package's quantisers (bit-identical to the reference's, computed on the GPU).
The output is streamed tensor by tensor, so host memory stays bounded by one fused tensor.
"""
import argparse
import json
import os
import sys
from pathlib import Path

import numpy as np
import torch

from . import format as fmt

MAX_SEQ_LEN = 4096
INT4_GROUP = 128

# The checkpoint this engine's kernels are built for (reference export.py:22-44).
EXPECTED_CONFIG = {
    "hidden_size": 2048,
    "intermediate_size": 8192,
    "num_hidden_layers": 16,
    "num_attention_heads": 32,
    "num_key_value_heads": 8,
    "head_dim": 64,
    "vocab_size": 128256,
    "rms_norm_eps": 1e-5,
    "rope_theta": 500000.0,
    "tie_word_embeddings": True,
    "bos_token_id": 128000,
}
EXPECTED_ROPE_SCALING = {
    "rope_type": "llama3",
    "factor": 32.0,
    "low_freq_factor": 1.0,
    "high_freq_factor": 4.0,
    "original_max_position_embeddings": 8192,
}
EXPECTED_EOS = [128001, 128008, 128009]


def _rope_scaling(config) -> dict:
    rs = getattr(config, "rope_scaling", None) or getattr(config, "rope_parameters", None) or {}
    return dict(rs)


def check_config(config) -> None:
    """Raise ValueError unless `config` is the Llama-3.2-1B configuration (reference export.py:46-53)."""
    for key, want in EXPECTED_CONFIG.items():
        got = getattr(config, key, None)
        if key == "rope_theta" and got is None:
            got = _rope_scaling(config).get("rope_theta")
        if got != want:
            raise ValueError(f"config.{key} = {got!r}, expected {want!r}")
    rs = _rope_scaling(config)
    for key, want in EXPECTED_ROPE_SCALING.items():
        if rs.get(key) != want:
            raise ValueError(f"config.rope_scaling[{key!r}] = {rs.get(key)!r}, expected {want!r}")
    eos = config.eos_token_id
    if list(eos if isinstance(eos, (list, tuple)) else [eos]) != EXPECTED_EOS:
        raise ValueError(f"config.eos_token_id = {eos!r}")
    dt = getattr(config, "torch_dtype", None) or getattr(config, "dtype", None)
    if dt not in (torch.bfloat16, "bfloat16"):
        raise ValueError(f"config.torch_dtype = {dt!r}")


def compute_inv_freq(config) -> np.ndarray:
    """transformers' Llama-3 rope frequencies, fp32 (reference export.py:56-60)."""
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    inv_freq, attn_scaling = ROPE_INIT_FUNCTIONS["llama3"](config, "cpu")
    if attn_scaling != 1.0:
        raise ValueError(f"attention scaling {attn_scaling} != 1.0")
    return inv_freq.to(torch.float32).numpy()


def hf_layer_keys(i: int) -> dict:
    p = f"model.layers.{i}."
    return {"attn_norm": p + "input_layernorm.weight", "q": p + "self_attn.q_proj.weight",
            "k": p + "self_attn.k_proj.weight", "v": p + "self_attn.v_proj.weight",
            "o": p + "self_attn.o_proj.weight", "ffn_norm": p + "post_attention_layernorm.weight",
            "gate": p + "mlp.gate_proj.weight", "up": p + "mlp.up_proj.weight", "down": p + "mlp.down_proj.weight"}


def expected_hf_keys(n_layers: int) -> list:
    keys = ["model.embed_tokens.weight", "model.norm.weight"]
    for i in range(n_layers):
        keys.extend(hf_layer_keys(i).values())
    return keys


class _Checkpoint:
    """Lazy access to the tensors of every *.safetensors file of a directory."""

    def __init__(self, hf_dir: Path):
        from safetensors import safe_open
        files = sorted(Path(hf_dir).glob("*.safetensors"))
        if not files:
            raise FileNotFoundError(f"no *.safetensors in {hf_dir}")
        self._where = {}
        self._handles = [safe_open(str(f), framework="pt") for f in files]
        for h in self._handles:
            for k in h.keys():
                self._where[k] = h

    def keys(self):
        return self._where.keys()

    def get(self, key: str) -> torch.Tensor:
        return self._where[key].get_tensor(key)


def _linear_specs(name: str, rows: int, cols: int, dtype: str) -> list:
    if dtype == "bf16":
        return [(name + ".weight", fmt.BF16, rows, cols)]
    if dtype == "int8":
        return [(name + ".weight", fmt.I8, rows, cols), (name + ".scales", fmt.F32, rows, 1)]
    return [(name + ".weight", fmt.I4X2, rows, cols), (name + ".scales", fmt.F16, rows, cols // INT4_GROUP)]


def _linear_data(t: torch.Tensor, dtype: str) -> list:
    if t.dtype != torch.bfloat16:
        raise ValueError(f"linear weight dtype {t.dtype}, expected bfloat16")
    if dtype == "bf16":
        return [t.contiguous().view(torch.int16).numpy().tobytes()]
    from . import quantize as qz
    w = t.float().numpy()  # the bf16 weight upcast to fp32 (reference export.py:90)
    if dtype == "int8":
        q, s = qz.quantize_int8_rows(w)
        return [q.tobytes(), s.astype(np.float32).tobytes()]
    packed, s = qz.quantize_int4_groups(w, INT4_GROUP)
    return [packed.tobytes(), s.astype(np.float16).tobytes()]


def export(hf_dir, out, dtype: str, check: bool = True) -> int:
    """Write `out` from the checkpoint in `hf_dir`; returns the number of tensors.  `check=False` skips the
    Llama-3.2-1B configuration check (for small test checkpoints; the engine itself needs that shape)."""
    from transformers import AutoConfig
    if dtype not in ("bf16", "int8", "int4"):
        raise ValueError("dtype must be bf16, int8 or int4")
    hf_dir, out = Path(hf_dir), Path(out)
    config = AutoConfig.from_pretrained(hf_dir)
    if check:
        check_config(config)
    n_layers = config.num_hidden_layers
    H, I = config.hidden_size, config.intermediate_size
    nh, nkv = config.num_attention_heads, config.num_key_value_heads
    hd = getattr(config, "head_dim", None) or H // nh
    V = config.vocab_size
    inv_freq = compute_inv_freq(config)

    ck = _Checkpoint(hf_dir)
    if "lm_head.weight" in ck.keys():
        raise ValueError("the checkpoint has its own lm_head.weight; this format stores one embedding for both ends")
    missing = [k for k in expected_hf_keys(n_layers) if k not in ck.keys()]
    if missing:
        raise ValueError(f"{len(missing)} tensors the format needs are absent from the checkpoint, e.g. {missing[:5]}")

    qkv_rows = (nh + 2 * nkv) * hd
    specs = [("rope.inv_freq", fmt.F32, inv_freq.size, 1)]
    specs += _linear_specs("tok_embeddings", V, H, dtype)
    specs.append(("norm.weight", fmt.F32, H, 1))
    for i in range(n_layers):
        p = f"layers.{i}."
        specs.append((p + "attn_norm.weight", fmt.F32, H, 1))
        specs += _linear_specs(p + "wqkv", qkv_rows, H, dtype)
        specs += _linear_specs(p + "wo", H, nh * hd, dtype)
        specs.append((p + "ffn_norm.weight", fmt.F32, H, 1))
        specs += _linear_specs(p + "w_gate_up", 2 * I, H, dtype)
        specs += _linear_specs(p + "w_down", H, I, dtype)
    if [s[0] for s in specs] != fmt.expected_names(n_layers, dtype != "bf16"):
        raise AssertionError("internal: the tensors were produced in another order than the file's table")

    header = {"weight_dtype": {"bf16": fmt.WEIGHT_BF16, "int8": fmt.WEIGHT_INT8, "int4": fmt.WEIGHT_INT4}[dtype],
              "hidden_size": H, "intermediate_size": I, "n_layers": n_layers, "n_heads": nh, "n_kv_heads": nkv,
              "head_dim": hd, "vocab_size": V, "max_seq_len": MAX_SEQ_LEN, "rms_eps": config.rms_norm_eps,
              "rope_theta": float(getattr(config, "rope_theta", None) or _rope_scaling(config).get("rope_theta")),
              "group_size": INT4_GROUP if dtype == "int4" else 0}
    out.parent.mkdir(parents=True, exist_ok=True)
    w = fmt.Writer(out, header, specs)

    def norm(key):
        w.write(ck.get(key).float().numpy().astype(np.float32).tobytes())

    def linear(t):
        for b in _linear_data(t, dtype):
            w.write(b)

    w.write(inv_freq.astype(np.float32).tobytes())
    linear(ck.get("model.embed_tokens.weight"))
    norm("model.norm.weight")
    for i in range(n_layers):
        k = hf_layer_keys(i)
        norm(k["attn_norm"])
        linear(torch.cat([ck.get(k["q"]), ck.get(k["k"]), ck.get(k["v"])], dim=0))
        linear(ck.get(k["o"]))
        norm(k["ffn_norm"])
        linear(torch.cat([ck.get(k["gate"]), ck.get(k["up"])], dim=0))
        linear(ck.get(k["down"]))
    w.close()
    print(f"wrote {out}: {os.path.getsize(out)} bytes, {len(specs)} tensors", flush=True)
    return len(specs)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Export a HF Llama-3.2-1B checkpoint to .cudallm")
    ap.add_argument("--hf-dir", type=Path, required=True)
    ap.add_argument("--out", type=Path, required=True)
    ap.add_argument("--dtype", choices=("bf16", "int8", "int4"), required=True)
    args = ap.parse_args(argv)
    export(args.hf_dir, args.out, args.dtype)
    return 0


if __name__ == "__main__":
    sys.exit(main())
