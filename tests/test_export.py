"""The HF -> .cudallm exporter (reference python/cudallm/export.py, tests/test_export.py:12-100).

CPU: a small random checkpoint in Hugging Face's layout checks the file the exporter writes byte for byte
(fused q|k|v and gate|up rows, fp32 norms, transformers' own Llama-3 inv_freq bits, tensor order, header),
and the configuration check.  GPU: a full-size random Llama-3.2-1B checkpoint is exported and decoded by
the engine, and compared with transformers' LlamaForCausalLM (fp32, eager attention) on the same tokens,
at the engine-vs-reference tolerances of the reference's tests/test_engine_vs_reference.py:72-82
(the engine keeps an fp16 KV cache, so not the 1e-4 of its fp32-cache ReferenceModel).
"""
import json

import numpy as np
import pytest
import torch

from cudallm_amd import export as X
from cudallm_amd import format as fmt

ROPE = {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
        "original_max_position_embeddings": 8192}
LLAMA_1B = dict(hidden_size=2048, intermediate_size=8192, num_hidden_layers=16, num_attention_heads=32,
                num_key_value_heads=8, head_dim=64, vocab_size=128256)
SMALL = dict(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
             head_dim=64, vocab_size=1000)


def hf_config(shape: dict):
    from transformers import LlamaConfig
    return LlamaConfig(**shape, rms_norm_eps=1e-5, rope_theta=500000.0, rope_scaling=dict(ROPE), tie_word_embeddings=True,
                       bos_token_id=128000, eos_token_id=[128001, 128008, 128009], torch_dtype="bfloat16",
                       max_position_embeddings=131072)


def write_hf_checkpoint(d, shape: dict, seed: int, device: str = "cpu") -> dict:
    """A random bf16 checkpoint in the HF layout (two safetensors files, tied embeddings); returns the tensors."""
    from safetensors.torch import save_file
    cfg = hf_config(shape)
    cfg.save_pretrained(d)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    H, I, hd = shape["hidden_size"], shape["intermediate_size"], shape["head_dim"]
    nh, nkv = shape["num_attention_heads"], shape["num_key_value_heads"]

    def lin(r, c):
        return (torch.randn(r, c, generator=g, device=device) * 0.02).to(torch.bfloat16).cpu()

    def norm(n):
        return (1.0 + 0.1 * torch.randn(n, generator=g, device=device)).to(torch.bfloat16).cpu()

    t = {"model.embed_tokens.weight": lin(shape["vocab_size"], H), "model.norm.weight": norm(H)}
    for i in range(shape["num_hidden_layers"]):
        k = X.hf_layer_keys(i)
        t[k["attn_norm"]] = norm(H)
        t[k["q"]], t[k["k"]], t[k["v"]] = lin(nh * hd, H), lin(nkv * hd, H), lin(nkv * hd, H)
        t[k["o"]] = lin(H, nh * hd)
        t[k["ffn_norm"]] = norm(H)
        t[k["gate"]], t[k["up"]], t[k["down"]] = lin(I, H), lin(I, H), lin(H, I)
    keys = list(t)
    half = len(keys) // 2
    files = {"model-00001-of-00002.safetensors": keys[:half], "model-00002-of-00002.safetensors": keys[half:]}
    for f, ks in files.items():
        save_file({k: t[k] for k in ks}, str(d / f))
    index = {"metadata": {"total_size": sum(v.numel() * 2 for v in t.values())},
             "weight_map": {k: f for f, ks in files.items() for k in ks}}
    (d / "model.safetensors.index.json").write_text(json.dumps(index))
    return t


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.fixture(scope="module")
def small(tmp_path_factory):
    d = tmp_path_factory.mktemp("hf_small")
    t = write_hf_checkpoint(d, SMALL, seed=3)
    out = d / "small_bf16.cudallm"
    X.export(d, out, "bf16", check=False)
    return d, t, out


def test_bf16_file_matches_the_checkpoint(small):
    d, t, out = small
    hdr = fmt.read_header(out)
    assert (hdr["magic"], hdr["version"], hdr["weight_dtype"]) == (b"CLLM", 1, fmt.WEIGHT_BF16)
    assert (hdr["hidden_size"], hdr["intermediate_size"], hdr["n_layers"], hdr["n_heads"], hdr["n_kv_heads"],
            hdr["head_dim"], hdr["vocab_size"], hdr["max_seq_len"]) == (256, 512, 2, 4, 2, 64, 1000, 4096)
    assert hdr["rms_eps"] == np.float32(1e-5) and hdr["rope_theta"] == np.float32(500000.0)
    assert hdr["group_size"] == 0 and hdr["table_offset"] == 256
    table = fmt.read_table(out)
    assert [e["name"] for e in table] == fmt.expected_names(2, False)
    assert out.stat().st_size == table[-1]["offset"] + table[-1]["nbytes"]
    e = {x["name"]: x for x in table}
    for i in range(2):
        k = X.hf_layer_keys(i)
        np.testing.assert_array_equal(fmt.load_tensor(out, e[f"layers.{i}.wqkv.weight"]),
                                      np.concatenate([_bits(t[k[n]]) for n in ("q", "k", "v")]))
        np.testing.assert_array_equal(fmt.load_tensor(out, e[f"layers.{i}.w_gate_up.weight"]),
                                      np.concatenate([_bits(t[k[n]]) for n in ("gate", "up")]))
        np.testing.assert_array_equal(fmt.load_tensor(out, e[f"layers.{i}.wo.weight"]), _bits(t[k["o"]]))
        np.testing.assert_array_equal(fmt.load_tensor(out, e[f"layers.{i}.w_down.weight"]), _bits(t[k["down"]]))
        assert np.array_equal(fmt.load_tensor(out, e[f"layers.{i}.attn_norm.weight"]).ravel(),
                              t[k["attn_norm"]].float().numpy())
    np.testing.assert_array_equal(fmt.load_tensor(out, e["tok_embeddings.weight"]), _bits(t["model.embed_tokens.weight"]))
    assert np.array_equal(fmt.load_tensor(out, e["norm.weight"]).ravel(), t["model.norm.weight"].float().numpy())


def test_inv_freq_is_transformers_llama3(small):
    """reference tests/test_export.py:83-88: the stored frequencies are transformers' own fp32 bits."""
    from transformers import AutoConfig
    from transformers.modeling_rope_utils import ROPE_INIT_FUNCTIONS
    d, _, out = small
    want, _ = ROPE_INIT_FUNCTIONS["llama3"](AutoConfig.from_pretrained(d), "cpu")
    got = fmt.load_tensor(out, {x["name"]: x for x in fmt.read_table(out)}["rope.inv_freq"]).ravel()
    assert got.dtype == np.float32 and np.array_equal(got, want.float().numpy())


def test_config_check():
    X.check_config(hf_config(LLAMA_1B))
    with pytest.raises(ValueError, match="hidden_size"):
        X.check_config(hf_config(SMALL))
    c = hf_config(LLAMA_1B)
    c.tie_word_embeddings = False
    with pytest.raises(ValueError, match="tie_word_embeddings"):
        X.check_config(c)


def test_rejects_untied_and_missing(tmp_path):
    from safetensors.torch import save_file
    write_hf_checkpoint(tmp_path, SMALL, seed=4)
    save_file({"lm_head.weight": torch.zeros(4, 4, dtype=torch.bfloat16)}, str(tmp_path / "z.safetensors"))
    with pytest.raises(ValueError, match="lm_head"):
        X.export(tmp_path, tmp_path / "x.cudallm", "bf16", check=False)


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_exported_checkpoint_matches_transformers(gpu, tmp_path):
    """Engine (bf16, persistent kernel, step_debug) on the exported file vs LlamaForCausalLM on the checkpoint."""
    from transformers import LlamaForCausalLM
    from cudallm_amd import engine as E
    print("[export] writing a random Llama-3.2-1B checkpoint", flush=True)
    t = write_hf_checkpoint(tmp_path, LLAMA_1B, seed=11, device="cuda")
    del t
    out = tmp_path / "hf_bf16.cudallm"
    X.export(tmp_path, out, "bf16")
    ids = [128000] + [int(v) for v in np.random.default_rng(5).integers(0, 128256, 15)]
    logits, res = [], []
    with E.Engine(out) as eng:
        for tok in ids:
            _, lg, r = eng.step_debug(tok)
            logits.append(lg)
            res.append(r)
    logits, res = np.stack(logits), np.stack(res)
    print("[export] transformers forward", flush=True)
    model = LlamaForCausalLM.from_pretrained(tmp_path, dtype=torch.float32, attn_implementation="eager").cuda().eval()
    with torch.no_grad():
        o = model(torch.tensor([ids], device="cuda"), output_hidden_states=True)
    hf_logits = o.logits[0].float().cpu().numpy()
    hidden = torch.stack([o.hidden_states[k][0] for k in range(16)]).float().cpu().numpy()  # [16, T, H]
    del model, o
    torch.cuda.empty_cache()
    worst = 0.0
    for p in range(len(ids)):
        for k in range(16):  # hidden_states[16] is after the final norm
            a, b = res[p, k].astype(np.float64), hidden[k, p].astype(np.float64)
            worst = max(worst, float(np.linalg.norm(a - b) / np.linalg.norm(b)))
    diff = float(np.max(np.abs(logits - hf_logits)))
    agree = int(np.sum(np.argmax(logits, 1) == np.argmax(hf_logits, 1)))
    print(f"[export] engine vs transformers: residual rel {worst:.2e}, max |dlogit| {diff:.2e}, argmax {agree}/16",
          flush=True)
    assert worst < 1e-3
    assert diff < 2e-2
    assert agree >= len(ids) - 1


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_exported_int8_int4_equal_quantised_bf16(gpu, small):
    """The quantised exports hold exactly the reference quantisers' output on the bf16 weights (checked with the
    CPU oracle's restatement of python/cudallm/quantize.py)."""
    from oracle import quantize as Q
    d, t, _ = small
    for dt in ("int8", "int4"):
        out = d / f"small_{dt}.cudallm"
        X.export(d, out, dt, check=False)
        e = {x["name"]: x for x in fmt.read_table(out)}
        assert list(e) == fmt.expected_names(2, True)
        w = torch.cat([t[X.hf_layer_keys(1)[n]] for n in ("gate", "up")]).float().numpy()
        if dt == "int8":
            q, s = Q.quantize_int8_rows(w)
            np.testing.assert_array_equal(fmt.load_tensor(out, e["layers.1.w_gate_up.weight"]), q)
            np.testing.assert_array_equal(fmt.load_tensor(out, e["layers.1.w_gate_up.scales"]).ravel(), s)
        else:
            p, s = Q.quantize_int4_groups(w)
            np.testing.assert_array_equal(fmt.load_tensor(out, e["layers.1.w_gate_up.weight"]), p)
            np.testing.assert_array_equal(fmt.load_tensor(out, e["layers.1.w_gate_up.scales"]), s)
