"""CPU lane: pins the oracle against the reference's known answers, golden vectors and the
mathematics, and checks the pure-Python format module of the product against it."""
import struct
import tempfile
from pathlib import Path

import numpy as np
import pytest

from oracle import fileformat as off
from oracle import kernels as K
from oracle import model as M
from oracle import quantize as Q
from oracle import synth

GOLDEN = Path(__file__).resolve().parent / "golden" / "decode_tiny.npz"


# ---- quantisers: the reference's known-answer tests (tests/test_quantize.py:10-63) ----------

def test_int8_error_bound():
    w = np.random.default_rng(1).normal(0, 0.02, size=(64, 256)).astype(np.float32)
    q, s = Q.quantize_int8_rows(w)
    assert q.dtype == np.int8 and s.dtype == np.float32 and s.shape == (64,)
    assert q.min() >= -127 and q.max() <= 127
    assert np.all(np.abs(Q.dequantize_int8_rows(q, s) - w) <= s[:, None] / 2 + 1e-7)


def test_int8_zero_rows():
    w = np.random.default_rng(2).normal(0, 0.02, size=(4, 128)).astype(np.float32)
    w[1] = 0.0
    q, s = Q.quantize_int8_rows(w)
    assert s[1] == 1.0 and np.all(q[1] == 0) and np.all(np.isfinite(s))


def test_int4_pack_unpack_roundtrip():
    q = np.random.default_rng(3).integers(-8, 8, size=(16, 256), dtype=np.int8)
    u = (q + 8).astype(np.uint8)
    np.testing.assert_array_equal(Q.unpack_int4((u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)), q)


def test_int4_nibble_order():
    packed = np.array([[0x0F, 0x08 | (0x09 << 4)]], dtype=np.uint8)
    np.testing.assert_array_equal(Q.unpack_int4(packed), [[7, -8, 0, 1]])
    w = np.zeros((1, 128), dtype=np.float32)
    w[0, :4] = [7.0, -7.0, 0.0, 1.0]
    p, s = Q.quantize_int4_groups(w)
    assert s[0, 0] == np.float16(1.0)
    assert p[0, 0] == (7 + 8) | ((-7 + 8) << 4) and p[0, 1] == (0 + 8) | ((1 + 8) << 4)


def test_int4_dequant_error_bound():
    w = np.random.default_rng(4).normal(0, 0.02, size=(32, 512)).astype(np.float32)
    p, s = Q.quantize_int4_groups(w, 128)
    assert p.dtype == np.uint8 and p.shape == (32, 256) and s.dtype == np.float16 and s.shape == (32, 4)
    bound = np.repeat(s.astype(np.float32), 128, axis=1) / 2 + 1e-6
    assert np.all(np.abs(Q.dequantize_int4_groups(p, s) - w) <= bound)


# ---- quantisers: brute force on small inputs ---------------------------------------------

def _nearest_even(v: np.ndarray, lo: int, hi: int) -> np.ndarray:
    """Brute force: the integer in [lo, hi] nearest to v, ties to the even one."""
    cand = np.arange(lo, hi + 1, dtype=np.float64)
    d = np.abs(v[..., None].astype(np.float64) - cand)
    best = d.min(axis=-1, keepdims=True)
    tie = np.isclose(d, best, rtol=0, atol=0)
    pick = np.where(tie & (cand % 2 == 0), cand, np.where(tie, cand, np.inf))
    even_first = np.where((tie & (cand % 2 == 0)).any(axis=-1), np.min(np.where(tie & (cand % 2 == 0), cand, np.inf), axis=-1),
                          np.min(pick, axis=-1))
    return even_first.astype(np.int64)


def test_int8_brute_force_with_ties():
    rng = np.random.default_rng(5)
    w = rng.normal(0, 0.02, size=(8, 64)).astype(np.float32)
    w[0, :4] = [1.27, -1.27, 0.005, 0.015]  # s = 0.01 -> exact half-way points 0.5 and 1.5
    q, s = Q.quantize_int8_rows(w)
    np.testing.assert_array_equal(s, (np.abs(w).max(axis=1) / np.float32(127)).astype(np.float32))
    ratio = (w / s[:, None]).astype(np.float32)
    np.testing.assert_array_equal(q, _nearest_even(ratio, -127, 127))


def test_int4_brute_force_scales_are_fp16_rounded():
    rng = np.random.default_rng(6)
    w = rng.normal(0, 0.02, size=(4, 256)).astype(np.float32)
    p, s16 = Q.quantize_int4_groups(w)
    raw = (np.abs(w.reshape(4, 2, 128)).max(axis=2) / np.float32(7)).astype(np.float32)
    np.testing.assert_array_equal(s16, raw.astype(np.float16))
    ratio = (w.reshape(4, 2, 128) / s16.astype(np.float32)[:, :, None]).astype(np.float32).reshape(4, 256)
    np.testing.assert_array_equal(Q.unpack_int4(p), _nearest_even(ratio, -8, 7))


def test_bf16_rounding_known_answers():
    vals = np.array([1.0, -2.5, 0.0, 3.140625], dtype=np.float32)
    bits = Q.bf16_round_bits(vals)
    np.testing.assert_array_equal(Q.bf16_bits_to_f32(bits), vals)
    # Half-way cases round to even: 1 + 2^-8 -> 1.0 ; 1 + 3*2^-8 -> 1 + 2^-6
    np.testing.assert_array_equal(Q.bf16_bits_to_f32(Q.bf16_round_bits(np.float32([1 + 2**-8, 1 + 3 * 2**-8]))),
                                  np.float32([1.0, 1 + 2**-6]))


# ---- file format (tests/test_format.py:31-106) -------------------------------------------

HEADER = {"weight_dtype": 1, "hidden_size": 2048, "intermediate_size": 8192, "n_layers": 16, "n_heads": 32,
          "n_kv_heads": 8, "head_dim": 64, "vocab_size": 128256, "max_seq_len": 4096, "rms_eps": 1e-5,
          "rope_theta": 500000.0, "group_size": 0}


def _tiny_tensors():
    rng = np.random.default_rng(0)
    return [("a.f32", off.F32, 5, 1, rng.standard_normal((5, 1)).astype(np.float32).tobytes()),
            ("b.bf16", off.BF16, 3, 7, rng.integers(0, 2**16, size=(3, 7), dtype=np.uint16).tobytes()),
            ("c.f16", off.F16, 2, 3, rng.standard_normal((2, 3)).astype(np.float16).tobytes()),
            ("d.i8", off.I8, 4, 9, rng.integers(-127, 128, size=(4, 9), dtype=np.int8).tobytes()),
            ("e.i4", off.I4X2, 3, 8, rng.integers(0, 256, size=(3, 4), dtype=np.uint8).tobytes())]


def test_struct_sizes():
    assert struct.calcsize(off.HEADER_FMT) == 72 and struct.calcsize(off.ENTRY_FMT) == 80


@pytest.mark.parametrize("writer", ["oracle", "product"])
def test_format_roundtrip_byte_layout(tmp_path, writer):
    from cudallm_amd import format as pf
    tensors = _tiny_tensors()
    path = tmp_path / "tiny.cudallm"
    (off.write if writer == "oracle" else pf.write_cudallm)(path, HEADER, tensors)
    hdr = off.read_header(path)
    assert (hdr["magic"], hdr["version"], hdr["n_tensors"], hdr["table_offset"], hdr["reserved0"]) == \
        (b"CLLM", 1, 5, 256, 0)
    raw = path.read_bytes()
    assert raw[72:256] == b"\0" * 184
    table = off.read_table(path)
    prev = 256 + 80 * len(tensors)
    for e, (name, dt, rows, cols, data) in zip(table, tensors):
        assert e["name"] == name and e["offset"] % 256 == 0 and e["offset"] >= prev
        assert raw[prev:e["offset"]] == b"\0" * (e["offset"] - prev)
        assert (e["dtype"], e["rows"], e["cols"], e["reserved"]) == (dt, rows, cols, 0)
        assert e["nbytes"] == off.nbytes_of(dt, rows, cols) == len(data)
        assert raw[e["offset"]:e["offset"] + e["nbytes"]] == data
        prev = e["offset"] + e["nbytes"]
    assert len(raw) == prev
    assert pf.read_header(path) == hdr and pf.read_table(path) == table


def test_product_and_oracle_writers_agree_bytewise(tmp_path):
    from cudallm_amd import format as pf
    off.write(tmp_path / "a", HEADER, _tiny_tensors())
    pf.write_cudallm(tmp_path / "b", HEADER, _tiny_tensors())
    assert (tmp_path / "a").read_bytes() == (tmp_path / "b").read_bytes()


def test_writer_rejects_wrong_nbytes(tmp_path):
    from cudallm_amd import format as pf
    with pytest.raises(ValueError):
        pf.write_cudallm(tmp_path / "bad", HEADER, [("x", pf.F32, 4, 1, b"\0" * 12)])
    with pytest.raises(ValueError):
        off.write(tmp_path / "bad2", HEADER, [("x", off.F32, 4, 1, b"\0" * 12)])


def test_expected_names():
    from cudallm_amd import format as pf
    bf16, quant = off.tensor_names(16, False), off.tensor_names(16, True)
    assert len(bf16) == 99 and len(quant) == 164
    assert bf16[:4] == ["rope.inv_freq", "tok_embeddings.weight", "norm.weight", "layers.0.attn_norm.weight"]
    assert quant[:5] == ["rope.inv_freq", "tok_embeddings.weight", "tok_embeddings.scales", "norm.weight",
                         "layers.0.attn_norm.weight"]
    assert bf16[-1] == "layers.15.w_down.weight" and quant[-1] == "layers.15.w_down.scales"
    assert pf.expected_names(16, False) == bf16 and pf.expected_names(16, True) == quant


@pytest.mark.parametrize("wd,known", [("bf16", 2471764096), ("int8", 1238037632), ("int4", 637452416)])
def test_weight_bytes_known_answers(wd, known):
    """results/decode/quant/Q_*.json: weight_bytes of the Llama-3.2-1B files, per weight type."""
    from cudallm_amd import synth as ps
    specs = ps._specs(wd, ps.LLAMA_1B)
    assert [s[0] for s in specs] == off.tensor_names(16, wd != "bf16")
    assert sum(off.nbytes_of(dt, r, c) for _, dt, r, c in specs) == known


# ---- kernel closed forms: identities that a wrong term, sign or index would break ---------

def test_llama3_inv_freq_properties():
    from cudallm_amd import synth as ps
    f = K.llama3_inv_freq()
    base = (1.0 / 500000.0 ** (np.arange(32) * 2 / 64))
    wl = 2 * np.pi / base
    assert f[0] == np.float32(1.0)
    np.testing.assert_array_equal(f[wl < 2048], base[wl < 2048].astype(np.float32))
    np.testing.assert_array_equal(f[wl > 8192], (base[wl > 8192] / 32).astype(np.float32))
    assert np.all(np.diff(f.astype(np.float64)) < 0)
    np.testing.assert_array_equal(f, ps.llama3_inv_freq())  # independent second implementation


def test_rope_known_answer_and_norm():
    inv = K.llama3_inv_freq()
    v = np.random.default_rng(8).standard_normal((3, 64))
    np.testing.assert_allclose(K.rope(v, inv, 0), v)
    r = K.rope(v, inv, 1)
    # pair 0 has inv_freq 1 -> rotation by exactly 1 radian
    np.testing.assert_allclose(r[:, 0], v[:, 0] * np.cos(1) - v[:, 32] * np.sin(1))
    np.testing.assert_allclose(r[:, 32], v[:, 32] * np.cos(1) + v[:, 0] * np.sin(1))
    pair = lambda a: a[:, :32] ** 2 + a[:, 32:] ** 2  # noqa: E731
    np.testing.assert_allclose(pair(K.rope(v, inv, 777)), pair(v))


def test_attention_single_token_is_v_and_gqa_mapping():
    nh, nkv, hd = 8, 2, 64
    rng = np.random.default_rng(9)
    q = rng.standard_normal(nh * hd)
    k = rng.standard_normal((nkv, 4, hd)).astype(np.float16)
    v = rng.standard_normal((nkv, 4, hd)).astype(np.float16)
    out = K.attention(q, k, v, 1, nh, nkv, hd).reshape(nh, hd)
    for h in range(nh):
        np.testing.assert_array_equal(out[h], v[h // 4, 0].astype(np.float64))


def test_attention_two_token_closed_form_scale():
    hd = 64
    k = np.zeros((1, 2, hd), dtype=np.float16)
    k[0, 1, 0] = 2.0
    v = np.zeros((1, 2, hd), dtype=np.float16)
    v[0, 1, :] = 1.0
    q = np.zeros(4 * hd)
    q[0::hd] = 3.0  # every head: q . k1 = 6 -> score 0.75 with scale 1/8
    out = K.attention(q, k, v, 2, 4, 1, hd).reshape(4, hd)
    np.testing.assert_allclose(out, 1.0 / (1.0 + np.exp(-0.75)))


def test_rmsnorm_unit_rms_and_silu():
    x = np.random.default_rng(10).standard_normal(2048) * 7
    y = K.rms_normalize(x, np.ones(2048), 0.0)
    np.testing.assert_allclose(np.sqrt(np.mean(y * y)), 1.0)
    assert K.silu(0.0) == 0.0
    np.testing.assert_allclose(K.silu(np.array([40.0, -40.0])), [40.0, 0.0], atol=1e-15)


def test_matvec_epilogues():
    rng = np.random.default_rng(11)
    w = rng.standard_normal((6, 4))
    x = rng.standard_normal(4)
    d = w @ x
    np.testing.assert_allclose(K.matvec(w, x, "add", y_init=np.ones(6)), d + 1)
    np.testing.assert_allclose(K.matvec(w, x, "swiglu"), d[:3] / (1 + np.exp(-d[:3])) * d[3:])


def test_argmax_known_answers():
    lg = np.random.default_rng(16).standard_normal(128256).astype(np.float32)
    lg[5] = lg[100000] = 50.0
    assert K.argmax_lowest(lg) == 5
    lg = np.random.default_rng(17).standard_normal(128256).astype(np.float32)
    lg[-1] = 50.0
    assert K.argmax_lowest(lg) == 128255


# ---- decode step: golden vectors written by the reference's own ReferenceModel ------------

@pytest.mark.parametrize("wd", ["bf16", "int8", "int4"])
def test_oracle_decode_matches_reference_golden(wd):
    g = np.load(GOLDEN)
    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "tiny.cudallm"
        synth.write_model(path, wd, seed=int(g["seed"]), dims=synth.TINY, norm="random")
        m = M.OracleModel(path, threads=4)
        logits, res = [], []
        for t in g["tokens"]:
            lg, r = m.step(int(t))
            logits.append(lg.numpy())
            res.append(np.stack([v.numpy() for v in r]))
        np.testing.assert_allclose(np.stack(logits), g[f"{wd}_logits"], rtol=0, atol=1e-6)
        np.testing.assert_allclose(np.stack(res), g[f"{wd}_residuals"], rtol=0, atol=1e-6)
        assert m.greedy([int(t) for t in g["tokens"][:3]], 6) == [int(t) for t in g[f"{wd}_greedy"]]


def test_oracle_decode_invariants():
    """Zero wo and w_down: every residual equals the embedding; logits = E . rmsnorm(emb) * norm."""
    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "tiny.cudallm"
        synth.write_model(path, "bf16", seed=3, dims=synth.TINY, norm="random")
        m = M.OracleModel(path, threads=4)
        for L in m.layers:
            for key in ("wo", "w_down"):
                L[key].w.zero_()
        lg, res = m.step(42)
        emb = res[0].numpy().astype(np.float64)
        for r in res[1:]:
            np.testing.assert_array_equal(r.numpy(), res[0].numpy())
        e64 = m.emb.dense().numpy().astype(np.float64)
        ref = e64 @ K.rms_normalize(emb, m.final_norm.numpy(), m.eps)
        np.testing.assert_allclose(lg.numpy(), ref, rtol=1e-4, atol=1e-5)
