"""GPU parity of every single-kernel hook against the oracle's float64 closed forms.

Mirrors the reference's tests/test_kernels.py:43-229 (same seeds, shapes, grids and tolerances),
then widens it: every Llama-3.2-1B projection shape the reference benchmarks, the generic-width
matvec path, context lengths up to 8192 (its long-context attention case), and the GPU quantisers bit-exact.
"""
import numpy as np
import pytest

from cudallm_amd import engine as E
from cudallm_amd import quantize as GQ
from oracle import kernels as K
from oracle import quantize as Q

pytestmark = pytest.mark.gpu

NH, NKV, HD, MAX_SEQ = 32, 8, 64, 4096


@pytest.fixture(autouse=True)
def _gpu(gpu):
    return gpu


def _operands(wtype: str, rows: int, cols: int, seed: int, bf16_master: bool = False):
    """(stored weight, scales or None, exact dequantised weight in float64)."""
    w = np.random.default_rng(seed).normal(0, 0.02, size=(rows, cols)).astype(np.float32)
    if bf16_master:
        w = Q.bf16_bits_to_f32(Q.bf16_round_bits(w))
    if wtype == "bf16":
        bits = Q.bf16_round_bits(w)
        return bits, None, Q.bf16_bits_to_f32(bits).astype(np.float64)
    if wtype == "int8":
        q, s = Q.quantize_int8_rows(w)
        return q, s, Q.dequantize_int8_rows(q, s).astype(np.float64)
    p, s = Q.quantize_int4_groups(w, 128)
    return p, s, Q.dequantize_int4_groups(p, s).astype(np.float64)


# ---- matvec (reference tests/test_kernels.py:43-96) ----------------------------------------

def test_matvec_naive_bf16_store():
    rows, cols = 1024, 2048
    rng = np.random.default_rng(10)
    bits = Q.bf16_round_bits(rng.normal(0, 0.02, size=(rows, cols)))
    x = rng.standard_normal(cols).astype(np.float32)
    y = E.kernel_matvec("naive", "bf16", "store", 0, 0, bits, None, x, None, 1e-5, None, rows, cols)
    ref = Q.bf16_bits_to_f32(bits).astype(np.float64) @ x.astype(np.float64)
    assert np.allclose(y, ref, rtol=1e-4, atol=1e-4)


def _check_matvec(wtype, epilogue, fuse_norm, rpb, rows, cols, seed, bf16_master=False):
    eps = 1e-5
    w, s, w64 = _operands(wtype, rows, cols, seed, bf16_master)
    rng = np.random.default_rng(seed + 1)
    x = rng.standard_normal(cols).astype(np.float32)
    norm_w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    out_rows = rows // 2 if epilogue == "swiglu" else rows
    y_init = rng.standard_normal(out_rows).astype(np.float32) if epilogue == "add" else None
    print(f"[matvec] {wtype} {epilogue} norm={fuse_norm} rpb={rpb} {rows}x{cols}", flush=True)
    y = E.kernel_matvec("opt", wtype, epilogue, fuse_norm, rpb, w, s, x, norm_w if fuse_norm else None, eps, y_init,
                        rows, cols)
    ref = K.matvec(w64, x, epilogue, norm_w if fuse_norm else None, eps, y_init)
    err = np.abs(y - ref) - (1e-4 + 1e-4 * np.abs(ref))
    assert np.all(err <= 0), f"max excess {err.max():.3e} at row {int(np.argmax(err))}"


@pytest.mark.parametrize("shape", [(1024, 2048), (2048, 8192)], ids=lambda s: f"{s[0]}x{s[1]}")
@pytest.mark.parametrize("rpb", [1, 2, 4, 8])
@pytest.mark.parametrize("fuse_norm", [0, 1])
@pytest.mark.parametrize("epilogue", ["store", "add", "swiglu"])
@pytest.mark.parametrize("wtype", ["bf16", "int8", "int4"])
def test_matvec_opt(wtype, epilogue, fuse_norm, rpb, shape):
    rows, cols = shape
    _check_matvec(wtype, epilogue, fuse_norm, rpb, rows, cols, seed=20 + rows + cols)


# Every projection shape the reference benchmarks, with the engine epilogues (norm fused on the input side
# of q/k/v/gate/up/lm_head, residual add on o/down), bf16-rounded N(0, 0.02) master weights.
MODEL_SHAPES = [("q", 2048, 2048, "store", 1), ("k", 512, 2048, "store", 1), ("v", 512, 2048, "store", 1),
                ("o", 2048, 2048, "add", 0), ("gate", 8192, 2048, "store", 1), ("up", 8192, 2048, "store", 1),
                ("down", 2048, 8192, "add", 0), ("wqkv", 3072, 2048, "store", 1),
                ("gate_up", 16384, 2048, "swiglu", 1), ("lm_head", 128256, 2048, "store", 1)]


@pytest.mark.parametrize("wtype", ["bf16", "int8", "int4"])
@pytest.mark.parametrize("name,rows,cols,epilogue,norm", MODEL_SHAPES, ids=[s[0] for s in MODEL_SHAPES])
def test_matvec_model_shapes(wtype, name, rows, cols, epilogue, norm):
    _check_matvec(wtype, epilogue, norm, 0, rows, cols, seed=rows * 7 + cols, bf16_master=True)


@pytest.mark.parametrize("wtype", ["bf16", "int8", "int4"])
@pytest.mark.parametrize("rows,cols", [(1000, 1024), (37, 3072), (130, 12288), (6, 2048), (10, 8192), (20483, 2048)])
@pytest.mark.parametrize("epilogue", ["store", "add", "swiglu"])
def test_matvec_generic_and_ragged(wtype, rows, cols, epilogue):
    """Widths other than 2048/8192 (LDS-staged path) and row counts that leave partial blocks; 20483 rows of 2048
    give the waves uneven row ranges of several passes each."""
    if epilogue == "swiglu" and rows % 2:
        rows += 1
    _check_matvec(wtype, epilogue, 1, 4, rows, cols, seed=rows + 3 * cols)


def test_stream_read_timed_hook():
    """The bandwidth kernel on a device buffer through its timed hook: every launch shape records both events, and the
    sink (written only for one XOR-folded word that a zero buffer never gives) stays untouched."""
    import torch
    buf = torch.zeros(8 << 20, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(16 * 1024, dtype=torch.int32, device="cuda")
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    stream = torch.cuda.current_stream()
    a.record(stream)
    b.record(stream)
    for bpc in (4, 8, 16):
        E.launch_stream_read_timed(buf.data_ptr(), buf.numel(), bpc, sink.data_ptr(), sink.numel(), stream.cuda_stream,
                                   a.cuda_event, b.cuda_event)
        b.synchronize()
        assert 0 < a.elapsed_time(b) < 100
    assert int(sink.abs().sum()) == 0


def test_matvec_config1_int8_known_case():
    """The reference's int8 8192x2048 matvec case: bf16 master N(0, 0.02), x bf16 N(0, 1), checked in float64."""
    rng = np.random.default_rng(1)
    w = Q.bf16_bits_to_f32(Q.bf16_round_bits(rng.normal(0, 0.02, size=(8192, 2048)).astype(np.float32)))
    x = Q.bf16_bits_to_f32(Q.bf16_round_bits(rng.standard_normal(2048).astype(np.float32)))
    q, s = Q.quantize_int8_rows(w)
    y = E.kernel_matvec("opt", "int8", "store", 0, 0, q, s, x, None, 1e-5, None, 8192, 2048)
    ref = (q.astype(np.float64) * s.astype(np.float64)[:, None]) @ x.astype(np.float64)
    assert np.allclose(y, ref, rtol=1e-4, atol=1e-4)
    assert np.max(np.abs(y - ref) / np.maximum(np.abs(ref), 1e-3)) < 1e-2


# ---- rmsnorm, rope, attention, silu, argmax (reference tests/test_kernels.py:101-229) -------

def test_rmsnorm():
    n, eps = 2048, 1e-5
    rng = np.random.default_rng(11)
    x = rng.standard_normal(n).astype(np.float32)
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    assert np.allclose(E.kernel_rmsnorm(x, w, eps), K.rms_normalize(x, w, eps), rtol=1e-5, atol=1e-5)


SENTINEL = np.float16(-7.25)


def _ulp_diff(a, b):
    def ordered(v):
        u = v.astype(np.float16).view(np.uint16).astype(np.int32)
        return np.where(u & 0x8000, 0x8000 - u, u)
    return np.abs(ordered(a) - ordered(b))


@pytest.mark.parametrize("pos", [0, 1, 777, 4095])
@pytest.mark.parametrize("fused", [0, 1])
def test_rope_kv(fused, pos):
    rng = np.random.default_rng(12 + pos)
    inv = K.llama3_inv_freq()
    qkv = rng.standard_normal((NH + 2 * NKV) * HD).astype(np.float32)
    kc = np.full((NKV, MAX_SEQ, HD), SENTINEL, dtype=np.float16)
    vc = np.full((NKV, MAX_SEQ, HD), SENTINEL, dtype=np.float16)
    out, k_out, v_out = E.kernel_rope_kv(fused, qkv, inv, pos, kc, vc, NH, NKV, HD, MAX_SEQ)
    k_out, v_out = k_out.reshape(NKV, MAX_SEQ, HD), v_out.reshape(NKV, MAX_SEQ, HD)
    q_ref, k_ref, _, vc_ref = K.rope_kv(qkv, inv, pos, kc, vc, NH, NKV, HD)
    assert np.allclose(out[:NH * HD].reshape(NH, HD), q_ref, rtol=0, atol=1e-5)
    if not fused:
        assert np.allclose(out[NH * HD:(NH + NKV) * HD].reshape(NKV, HD), k_ref, rtol=0, atol=1e-5)
        np.testing.assert_array_equal(out[(NH + NKV) * HD:], qkv[(NH + NKV) * HD:])
    else:
        np.testing.assert_array_equal(out[NH * HD:], qkv[NH * HD:])  # k and v slices untouched
    assert np.all(_ulp_diff(k_out[:, pos, :], k_ref.astype(np.float16)) <= 1)
    np.testing.assert_array_equal(v_out, vc_ref)  # v row bit-exact, every other slot untouched
    others = np.ones(MAX_SEQ, dtype=bool)
    others[pos] = False
    assert np.all(k_out[:, others, :] == SENTINEL)


@pytest.fixture(scope="module")
def attn_data():
    rng = np.random.default_rng(13)
    return (rng.standard_normal(NH * HD).astype(np.float32),
            rng.standard_normal((NKV, MAX_SEQ, HD)).astype(np.float16),
            rng.standard_normal((NKV, MAX_SEQ, HD)).astype(np.float16))


@pytest.mark.parametrize("ctx", [1, 7, 128, 129, 1000, 4096])
@pytest.mark.parametrize("impl", ["naive", "opt"])
def test_attention(impl, ctx, attn_data):
    q, k, v = attn_data
    out = E.kernel_attention(impl, q, k, v, ctx, NH, NKV, HD, MAX_SEQ)
    assert np.allclose(out, K.attention(q, k, v, ctx, NH, NKV, HD), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("ctx", [128, 512, 2048, 4096, 8192, 8191])
def test_attention_config4_long_context(ctx):
    """The reference's long-context attention case: max_seq 8192 (grid 8 x 64 splits), chunk 128, LSE merge."""
    rng = np.random.default_rng(40 + ctx)
    q = rng.standard_normal(NH * HD).astype(np.float32)
    k = rng.standard_normal((NKV, 8192, HD)).astype(np.float16)
    v = rng.standard_normal((NKV, 8192, HD)).astype(np.float16)
    out = E.kernel_attention("opt", q, k, v, ctx, NH, NKV, HD, 8192)
    assert np.allclose(out, K.attention(q, k, v, ctx, NH, NKV, HD), rtol=1e-4, atol=1e-4)


def test_attention_large_scores_are_stable():
    """Scores up to ~+-200: the split-local max and the LSE merge must not overflow."""
    rng = np.random.default_rng(14)
    q = (rng.standard_normal(NH * HD) * 12).astype(np.float32)
    k = (rng.standard_normal((NKV, 1024, HD)) * 2).astype(np.float16)
    v = rng.standard_normal((NKV, 1024, HD)).astype(np.float16)
    out = E.kernel_attention("opt", q, k, v, 1000, NH, NKV, HD, 1024)
    assert np.all(np.isfinite(out))
    assert np.allclose(out, K.attention(q, k, v, 1000, NH, NKV, HD), rtol=1e-4, atol=1e-4)


def test_silu_mul():
    gu = (np.random.default_rng(14).standard_normal(2 * 8192) * 2).astype(np.float32)
    assert np.allclose(E.kernel_silu_mul(gu), K.silu_mul(gu), rtol=1e-5)
    # the whole range where e^-g is a finite float, and past it (silu -> 0 below, -> g above)
    g = np.concatenate([np.linspace(-87, 87, 8192), np.array([-200.0, -100.0, -88.5, 88.5, 100.0, 200.0] + [0.0] * 8186)])
    gu = np.concatenate([g, np.ones_like(g)]).astype(np.float32)
    got, want = E.kernel_silu_mul(gu), K.silu_mul(gu)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-30)


VOCAB = 128256


def test_argmax_random():
    lg = np.random.default_rng(15).standard_normal(VOCAB).astype(np.float32)
    assert E.kernel_argmax(lg) == K.argmax_lowest(lg)


def test_argmax_tie_lowest_index():
    lg = np.random.default_rng(16).standard_normal(VOCAB).astype(np.float32)
    lg[5] = lg[100000] = 50.0
    assert E.kernel_argmax(lg) == 5


def test_argmax_last_index():
    lg = np.random.default_rng(17).standard_normal(VOCAB).astype(np.float32)
    lg[-1] = 50.0
    assert E.kernel_argmax(lg) == VOCAB - 1


@pytest.mark.parametrize("n", [1, 255, 256, 65537])
def test_argmax_sizes_and_all_equal(n):
    assert E.kernel_argmax(np.zeros(n, np.float32)) == 0
    lg = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    assert E.kernel_argmax(lg) == K.argmax_lowest(lg)


# ---- quantisers: bit-exact against the oracle (reference python/cudallm/quantize.py) ----------

@pytest.mark.parametrize("rows,cols", [(64, 256), (8192, 2048), (3, 128)])
def test_quantize_int8_bit_exact(rows, cols):
    w = np.random.default_rng(rows + cols).normal(0, 0.02, size=(rows, cols)).astype(np.float32)
    w[0, :4] = [1.27, -1.27, 0.005, 0.015]  # exact .5 ties under s = 0.01
    w[-1] = 0.0  # zero row -> scale 1
    q, s = GQ.quantize_int8_rows(w)
    q_ref, s_ref = Q.quantize_int8_rows(w)
    np.testing.assert_array_equal(s, s_ref)
    np.testing.assert_array_equal(q, q_ref)


@pytest.mark.parametrize("rows,cols", [(32, 512), (8192, 2048), (1, 128)])
def test_quantize_int4_bit_exact(rows, cols):
    w = np.random.default_rng(rows * cols).normal(0, 0.02, size=(rows, cols)).astype(np.float32)
    w[0, :4] = [7.0, -7.0, 0.0, 1.0]
    if rows > 1:
        w[1, :128] = 0.0  # zero group -> scale fp16(1)
    p, s = GQ.quantize_int4_groups(w, 128)
    p_ref, s_ref = Q.quantize_int4_groups(w, 128)
    np.testing.assert_array_equal(s.view(np.uint16), s_ref.view(np.uint16))
    np.testing.assert_array_equal(p, p_ref)
    np.testing.assert_array_equal(GQ.unpack_int4(p), Q.unpack_int4(p_ref))


def test_unpack_roundtrip_and_known_answer():
    np.testing.assert_array_equal(GQ.unpack_int4(np.array([[0x0F, 0x98]], dtype=np.uint8)), [[7, -8, 0, 1]])
    q = np.random.default_rng(3).integers(-8, 8, size=(16, 256), dtype=np.int8)
    u = (q + 8).astype(np.uint8)
    np.testing.assert_array_equal(GQ.unpack_int4((u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)), q)
