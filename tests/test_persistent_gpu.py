"""GPU parity of the persistent decode kernel past one attention split, phase by phase.

* Every phase of the fused kernel against float64, from that phase's own inputs as the kernel saw them
  (cudallm_step_trace), at the reference's single-kernel tolerances (tests/test_kernels.py:50,96,196 of the
  reference: rtol = atol = 1e-4): qkv with the RMSNorm prologue and RoPE, split-K attention with its LSE merge,
  wo + residual, gate_up with the RMSNorm prologue and SwiGLU, down + residual, lm_head with the final norm.
  This pins the persistent kernel's own row dots (fp32 FMA for bf16, biased-byte and integer-digit dots for
  int8/int4), not only the standalone matvec kernels the hooks run.
* The headline benchmark's whole sequence (16 prompt tokens + 256 greedy tokens) against the CPU oracle at the
  integration tolerances of the reference's tests/test_engine_vs_reference.py:62-94.
* Timing perturbation, the epoch restart of the tagged words, contexts past 8192 and the largest max_seq_len
  against unperturbed runs or the multi-kernel path, for every weight type.
Every engine these tests time or trace is checked to run the persistent kernel (cudallm_get_step_kind), so a
device where its grid was not resident cannot pass them on the multi-kernel step.
"""
import os

import numpy as np
import pytest

from cudallm_amd import engine as E
from oracle import fileformat as ff
from oracle import kernels as K
from oracle.model import OracleModel

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

RTOL = ATOL = 1e-4          # reference tests/test_kernels.py:50,96 (matvec), :196 (attention)
NH, NKV, HD, H, I = 32, 8, 64, 2048, 8192
PROMPT = [128000] + [int(t) for t in np.random.default_rng(16).integers(0, 128256, 15)]
SEQ_STEPS = 272             # the headline run: 16 prompt + 256 generated positions
TRACE_CHECK_POS = (0, 1, 127, 128, 129, 255, 256, 257, 271)
TRACE_CHECK_LAYERS = (0, 6, 15)


def _threads() -> int:
    return min(16, os.cpu_count() or 1)


class _Weights:
    """float64 dequantised operands of selected layers, read from the file with the oracle's reader."""

    def __init__(self, path):
        self.path = str(path)
        self.table = {e["name"]: e for e in ff.read_table(path)}
        self.quant = ff.read_header(path)["weight_dtype"] != ff.WEIGHT_BF16

    def vec(self, name):
        return np.asarray(ff.load(self.path, self.table[name]), dtype=np.float64)

    def mat(self, name, rows=None):
        from oracle import quantize as Q
        w = self.table[name + ".weight"]
        raw = np.asarray(ff.load(self.path, w))
        if rows is not None:
            raw = raw[rows]
        if w["dtype"] == ff.BF16:
            return Q.bf16_bits_to_f32(raw.view(np.uint16)).astype(np.float64)
        s = np.asarray(ff.load(self.path, self.table[name + ".scales"]))
        if rows is not None:
            s = s[rows]
        if w["dtype"] == ff.I8:
            return raw.astype(np.float64) * s.astype(np.float64).reshape(-1, 1)
        q = Q.unpack_int4(raw).astype(np.float64)
        g = s.astype(np.float64)
        return (q.reshape(q.shape[0], g.shape[1], -1) * g[:, :, None]).reshape(q.shape[0], -1)


def _persistent(eng):
    kind, grid = eng.step_kind
    assert kind == "persistent" and grid > 0, f"the engine runs the {kind} step, not the persistent kernel"
    return eng


def _close(name, got, want):
    got = np.asarray(got, dtype=np.float64)
    err = np.abs(got - want) - (ATOL + RTOL * np.abs(want))
    worst = int(np.argmax(err))
    assert err[worst] <= 0, (f"{name}: |got - want| exceeds atol + rtol*|want| at {worst}: got {got.flat[worst]:.7g}, "
                             f"want {want.flat[worst]:.7g}")
    return float(np.max(np.abs(got - want)))


@pytest.mark.parametrize("wd", ["bf16", "int8", "int4"])
def test_phases_match_float64(wd, model_path):
    """272 greedy steps traced; at positions on both sides of the 128- and 256-token split boundaries, layers 0, 6
    and 15 are recomputed in float64 from the kernel's own phase inputs.  The attention reference uses the fp16 K/V
    cache rebuilt from every earlier step's traced k and v (the kernel rounds them to fp16 the same way)."""
    path = model_path(wd)
    ws = _Weights(path)
    inv_freq = ws.vec("rope.inv_freq").astype(np.float32)
    traces, logits_at = {}, {}
    kv = {l: (np.zeros((NKV, SEQ_STEPS, HD), np.float16), np.zeros((NKV, SEQ_STEPS, HD), np.float16))
          for l in TRACE_CHECK_LAYERS}
    with E.Engine(path, max_seq_len=4096) as eng:
        _persistent(eng)
        tok = PROMPT[0]
        for p in range(SEQ_STEPS):
            nxt, lg, tr = eng.step_trace(PROMPT[p] if p < len(PROMPT) else None)
            for l in TRACE_CHECK_LAYERS:
                kv[l][0][:, p] = tr["qkv"][l][NH * HD:(NH + NKV) * HD].reshape(NKV, HD).astype(np.float16)
                kv[l][1][:, p] = tr["qkv"][l][(NH + NKV) * HD:].reshape(NKV, HD).astype(np.float16)
            if p in TRACE_CHECK_POS:
                traces[p] = {k: v.copy() for k, v in tr.items()}
                logits_at[p] = lg
            assert nxt == int(np.argmax(lg))
            tok = nxt
    del tok
    worst = {}
    for l in TRACE_CHECK_LAYERS:
        pre = f"layers.{l}."
        an, fn = ws.vec(pre + "attn_norm.weight"), ws.vec(pre + "ffn_norm.weight")
        wqkv, wo = ws.mat(pre + "wqkv"), ws.mat(pre + "wo")
        wgu, wd_ = ws.mat(pre + "w_gate_up"), ws.mat(pre + "w_down")
        for p in TRACE_CHECK_POS:
            tr = traces[p]
            x_in = tr["residuals"][l]
            qkv = K.matvec(wqkv, x_in, "store", an, 1e-5)
            q = K.rope(qkv[:NH * HD].reshape(NH, HD), inv_freq, p).reshape(-1)
            k = K.rope(qkv[NH * HD:(NH + NKV) * HD].reshape(NKV, HD), inv_freq, p).reshape(-1)
            want_qkv = np.concatenate([q, k, qkv[(NH + NKV) * HD:]])
            worst["qkv"] = max(worst.get("qkv", 0), _close(f"L{l} pos {p} qkv", tr["qkv"][l], want_qkv))
            kc, vc = kv[l]
            want_att = K.attention(tr["qkv"][l][:NH * HD], kc, vc, p + 1, NH, NKV, HD)
            worst["att"] = max(worst.get("att", 0), _close(f"L{l} pos {p} attention", tr["att"][l], want_att))
            want_xa = K.matvec(wo, tr["att"][l], "add", None, 1e-5, x_in)
            worst["xa"] = max(worst.get("xa", 0), _close(f"L{l} pos {p} wo + residual", tr["xa"][l], want_xa))
            want_act = K.matvec(wgu, tr["xa"][l], "swiglu", fn, 1e-5)
            worst["act"] = max(worst.get("act", 0), _close(f"L{l} pos {p} gate_up SwiGLU", tr["act"][l], want_act))
            want_x = K.matvec(wd_, tr["act"][l], "add", None, 1e-5, tr["xa"][l])
            worst["down"] = max(worst.get("down", 0),
                                _close(f"L{l} pos {p} down + residual", tr["residuals"][l + 1], want_x))
        del wqkv, wo, wgu, wd_
    # lm_head with the final norm, in blocks of rows (the float64 embedding would take 2 GB at once).
    fin = ws.vec("norm.weight")
    for p in (0, 128, 271):
        x = K.rms_normalize(traces[p]["residuals"][-1], fin, 1e-5)
        want = np.concatenate([ws.mat("tok_embeddings", slice(r, min(r + 16384, 128256))) @ x
                               for r in range(0, 128256, 16384)])
        worst["lm_head"] = max(worst.get("lm_head", 0), _close(f"pos {p} lm_head", logits_at[p], want))
    print(f"[phases {wd}] worst |got - float64| per phase: " + ", ".join(f"{k} {v:.2e}" for k, v in worst.items()),
          flush=True)


@pytest.mark.parametrize("wd", ["bf16", "int8", "int4"])
def test_config5_sequence_matches_oracle(wd, model_path):
    """The headline run: a 16-token prompt and the oracle's own 256 greedy tokens, teacher-forced through the
    persistent kernel.  Logits within 2e-2 at every position, the engine's argmax equal to the oracle's token
    except at near-ties (oracle margin < 2e-2), and the residual stream within rel-L2 1e-3 at the split
    boundaries (reference tests/test_engine_vs_reference.py:62-94)."""
    path = model_path(wd)
    m = OracleModel(path, cache_dense=True, threads=_threads())
    toks, ref_logits, ref_res = list(PROMPT), [], {}
    check_res = {0, 15, 127, 128, 129, 255, 256, 257, SEQ_STEPS - 1}
    for p in range(SEQ_STEPS):
        lg, res = m.step(toks[p])
        ref_logits.append(lg.numpy())
        if p in check_res:
            ref_res[p] = np.stack([r.numpy() for r in res])
        if p + 1 >= len(toks):
            toks.append(int(np.argmax(ref_logits[-1])))
    del m
    worst_lg, worst_res, ties = 0.0, 0.0, []
    with E.Engine(path, max_seq_len=4096) as eng:
        _persistent(eng)
        for p in range(SEQ_STEPS):
            if p in check_res:
                nxt, lg, res = eng.step_debug(toks[p])
                ref = ref_res[p].astype(np.float64)
                rel = np.linalg.norm(res - ref, axis=1) / np.linalg.norm(ref, axis=1)
                worst_res = max(worst_res, float(rel.max()))
                assert rel.max() < 1e-3, f"position {p}: residual rel-L2 {rel.max():.3e} at layer {int(rel.argmax())}"
            else:
                nxt, lg = eng.step(toks[p], want_logits=True)
            ref = ref_logits[p]
            d = float(np.abs(lg - ref).max())
            worst_lg = max(worst_lg, d)
            assert d < 2e-2, f"position {p}: max |logit - oracle| = {d:.3e}"
            want = int(np.argmax(ref))
            if nxt != want:
                margin = float(ref[want] - ref[nxt])
                ties.append((p, margin))
                assert margin < 2e-2, f"position {p}: engine {nxt}, oracle {want}, oracle margin {margin:.3e}"
    assert len(ties) <= 2, f"argmax differs at {ties}"
    print(f"[config5 {wd}] {SEQ_STEPS} positions: worst |dlogit| {worst_lg:.2e}, worst residual rel {worst_res:.2e}, "
          f"near-tie argmax differences {ties}", flush=True)


# Bits of DecodeParams::stall (cudallm_amd/csrc/decode.h): 0x10 before the down projection's input wait,
# 0x02 before attention, 0x40 loader segment switches, 0x80 odd workgroups only, 0x100 + 0x200 compute wave 0
# between its input barrier and its input reads.
SPLIT_STALLS = {"attn_odd": 0x82, "down_odd": 0x90, "loader": 0x40, "w0_inputs_odd": 0x380}


@pytest.mark.parametrize("wd", ["bf16", "int8", "int4"])
def test_stalls_across_splits_bit_identical(wd, model_path, monkeypatch):
    """Timing perturbation with 2 attention splits (positions 128..139): the split partial handoff and the LSE
    merge phase under skew.  Residuals and logits must equal the unperturbed run bit for bit."""
    steps = 140
    toks = PROMPT + [int(t) for t in np.random.default_rng(5).integers(0, 128256, steps - len(PROMPT))]

    def run():
        out = []
        with E.Engine(model_path(wd), max_seq_len=256) as eng:
            _persistent(eng)
            for p, t in enumerate(toks):
                if p >= 126:
                    _, lg, res = eng.step_debug(t)
                    out.append((lg, res))
                else:
                    eng.step_async(t)
        return out

    base = run()
    for name, mask in SPLIT_STALLS.items():
        monkeypatch.setenv("CUDALLM_STALL", hex(mask))
        try:
            got = run()
        finally:
            monkeypatch.delenv("CUDALLM_STALL")
        for i, ((lg, res), (blg, bres)) in enumerate(zip(got, base)):
            np.testing.assert_array_equal(res, bres, err_msg=f"stall {name}, position {126 + i}: residuals")
            np.testing.assert_array_equal(lg, blg, err_msg=f"stall {name}, position {126 + i}: logits")
        print(f"[stalls {wd}] {name} ({mask:#x}): bit-identical over positions 126..{steps - 1}", flush=True)


@pytest.mark.parametrize("wd", ["bf16", "int8", "int4"])
def test_epoch_restart_is_bit_identical(wd, model_path, monkeypatch):
    """The host restarts the tag epochs (clears every tagged word, step counter back to 0) before the 32-bit tags
    could repeat; CUDALLM_EPOCH_LIMIT brings that point down to every 50 launches.  200 positions (2 splits, 3
    restarts, one of them between a reset and the next sequence) must give the same logits bit for bit."""
    toks = PROMPT + [int(t) for t in np.random.default_rng(9).integers(0, 128256, 200 - len(PROMPT))]

    def run():
        lgs = []
        with E.Engine(model_path(wd), max_seq_len=256) as eng:
            _persistent(eng)
            for t in toks[:30]:
                eng.step_async(t)
            eng.reset()
            for p, t in enumerate(toks):
                if p % 13 == 0 or p >= 190:
                    lgs.append(eng.step(t, want_logits=True)[1])
                else:
                    eng.step_async(t)
        return np.stack(lgs)

    base = run()
    monkeypatch.setenv("CUDALLM_EPOCH_LIMIT", "50")
    try:
        got = run()
    finally:
        monkeypatch.delenv("CUDALLM_EPOCH_LIMIT")
    np.testing.assert_array_equal(got, base)


@pytest.mark.parametrize("wd", ["bf16", "int8", "int4"])
def test_context_past_8192_matches_multikernel(wd, model_path, monkeypatch):
    """max_seq_len 16384 on the persistent kernel (more than 64 splits: the merge loops over 64-split blocks)
    against the multi-kernel path, teacher-forced to position 9000.  int4 writes the current token's KV rows from
    the attention workgroup, bf16 and int8 from the qkv phase: both writers are covered past 8192 positions."""
    steps = 9000
    monkeypatch.setenv("CUDALLM_PERSISTENT", "0")
    ref = E.Engine(model_path(wd), max_seq_len=16384)
    monkeypatch.delenv("CUDALLM_PERSISTENT")
    eng = E.Engine(model_path(wd), max_seq_len=16384)
    try:
        assert ref.step_kind[0] == "program"
        _persistent(eng)
        toks, worst, agree, checked = [128000], 0.0, 0, 0
        for i in range(steps):
            check = i in (8190, 8191, 8192, 8193, 8319, 8320, 8999)
            n_ref, lg_ref = ref.step(toks[-1], want_logits=check)
            n_eng, lg_eng = eng.step(toks[-1], want_logits=check)
            if check:
                worst = max(worst, float(np.abs(lg_eng - lg_ref).max()) / float(np.abs(lg_ref).max()))
                agree += int(n_eng == n_ref)
                checked += 1
            toks.append(n_ref)
        print(f"[engine] {wd} persistent vs multi-kernel to ctx {steps}: worst rel logit diff {worst:.2e}, "
              f"argmax agree {agree}/{checked}", flush=True)
        assert worst < 2e-3 and agree >= checked - 1
    finally:
        eng.close()
        ref.close()


@pytest.mark.parametrize("wd", ["bf16", "int8", "int4"])
def test_largest_max_seq_matches_multikernel(wd, model_dir, gpu):
    """max_seq_len 131072 (Llama-3.2's context, the kernel's largest: 1024 split slots per head, 4.3 GB of KV cache)
    against the multi-kernel path over 300 positions (three splits): every stride that grows with max_seq_len (the
    layer's KV cache, the split partials) at its largest value.  Contexts past 64 splits are the test above."""
    from cudallm_amd import synth
    path = model_dir / f"synth_seed7_{wd}_ms131072.cudallm"
    if not path.exists():
        synth.write_model(path, wd, seed=7, max_seq_len=131072)
    os.environ["CUDALLM_PERSISTENT"] = "0"
    try:
        ref = E.Engine(path)
    finally:
        del os.environ["CUDALLM_PERSISTENT"]
    eng = E.Engine(path)
    try:
        assert ref.step_kind[0] == "program" and eng.config["max_seq_len"] == 131072
        _persistent(eng)
        toks, worst = [128000], 0.0
        for i in range(300):
            check = i in (0, 127, 128, 255, 256, 299)
            n_ref, lg_ref = ref.step(toks[-1], want_logits=check)
            n_eng, lg_eng = eng.step(toks[-1], want_logits=check)
            if check:
                worst = max(worst, float(np.abs(lg_eng - lg_ref).max()) / float(np.abs(lg_ref).max()))
                assert n_eng == n_ref or np.sort(lg_ref)[-2] > np.max(lg_ref) - 1e-3, f"argmax differs at {i}"
            toks.append(n_ref)
        print(f"[engine] {wd} max_seq 131072, 300 positions: worst rel logit diff {worst:.2e}", flush=True)
        assert worst < 2e-3
    finally:
        eng.close()
        ref.close()


def test_context_past_16384_matches_multikernel(model_dir, gpu):
    """Past 128 splits (three 64-split blocks in the long merge) on the persistent kernel at max_seq_len 32768, int8
    (its KV rows written in the qkv phase), against the multi-kernel path teacher-forced to position 17000."""
    from cudallm_amd import synth
    wd, steps = "int8", 17000
    path = model_dir / f"synth_seed7_{wd}_ms131072.cudallm"
    if not path.exists():
        synth.write_model(path, wd, seed=7, max_seq_len=131072)
    os.environ["CUDALLM_PERSISTENT"] = "0"
    try:
        ref = E.Engine(path, max_seq_len=32768)
    finally:
        del os.environ["CUDALLM_PERSISTENT"]
    eng = E.Engine(path, max_seq_len=32768)
    try:
        assert ref.step_kind[0] == "program"
        _persistent(eng)
        toks, worst, agree, checked = [128000], 0.0, 0, 0
        for i in range(steps):
            check = i in (8191, 16383, 16384, 16385, 16511, 16512, 16999)
            n_ref, lg_ref = ref.step(toks[-1], want_logits=check)
            n_eng, lg_eng = eng.step(toks[-1], want_logits=check)
            if check:
                worst = max(worst, float(np.abs(lg_eng - lg_ref).max()) / float(np.abs(lg_ref).max()))
                agree += int(n_eng == n_ref)
                checked += 1
            toks.append(n_ref)
        print(f"[engine] {wd} persistent vs multi-kernel to ctx {steps} (max_seq 32768): worst rel logit diff "
              f"{worst:.2e}, argmax agree {agree}/{checked}", flush=True)
        assert worst < 2e-3 and agree >= checked - 1
    finally:
        eng.close()
        ref.close()


def test_trace_needs_the_persistent_kernel(model_path):
    with E.Engine(model_path("int4"), fuse=False, max_seq_len=256) as eng:
        with pytest.raises(E.CudaLLMError) as ei:
            eng.step_trace(1)
        assert ei.value.code == 5
