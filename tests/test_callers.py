"""The reference's callers and benchmark tools: generate.py (python/cudallm/generate.py:1-57), eval_ppl.py
(bench/eval_ppl.py:1-92), cudallm_kernelbench --op shapes (src/tools/cudallm_kernelbench.cpp:253-298) and
sweep_matvec.py (bench/sweep_matvec.py:1-48).

The Llama-3 tokenizer and checkpoint are not available offline, so a word-level tokenizer over the same 128,256 ids
(with the Llama-3 special ids and a chat template) is built in the test, and the model is a seeded synthetic file.
"""
import io
import math
import re
from pathlib import Path

import numpy as np
import pytest

from cudallm_amd import eval_ppl as P
from cudallm_amd import generate as G
from cudallm_amd import kernelbench as K
from cudallm_amd import profsum as PS
from cudallm_amd import sweep_matvec as S

VOCAB = 128256
SPECIAL = {0: "<unk>", 128000: "<|begin_of_text|>", 128001: "<|end_of_text|>", 128006: "<|start_header_id|>",
           128007: "<|end_header_id|>", 128008: "<|eom_id|>", 128009: "<|eot_id|>"}
CHAT = ("{{ bos_token }}{% for m in messages %}<|start_header_id|> {{ m['role'] }} <|end_header_id|> "
        "{{ m['content'] }} <|eot_id|> {% endfor %}{% if add_generation_prompt %}<|start_header_id|> w7 "
        "<|end_header_id|>{% endif %}")


def make_tokenizer(d: Path):
    """Word-level tokenizer: id i is the word "w<i>" except the special ids; saved to `d` and loaded back with
    AutoTokenizer, as the callers load theirs."""
    from tokenizers import Tokenizer, decoders, models, pre_tokenizers
    from transformers import AutoTokenizer, PreTrainedTokenizerFast
    tok = Tokenizer(models.WordLevel(vocab={SPECIAL.get(i, f"w{i}"): i for i in range(VOCAB)}, unk_token="<unk>"))
    tok.pre_tokenizer = pre_tokenizers.WhitespaceSplit()
    tok.decoder = decoders.WordPiece(prefix="##")
    ft = PreTrainedTokenizerFast(tokenizer_object=tok, bos_token=SPECIAL[128000], eos_token=SPECIAL[128009],
                                 unk_token="<unk>", additional_special_tokens=[v for k, v in SPECIAL.items() if k])
    ft.chat_template = CHAT
    ft.save_pretrained(d)
    return AutoTokenizer.from_pretrained(d)


@pytest.fixture(scope="module")
def tokenizer_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("tok")
    make_tokenizer(d)
    return d


@pytest.fixture(scope="module")
def tokenizer(tokenizer_dir):
    from transformers import AutoTokenizer
    return AutoTokenizer.from_pretrained(tokenizer_dir)


# ---- eval_ppl -------------------------------------------------------------------------------------------------

def test_nll_from_logits():
    """Closed forms: logits (0, ln 3) are probabilities (1/4, 3/4); uniform logits give log(n); a common offset that
    would overflow a naive exp does not change the result; and the token NLLs of a random row sum, after exp, to
    softmax's total of 1."""
    z = np.array([0.0, math.log(3.0)], np.float32)
    assert math.isclose(P.nll_from_logits(z, 0), math.log(4.0), rel_tol=1e-6)
    assert math.isclose(P.nll_from_logits(z, 1), math.log(4.0 / 3.0), rel_tol=1e-6)
    big = np.array([1e4, 1e4 + math.log(3.0)])  # exp(1e4) overflows float64: the evaluation must shift
    assert math.isclose(P.nll_from_logits(big, 0), math.log(4.0), rel_tol=1e-9)
    assert math.isclose(P.nll_from_logits(np.zeros(VOCAB, np.float32), 5), math.log(VOCAB), rel_tol=1e-14)
    r = (np.random.default_rng(0).standard_normal(5000) * 4).astype(np.float32)
    assert math.isclose(sum(math.exp(-P.nll_from_logits(r, t)) for t in range(r.size)), 1.0, rel_tol=1e-9)


def test_windows_and_perplexity():
    ids = [G.BOS_ID] + list(range(1, 26))
    w = P.windows_from_ids(ids, 3, 8)
    assert w == [list(range(1, 9)), list(range(9, 17)), list(range(17, 25))]
    assert P.windows_from_ids(list(range(1, 26)), 3, 8) == w  # no BOS to drop
    with pytest.raises(ValueError, match="only 25 tokens"):
        P.windows_from_ids(ids, 4, 8)
    assert math.isclose(P.perplexity([1.0, 2.0, 3.0]), math.exp(2.0))


def test_eval_ppl_text_pipeline(tokenizer, tmp_path):
    """Tokenise a local text the way main() does: the BOS the tokenizer adds is dropped, windows are consecutive."""
    f = tmp_path / "t.txt"
    f.write_text(" ".join(f"w{i}" for i in range(100, 140)), encoding="utf-8")
    text, desc = P.load_text(f)
    assert desc == "file t.txt"
    ids = tokenizer(text).input_ids
    wins = P.windows_from_ids(ids, 2, 16)
    assert wins == [list(range(100, 116)), list(range(116, 132))]


# ---- generate -------------------------------------------------------------------------------------------------

class ScriptedEngine:
    """Stands in for Engine.step: returns the scripted next tokens and records what was fed."""

    def __init__(self, nexts):
        self.nexts, self.fed = list(nexts), []

    def step(self, token=None):
        self.fed.append(token)
        return self.nexts.pop(0), None


def test_prompt_ids(tokenizer):
    assert G.prompt_ids(tokenizer, "w5 w17", chat=False)[-2:] == [5, 17]
    chat = G.prompt_ids(tokenizer, "w5 w17")
    assert chat == [128000, 128006, 0, 128007, 5, 17, 128009, 128006, 7, 128007]


def test_generate_stops_at_end_ids_and_limit(tokenizer):
    """generate.py:36-53: prompt fed in order, then the argmax fed back (token None) until an end id."""
    eng = ScriptedEngine([9, 9, 10, 11, 12, 128009, 13])
    out = io.StringIO()
    gen, _ = G.generate(eng, tokenizer, [1, 2, 3], 100, out)
    assert eng.fed == [1, 2, 3, None, None, None]
    assert gen == [10, 11, 12] and out.getvalue() == "w10 w11 w12"
    for end in G.EOS_IDS:
        assert G.generate(ScriptedEngine([10, end, 11]), tokenizer, [1], 100)[0] == [10]
    eng = ScriptedEngine([10, 11, 12, 13])
    assert G.generate(eng, tokenizer, [1], 2)[0] == [10, 11] and eng.fed == [1, None]


def test_default_paths_follow_the_reference_layout(tmp_path):
    m, t = G.default_paths(tmp_path, "int4")
    assert m == tmp_path / "llama-3.2-1b-instruct.int4.cudallm"
    assert t == tmp_path / "hf" / "Llama-3.2-1B-Instruct"


# ---- kernelbench / sweep ---------------------------------------------------------------------------------------

def test_matvec_bytes_known_answers():
    """Algorithmic bytes of the engine's shapes (weights + scales), as the reference's results report them."""
    want = {("qkv", "bf16"): 12582912, ("qkv", "int8"): 6303744, ("qkv", "int4"): 3244032,
            ("gate_up", "bf16"): 67108864, ("gate_up", "int8"): 33619968, ("gate_up", "int4"): 17301504,
            ("down", "bf16"): 33554432, ("down", "int8"): 16785408, ("down", "int4"): 8650752,
            ("lm_head", "bf16"): 525336576, ("lm_head", "int8"): 263181312, ("lm_head", "int4"): 135438336}
    shapes = {s[0]: s for s in K.SHAPES}
    for (name, wd), b in want.items():
        assert K.matvec_bytes(wd, shapes[name][1], shapes[name][2]) == b


def test_weighted_us_and_winner_rule():
    assert K.weighted_us({"qkv": 1.0, "wo": 2.0, "gate_up": 3.0, "down": 4.0, "lm_head": 5.0}) == 165.0
    assert S.pick_winners({"bf16": {8: 4.0, 4: 4.0, 2: 4.5, 1: 9.0}, "int8": {1: 3.0, 2: 2.0, 4: 2.5, 8: 2.0}}) == \
        {"bf16": 4, "int8": 2}


def test_default_rpb_matches_the_library():
    src = (Path(__file__).resolve().parents[1] / "cudallm_amd/csrc/kernels/small.hip").read_text()
    body = src[src.index("constexpr int kDefaultRpb[3][4]"):]
    got = {m.group(5): tuple(int(m.group(i)) for i in range(1, 5))
           for m in re.finditer(r"\{(\d+), (\d+), (\d+), (\d+)\},\s*// (\w+)", body[:body.index("kGridPerCu")])}
    assert got == K.DEFAULT_RPB
    grid = src[src.index("constexpr int kGridPerCu[3][4]"):]
    got = {m.group(5): tuple(int(m.group(i)) for i in range(1, 5))
           for m in re.finditer(r"\{(\d+), (\d+), (\d+), (\d+)\},\s*// (\w+)", grid[:300])}
    assert got == K.GRID_PER_CU
    assert "ep == Epilogue::SWIGLU ? 1 : cols >= 8192 ? 2 : rows >= 65536 ? 3 : 0" in body
    assert [K.default_rpb("bf16", ep, r, c) for _, r, c, ep, _ in K.SHAPES] == [1, 1, 1, 2, 2]
    assert [K.default_rpb("int4", ep, r, c) for _, r, c, ep, _ in K.SHAPES] == [4, 4, 4, 8, 4]


def test_shape_winners():
    rec = lambda ts: {"results": [{"name": n, "avg_us": t} for n, t in zip(("qkv", "lm_head"), ts)]}
    data = {"bf16": {"1": rec((5.0, 90.0)), "2": rec((5.0, 80.0)), "4": rec((4.0, 85.0))}}
    assert S.shape_winners(data) == {"bf16": {"qkv": 4, "lm_head": 2}}


def test_clis_parse():
    for main in (G.main, P.main, K.main, S.main):
        with pytest.raises(SystemExit) as e:
            main(["--help"])
        assert e.value.code == 0


# ---- on the GPU ------------------------------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_generate_cli_matches_engine_greedy(gpu, tokenizer_dir, tmp_path, capsys):
    """The CLI's streamed text is the decoded greedy continuation, with the reference's summary line."""
    from transformers import AutoTokenizer
    from cudallm_amd import engine as E
    from cudallm_amd import synth
    path = tmp_path / "gen_bf16.cudallm"
    synth.write_model(path, "bf16", seed=7)
    tok = AutoTokenizer.from_pretrained(tokenizer_dir)
    prompt = "w5 w17 w300 w4096"
    ids = G.prompt_ids(tok, prompt)
    n = 12
    with E.Engine(path) as eng:
        nxt = None
        for t in ids:
            nxt, _ = eng.step(t)
        greedy = []
        while nxt not in G.EOS_IDS and len(greedy) < n:
            greedy.append(nxt)
            if len(greedy) < n:
                nxt, _ = eng.step(None)
    assert G.main(["--prompt", prompt, "--max-new-tokens", str(n), "--model", str(path),
                   "--tokenizer", str(tokenizer_dir)]) == 0
    out = capsys.readouterr().out
    text, summary = out.rsplit("\n", 2)[-3], out.rstrip("\n").rsplit("\n", 1)[-1]
    print(f"[callers] generated {greedy}", flush=True)
    assert text == tok.decode(greedy)
    m = re.fullmatch(r"\[prompt_tokens=(\d+) generated=(\d+) decode_tok_s=([\d.]+)\]", summary)
    assert m and int(m.group(1)) == len(ids) and int(m.group(2)) == len(greedy) and float(m.group(3)) > 0


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_eval_ppl_cli(gpu, tokenizer_dir, tmp_path):
    """main() end to end on a local text: the JSON record of the reference's schema, PPL = exp(mean window NLL)."""
    import json
    from cudallm_amd import synth
    path = tmp_path / "ppl_int8.cudallm"
    synth.write_model(path, "int8", seed=7)
    text = tmp_path / "t.txt"
    text.write_text(" ".join(f"w{(i * 7919) % 120000 + 1000}" for i in range(40)), encoding="utf-8")
    assert P.main(["--target", "engine", "--dtype", "int8", "--windows", "2", "--window-len", "16", "--text-file",
                   str(text), "--model", str(path), "--tokenizer", str(tokenizer_dir), "--out", str(tmp_path)]) == 0
    rec = json.loads((tmp_path / "engine_int8.json").read_text())
    assert rec["tool"] == "eval_ppl" and rec["n_tokens"] == 32 and len(rec["window_mean_nll"]) == 2
    assert math.isclose(rec["ppl"], math.exp(np.mean(rec["window_mean_nll"])), rel_tol=1e-12)
    print(f"[callers] synthetic int8 PPL {rec['ppl']:.1f}", flush=True)
    assert 1.0 < rec["ppl"] < 10 * VOCAB


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_kernelbench_shapes_record(gpu):
    """--op shapes on small rotations: the reference's fields, weighted_us from the medians."""
    import torch
    rec_rows = []
    for name, rows, cols, ep, norm in K.SHAPES[:4]:
        r = K.bench_matvec("int4", name, rows, cols, ep, norm, 20, rpb=2, rotate_bytes=64 << 20)
        rec_rows.append(r)
        assert r["rpb"] == 2 and r["bytes"] == K.matvec_bytes("int4", rows, cols)
        assert 0 < r["median_us"] < 1e4 and r["gbps"] == pytest.approx(r["bytes"] / r["median_us"] / 1e3)
    torch.cuda.synchronize()


def _row(name, start_us, dur_us, grid=65536):
    return {"Kernel_Name": name, "Start_Timestamp": str(int(start_us * 1000)),
            "End_Timestamp": str(int((start_us + dur_us) * 1000)), "Grid_Size_X": str(grid)}


def test_profsum_matvec_blocks_with_stream_reads():
    """Runs of one matvec kernel per shape, each followed by stream reads at two grid sizes (5 warm-up each)."""
    rows, t = [], 0.0
    for k, (name, r, c, ep, norm) in enumerate(K.SHAPES):
        for _ in range(3):
            rows.append(_row(f"void cllm::mv::matvec_fast<k{k}>(cllm::MatvecArgs)", t, 10.0 + k))
            t += 20
        for grid, dur in ((1024, 9.0), (2048, 8.0)):
            for i in range(7):
                rows.append(_row("stream_read_kernel<8>", t, 100.0 if i < 5 else dur, grid))
                t += 200
    out = PS.matvec_blocks(rows, "bf16")
    assert [o["shape"] for o in out] == [s[0] for s in K.SHAPES]
    assert [o["calls"] for o in out] == [3] * 5 and out[2]["mean_us"] == pytest.approx(12.0)
    assert all(o["stream_mean_us"] == pytest.approx(8.0) for o in out)
    assert out[0]["bytes"] == K.matvec_bytes("bf16", 3072, 2048)


def test_profsum_bench_legs():
    """bench.py's launch sequence: warm-up sequence, prompt, K timed, one more, then 6 config-5 sequences."""
    K_, W = 3, 2
    durs = [1.0] * (16 + W + 16) + [5.0] * K_ + [1.0]
    for rep in range(6):
        durs += [1.0] * 16 + [7.0 if rep else 3.0] * 256
    rows = [_row("decode_kernel<(cllm::WType)4>", 1000.0 * i, 60.0 + d) for i, d in enumerate(durs)]
    rows.append(_row("decode_kernel<(cllm::WType)4>", -100.0, 5.0))  # a co-residency probe
    leg = PS.bench_legs(rows, K_, W)["int4"]
    assert leg["decode_timed"]["calls"] == K_ and leg["decode_timed"]["mean_us"] == pytest.approx(65.0)
    assert leg["config5_timed"]["calls"] == 1280 and leg["config5_timed"]["mean_us"] == pytest.approx(67.0)
    assert leg["launches"] == leg["expected_launches"] == len(durs)


def test_bench_decode_markdown_table(tmp_path):
    """--table: saved runs in suite order, and the long-context and ctx-4000 ratios."""
    import json
    from cudallm_amd import bench_decode as B

    def save(suite, name, wd, plen, tok):
        d = tmp_path / suite
        d.mkdir(exist_ok=True)
        rec = {"weight_dtype": wd, "options": {"matvec": "opt", "attn": "opt", "fuse": 1, "graph": 1},
               "prompt_len": plen, "gen": 32, "decode_tok_s_median": tok, "ms_per_token_median": 1e3 / tok,
               "achieved_gbps_median": 4000.0, "pct_of_peak": 50.0}
        (d / f"{name}.json").write_text(json.dumps(rec))

    save("long", "long_bf16_8000", "bf16", 8000, 1600.0)
    save("tg", "tg_bf16", "bf16", 1, 2000.0)
    save("context", "ctx_opt_128", "bf16", 128, 1850.0)
    text = B.markdown_table(tmp_path)
    rows = [l for l in text.splitlines() if l.startswith("| ") and "---" not in l][1:]
    assert [r.split(" | ")[1] for r in rows] == ["ctx_opt_128", "tg_bf16", "long_bf16_8000"]
    assert "long_bf16_8000: 1600.0 tok/s, 20.0 % below tg_bf16 (2000.0)" in text
    assert "ctx_opt_4000" not in text
