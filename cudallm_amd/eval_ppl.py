"""Perplexity of the engine, or of HF transformers, over fixed-length token windows (the reference's
bench/eval_ppl.py:1-92 measures the same quantity; its options and JSON record are kept).

    python -m cudallm_amd.eval_ppl --target {engine,hf} [--dtype bf16|int8|int4] [--windows 40] [--window-len 512]
                                   [--text-file FILE] [--model FILE] [--tokenizer DIR] [--models-dir DIR] [--out DIR]

Protocol (what makes the numbers comparable with the reference's): the text is tokenised once and a leading BOS is
dropped; the first `windows` x `window_len` tokens form consecutive windows.  Each window is scored from a fresh
sequence that starts with BOS: the logits after BOS score w[0], those after w[j] score w[j+1]; the negative
log-likelihoods are float64 log-softmax values of the fp32 logits, and PPL = exp(mean over windows of the window
mean), which equals the token mean because the windows have equal length.  The HF target scores the same windows
with the checkpoint in bf16 and must land in a sanity range, a guard against tokenisation or protocol mistakes.
The reference reads WikiText-2 (raw, test split) with `datasets`, which works here only where the dataset is in
the local cache; --text-file scores any local text instead.
"""
import argparse
import json
import math
import subprocess
import sys
from dataclasses import asdict, dataclass, field
from pathlib import Path

import numpy as np
from scipy.special import logsumexp

from .generate import BOS_ID, default_paths

HF_PPL_RANGE = (6.0, 25.0)  # the reference's sanity bounds for the bf16 checkpoint on WikiText-2
WIKITEXT = ("Salesforce/wikitext", "wikitext-2-raw-v1", "test")


def nll_from_logits(logits: np.ndarray, target: int) -> float:
    """Negative log-likelihood of `target` under softmax(logits), evaluated in float64."""
    z = np.asarray(logits, dtype=np.float64)
    return float(logsumexp(z) - z[target])


def windows_from_ids(ids, n_windows: int, window_len: int) -> list:
    """The token stream without its leading BOS, cut into `n_windows` consecutive windows of `window_len`."""
    stream = list(ids)[1:] if len(ids) and ids[0] == BOS_ID else list(ids)
    need = n_windows * window_len
    if len(stream) < need:
        raise ValueError(f"only {len(stream)} tokens in the text; {n_windows} windows of {window_len} need {need}")
    return [stream[at:at + window_len] for at in range(0, need, window_len)]


def load_text(text_file=None) -> tuple:
    """(text, dataset description): a local file, or the WikiText-2 test split with its lines joined by blank lines."""
    if text_file:
        return Path(text_file).read_text(encoding="utf-8"), f"file {Path(text_file).name}"
    from datasets import load_dataset
    name, config, split = WIKITEXT
    return "\n\n".join(load_dataset(name, config, split=split)["text"]), " ".join(WIKITEXT)


def _window_nll_engine(eng, window) -> float:
    """Mean NLL of one window through the engine, from a fresh sequence: BOS, then every token but the last."""
    eng.reset()
    inputs = [BOS_ID] + list(window[:-1])
    total = 0.0
    for fed, target in zip(inputs, window):
        _, logits = eng.step(fed, want_logits=True)
        total += nll_from_logits(logits, target)
    return total / len(window)


def eval_engine(model_path, windows: list, **engine_options) -> list:
    """Per-window mean NLL through this library's engine."""
    from .engine import Engine
    with Engine(model_path, **engine_options) as eng:
        return [_window_nll_engine(eng, w) for w in windows]


def eval_hf(hf_dir, windows: list) -> list:
    """Per-window mean NLL of the HF checkpoint in bf16 (float64 log-softmax of its logits)."""
    import torch
    from transformers import AutoModelForCausalLM
    model = AutoModelForCausalLM.from_pretrained(hf_dir, dtype=torch.bfloat16, attn_implementation="sdpa")
    model.to("cuda").eval()
    scores = []
    with torch.no_grad():
        for w in windows:
            seq = torch.tensor([[BOS_ID, *w]], dtype=torch.int64, device="cuda")
            logp = torch.log_softmax(model(seq).logits[0, :-1].to(torch.float64), dim=-1)
            picked = logp.gather(1, torch.tensor(w, device="cuda").unsqueeze(1))
            scores.append(float(-picked.mean().item()))
    return scores


def perplexity(window_nll: list) -> float:
    return math.exp(float(np.mean(window_nll)))


def _commit() -> str:
    r = subprocess.run(["git", "rev-parse", "--short", "HEAD"], capture_output=True, text=True,
                       cwd=Path(__file__).resolve().parents[1])
    return r.stdout.strip() if r.returncode == 0 else "unknown"


@dataclass
class PplRecord:
    """The JSON record the reference's tool writes (results/ppl/<target>_<dtype>.json)."""
    target: str
    dtype: str
    ppl: float
    n_tokens: int
    windows: int
    window_len: int
    window_mean_nll: list = field(default_factory=list)
    dataset: str = ""
    git_commit: str = ""
    tool: str = "eval_ppl"


def _args(argv):
    ap = argparse.ArgumentParser(description="perplexity over token windows")
    opts = [("--target", dict(choices=("engine", "hf"), required=True)),
            ("--dtype", dict(choices=("bf16", "int8", "int4"), default="bf16")),
            ("--windows", dict(type=int, default=40)), ("--window-len", dict(type=int, default=512)),
            ("--text-file", dict(type=Path)), ("--model", dict(type=Path)), ("--tokenizer", dict(type=Path)),
            ("--models-dir", dict(type=Path)), ("--out", dict(type=Path, default=Path("results/ppl")))]
    for flag, kw in opts:
        ap.add_argument(flag, **kw)
    args = ap.parse_args(argv)
    if args.target == "hf" and args.dtype != "bf16":
        ap.error("the HF target is scored in bf16 only")
    return args


def main(argv=None) -> int:
    args = _args(argv)
    from transformers import AutoTokenizer
    model, hf_dir = default_paths(args.models_dir, args.dtype)
    tok_dir = args.tokenizer or hf_dir
    text, dataset = load_text(args.text_file)
    windows = windows_from_ids(AutoTokenizer.from_pretrained(tok_dir)(text).input_ids, args.windows, args.window_len)
    nll = eval_engine(args.model or model, windows) if args.target == "engine" else eval_hf(tok_dir, windows)
    ppl = perplexity(nll)
    lo, hi = HF_PPL_RANGE
    if args.target == "hf" and not lo <= ppl <= hi:
        raise RuntimeError(f"the bf16 checkpoint scores PPL {ppl:.3f}, outside [{lo}, {hi}]: check the tokenizer and "
                           f"the window protocol")
    rec = PplRecord(target=args.target, dtype=args.dtype, ppl=ppl, n_tokens=len(windows) * args.window_len,
                    windows=len(windows), window_len=args.window_len, window_mean_nll=nll, dataset=dataset,
                    git_commit=_commit())
    print(f"{rec.target} {rec.dtype}: PPL {rec.ppl:.4f} over {rec.n_tokens} tokens")
    args.out.mkdir(parents=True, exist_ok=True)
    (args.out / f"{rec.target}_{rec.dtype}.json").write_text(json.dumps(asdict(rec), indent=2) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
