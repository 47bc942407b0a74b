"""Perplexity of the engine, or of HF transformers, over fixed-length token windows (the reference's
bench/eval_ppl.py:1-92).

    python -m cudallm_amd.eval_ppl --target {engine,hf} [--dtype bf16|int8|int4] [--windows 40] [--window-len 512]
                                   [--text-file FILE] [--model FILE] [--tokenizer DIR] [--models-dir DIR] [--out DIR]

Same protocol as the reference: the text is tokenised once, a leading BOS is dropped, and it is cut into `windows`
windows of `window_len` tokens.  Per window the engine is reset, step(BOS) predicts w[0] and step(w[j]) predicts
w[j+1]; each negative log-likelihood is computed in float64 from the step's fp32 logits; PPL = exp(mean of the window
means).  The HF target runs the checkpoint in bf16 on [BOS] + window; its PPL must fall in the reference's sanity range.
The reference reads WikiText-2 (raw, test split) with `datasets`; that works here only where the dataset is already
in the local cache, so --text-file takes any local text instead.
"""
import argparse
import json
import math
import subprocess
import sys
from pathlib import Path

import numpy as np

from .generate import BOS_ID, default_paths

HF_PPL_RANGE = (6.0, 25.0)
WIKITEXT = ("Salesforce/wikitext", "wikitext-2-raw-v1", "test")


def nll_from_logits(logits: np.ndarray, target: int) -> float:
    """-log softmax(logits)[target] in float64 (eval_ppl.py:22-26)."""
    z = np.asarray(logits, dtype=np.float64)
    m = z.max()
    return float(m + math.log(np.exp(z - m).sum()) - z[target])


def windows_from_ids(ids: list, n_windows: int, window_len: int) -> list:
    """eval_ppl.py:29-36 after tokenisation: drop a leading BOS, then consecutive windows."""
    ids = list(ids)
    if ids and ids[0] == BOS_ID:
        ids = ids[1:]
    if len(ids) < n_windows * window_len:
        raise ValueError(f"only {len(ids)} tokens for {n_windows} windows of {window_len}")
    return [ids[k * window_len:(k + 1) * window_len] for k in range(n_windows)]


def load_text(text_file=None) -> tuple:
    """(text, dataset description): a local file, or WikiText-2 test joined by blank lines (eval_ppl.py:30-31)."""
    if text_file:
        return Path(text_file).read_text(encoding="utf-8"), f"file {Path(text_file).name}"
    from datasets import load_dataset
    ds = load_dataset(WIKITEXT[0], WIKITEXT[1], split=WIKITEXT[2])
    return "\n\n".join(ds["text"]), f"{WIKITEXT[0]} {WIKITEXT[1]} {WIKITEXT[2]}"


def eval_engine(model_path, windows: list, **engine_options) -> list:
    """Per-window mean NLL through the engine (eval_ppl.py:39-52)."""
    from .engine import Engine
    out = []
    with Engine(model_path, **engine_options) as eng:
        for w in windows:
            eng.reset()
            _, logits = eng.step(BOS_ID, want_logits=True)
            nll = [nll_from_logits(logits, w[0])]
            for j in range(len(w) - 1):
                _, logits = eng.step(w[j], want_logits=True)
                nll.append(nll_from_logits(logits, w[j + 1]))
            out.append(float(np.mean(nll)))
    return out


def eval_hf(hf_dir, windows: list) -> list:
    """Per-window mean NLL of the HF checkpoint in bf16 (eval_ppl.py:55-66)."""
    import torch
    from transformers import AutoModelForCausalLM
    model = AutoModelForCausalLM.from_pretrained(hf_dir, dtype=torch.bfloat16, attn_implementation="sdpa")
    model.to("cuda").eval()
    out = []
    with torch.no_grad():
        for w in windows:
            inp = torch.tensor([[BOS_ID] + list(w)], dtype=torch.int64, device="cuda")
            logits = model(inp).logits[0, :-1].to(torch.float64)
            nll = torch.nn.functional.cross_entropy(logits, torch.tensor(w, device="cuda"), reduction="none")
            out.append(float(nll.mean().item()))
    return out


def perplexity(window_nll: list) -> float:
    """Equal-length windows, so the mean of the window means is the mean over all tokens."""
    return math.exp(float(np.mean(window_nll)))


def _git_commit() -> str:
    try:
        return subprocess.run(["git", "rev-parse", "--short", "HEAD"], check=True, capture_output=True, text=True,
                              cwd=Path(__file__).resolve().parents[1]).stdout.strip()
    except (OSError, subprocess.CalledProcessError):
        return "unknown"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="perplexity over token windows")
    ap.add_argument("--target", choices=("engine", "hf"), required=True)
    ap.add_argument("--dtype", choices=("bf16", "int8", "int4"), default="bf16")
    ap.add_argument("--windows", type=int, default=40)
    ap.add_argument("--window-len", type=int, default=512)
    ap.add_argument("--text-file", type=Path)
    ap.add_argument("--model", type=Path)
    ap.add_argument("--tokenizer", type=Path)
    ap.add_argument("--models-dir", type=Path)
    ap.add_argument("--out", type=Path, default=Path("results/ppl"))
    args = ap.parse_args(argv)
    if args.target == "hf" and args.dtype != "bf16":
        raise SystemExit("HF perplexity is measured in bf16 only")

    from transformers import AutoTokenizer
    model, hf_dir = default_paths(args.models_dir, args.dtype)
    hf_dir = args.tokenizer or hf_dir
    tokenizer = AutoTokenizer.from_pretrained(hf_dir)
    text, dataset = load_text(args.text_file)
    windows = windows_from_ids(tokenizer(text).input_ids, args.windows, args.window_len)
    window_nll = eval_engine(args.model or model, windows) if args.target == "engine" else eval_hf(hf_dir, windows)
    ppl = perplexity(window_nll)
    if args.target == "hf" and not HF_PPL_RANGE[0] <= ppl <= HF_PPL_RANGE[1]:
        raise RuntimeError(f"HF bf16 PPL {ppl:.3f} outside sanity range {HF_PPL_RANGE}: tokenization/protocol bug?")
    n_tokens = len(windows) * args.window_len
    print(f"{args.target} {args.dtype}: PPL {ppl:.4f} over {n_tokens} tokens")
    args.out.mkdir(parents=True, exist_ok=True)
    (args.out / f"{args.target}_{args.dtype}.json").write_text(json.dumps({
        "tool": "eval_ppl", "target": args.target, "dtype": args.dtype, "ppl": ppl, "n_tokens": n_tokens,
        "windows": len(windows), "window_len": args.window_len, "window_mean_nll": window_nll, "dataset": dataset,
        "git_commit": _git_commit()}, indent=2) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
