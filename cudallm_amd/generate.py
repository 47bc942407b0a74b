"""Greedy text generation through the engine (the reference's python/cudallm/generate.py:1-57).

    python -m cudallm_amd.generate --prompt TEXT [--dtype bf16|int8|int4] [--max-new-tokens 128] [--no-chat]
                                   [--matvec opt|naive] [--attn opt|naive] [--no-fuse] [--no-graph]
                                   [--model FILE] [--tokenizer DIR] [--models-dir DIR]

Same options, stopping rule (the Llama-3 end-of-turn ids) and output as the reference: the prompt (as a one-turn chat
unless --no-chat) is fed token by token, then the argmax is fed back until an end id or --max-new-tokens, and the text
is printed as it grows, followed by ``[prompt_tokens=.. generated=.. decode_tok_s=..]``.  The reference finds its
files at fixed places under its repository (python/cudallm/paths.py); here they are arguments, defaulting to the same
names under --models-dir ($CUDALLM_MODELS or ./models): llama-3.2-1b-instruct.{dtype}.cudallm and
hf/Llama-3.2-1B-Instruct (a Hugging Face directory with the tokenizer files).
"""
import argparse
import os
import sys
import time
from pathlib import Path

BOS_ID = 128000
EOS_IDS = (128001, 128008, 128009)


def default_paths(models_dir=None, dtype: str = "bf16") -> tuple:
    """(model file, tokenizer directory) in the reference's layout (python/cudallm/paths.py:6-10)."""
    d = Path(models_dir or os.environ.get("CUDALLM_MODELS", "models"))
    return d / f"llama-3.2-1b-instruct.{dtype}.cudallm", d / "hf" / "Llama-3.2-1B-Instruct"


def prompt_ids(tokenizer, prompt: str, chat: bool = True) -> list:
    """generate.py:29-32: a one-turn chat with the generation prompt, or the plain tokenisation.  return_dict=False
    keeps the reference's list of ids on transformers 5, whose default became a BatchEncoding."""
    if not chat:
        return list(tokenizer(prompt).input_ids)
    return list(tokenizer.apply_chat_template([{"role": "user", "content": prompt}], add_generation_prompt=True,
                                              return_dict=False))


def generate(eng, tokenizer, ids: list, max_new_tokens: int, out=None) -> tuple:
    """Feed `ids`, then decode greedily until an end id or `max_new_tokens` (generate.py:34-53).  Writes the text
    as it grows to `out` (decoding the whole continuation each time, so multi-token characters print whole).
    Returns (generated ids, decode seconds)."""
    nxt = None
    for t in ids:
        nxt, _ = eng.step(t)
    generated, printed = [], ""
    t0 = time.perf_counter()
    while True:
        if nxt in EOS_IDS:
            break
        generated.append(nxt)
        text = tokenizer.decode(generated)
        if out is not None:
            out.write(text[len(printed):])
            out.flush()
        printed = text
        if len(generated) >= max_new_tokens:
            break
        nxt, _ = eng.step(None)
    return generated, time.perf_counter() - t0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Greedy generation with the MI355X cudallm engine")
    ap.add_argument("--prompt", required=True)
    ap.add_argument("--dtype", choices=("bf16", "int8", "int4"), default="bf16")
    ap.add_argument("--max-new-tokens", type=int, default=128)
    ap.add_argument("--no-chat", action="store_true")
    ap.add_argument("--matvec", choices=("opt", "naive"), default="opt")
    ap.add_argument("--attn", choices=("opt", "naive"), default="opt")
    ap.add_argument("--no-fuse", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--model", type=Path, help="the .cudallm file (default: from --models-dir and --dtype)")
    ap.add_argument("--tokenizer", type=Path, help="tokenizer directory (default: <models-dir>/hf/Llama-3.2-1B-Instruct)")
    ap.add_argument("--models-dir", type=Path)
    args = ap.parse_args(argv)

    from transformers import AutoTokenizer
    from .engine import Engine
    model, tok_dir = default_paths(args.models_dir, args.dtype)
    tokenizer = AutoTokenizer.from_pretrained(args.tokenizer or tok_dir)
    ids = prompt_ids(tokenizer, args.prompt, chat=not args.no_chat)
    with Engine(args.model or model, matvec=args.matvec, attn=args.attn, fuse=not args.no_fuse,
                cuda_graph=not args.no_graph) as eng:
        generated, elapsed = generate(eng, tokenizer, ids, args.max_new_tokens, sys.stdout)
    tok_s = len(generated) / elapsed if elapsed > 0 else 0.0
    print(f"\n[prompt_tokens={len(ids)} generated={len(generated)} decode_tok_s={tok_s:.2f}]")
    return 0


if __name__ == "__main__":
    sys.exit(main())
