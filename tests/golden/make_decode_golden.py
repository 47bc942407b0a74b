"""Writes tests/golden/decode_tiny.npz: decode-step vectors from the REFERENCE's own CPU model.

Run in the build container only (the reference tree is not present on the GPU box):

    python tests/golden/make_decode_golden.py [/root/reference]

For each weight type it writes a tiny seeded model with ``oracle.synth`` (hidden 256, 2 layers,
4 query heads sharing 1 kv head, vocab 1000, head_dim 64, random norm weights), decodes a fixed
token sequence with ``cudallm.reference.ReferenceModel`` (``python/cudallm/reference.py:66-158``,
fp16 KV cache) and records the logits, the residual stream after the embedding and after each
layer, and the greedy continuation (``reference.py:160-171``).  The fixture holds only those
input ids, seeds and output arrays.  ``tests/test_oracle.py`` rebuilds the same model files and
checks ``oracle.model`` against them.
"""
import sys
import tempfile
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO))

from oracle import synth  # noqa: E402

SEED = 7
TOKENS = [3, 999, 0, 512, 77, 77, 250, 1]
N_GREEDY = 6


def main() -> None:
    ref_root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    sys.path.insert(0, str(ref_root / "python"))
    from cudallm.reference import ReferenceModel  # the reference's CPU model

    out = {"tokens": np.array(TOKENS, dtype=np.int32), "seed": np.array(SEED)}
    with tempfile.TemporaryDirectory() as d:
        for wd in ("bf16", "int8", "int4"):
            path = Path(d) / f"tiny_{wd}.cudallm"
            synth.write_model(path, wd, seed=SEED, dims=synth.TINY, norm="random")
            ref = ReferenceModel(path)
            logits, res = [], []
            for t in TOKENS:
                lg, r = ref.step(t)
                logits.append(lg.numpy())
                res.append(np.stack([v.numpy() for v in r]))
            out[f"{wd}_logits"] = np.stack(logits).astype(np.float32)
            out[f"{wd}_residuals"] = np.stack(res).astype(np.float32)
            out[f"{wd}_greedy"] = np.array(ref.greedy(TOKENS[:3], N_GREEDY), dtype=np.int32)
    np.savez_compressed(REPO / "tests/golden/decode_tiny.npz", **out)
    print("wrote", REPO / "tests/golden/decode_tiny.npz")


if __name__ == "__main__":
    main()
