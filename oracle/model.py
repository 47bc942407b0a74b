"""One batch-1 decode step on the CPU, restated from the reference (test infrastructure only).

Follows ``python/cudallm/reference.py:66-171`` (itself the spec of ``src/engine/engine.cpp:181-237``):

    x = dequant(E[token])
    per layer:  xb = rmsnorm(x, attn_norm); qkv = Wqkv xb; q,k = rope(q,k); cache[pos] = fp16(k), fp16(v)
                att_h = softmax(0.125 * K_{h//g} q_h) V_{h//g};  x += Wo att
                xb = rmsnorm(x, ffn_norm); gu = Wgu xb; x += Wdown (silu(gu[:I]) * gu[I:])
    logits = E rmsnorm(x, final_norm)          (tied lm_head)

Arithmetic is torch float32 on the CPU with an fp16 KV cache, like the reference.  Weights stay in
their stored form and are dequantised to fp32 per matmul unless ``cache_dense`` is set, which keeps
the dense fp32 copies (same values, faster repeated steps, ~4x the file size in memory).
"""
import os

import numpy as np
import torch

from . import fileformat as ff


class _Linear:
    def __init__(self, path, w: dict, s: dict | None, cache_dense: bool):
        self.dtype, self.rows, self.cols = w["dtype"], w["rows"], w["cols"]
        raw = np.asarray(ff.load(path, w))
        if self.dtype == ff.BF16:
            self.w = torch.from_numpy(raw.view(np.int16).copy()).view(torch.bfloat16)
            self.s = None
        elif self.dtype == ff.I8:
            self.w = torch.from_numpy(raw.copy())
            self.s = torch.from_numpy(np.asarray(ff.load(path, s), dtype=np.float32).copy())
        elif self.dtype == ff.I4X2:
            self.w = torch.from_numpy(raw.copy())
            self.s = torch.from_numpy(np.asarray(ff.load(path, s)).copy())
        else:
            raise ValueError(f"unsupported linear dtype {self.dtype}")
        self._dense = self._dequant(self.w, self.s) if cache_dense else None

    def _dequant(self, w: torch.Tensor, s) -> torch.Tensor:
        if self.dtype == ff.BF16:
            return w.float()
        if self.dtype == ff.I8:
            return w.float() * s[:, None]
        rows = w.shape[0]
        q = torch.empty((rows, self.cols), dtype=torch.float32)
        q[:, 0::2] = (w & 0x0F).float() - 8.0
        q[:, 1::2] = (w >> 4).float() - 8.0
        ng = s.shape[1]
        return (q.view(rows, ng, self.cols // ng) * s.float()[:, :, None]).view(rows, self.cols)

    def dense(self) -> torch.Tensor:
        return self._dense if self._dense is not None else self._dequant(self.w, self.s)

    def row(self, r: int) -> torch.Tensor:
        return self._dequant(self.w[r:r + 1], None if self.s is None else self.s[r:r + 1])[0]

    def __matmul__(self, x: torch.Tensor) -> torch.Tensor:
        return self.dense() @ x


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    return x * torch.rsqrt(torch.mean(x * x) + eps) * w


def silu(g: torch.Tensor) -> torch.Tensor:
    return g / (1.0 + torch.exp(-g))


class OracleModel:
    """CPU decode of a ``.cudallm`` file (any dimensions whose head_dim is 64)."""

    def __init__(self, path, cache_dense: bool = False, threads: int | None = None):
        torch.set_num_threads(threads or os.cpu_count())
        self.path = str(path)
        h = ff.read_header(path)
        self.hidden, self.inter, self.n_layers = h["hidden_size"], h["intermediate_size"], h["n_layers"]
        self.n_heads, self.n_kv, self.head_dim = h["n_heads"], h["n_kv_heads"], h["head_dim"]
        self.vocab, self.max_seq, self.eps = h["vocab_size"], h["max_seq_len"], h["rms_eps"]
        quant = h["weight_dtype"] != ff.WEIGHT_BF16
        table = {e["name"]: e for e in ff.read_table(path)}
        if list(table) != ff.tensor_names(self.n_layers, quant):
            raise ValueError("unexpected tensor names or order")

        def lin(n):
            return _Linear(path, table[n + ".weight"], table.get(n + ".scales"), cache_dense)

        def vec(n):
            return torch.from_numpy(np.asarray(ff.load(path, table[n]), dtype=np.float32).copy())

        self.inv_freq = vec("rope.inv_freq")
        self.emb = lin("tok_embeddings")
        self.final_norm = vec("norm.weight")
        self.layers = []
        for i in range(self.n_layers):
            p = f"layers.{i}."
            self.layers.append(dict(attn_norm=vec(p + "attn_norm.weight"), wqkv=lin(p + "wqkv"), wo=lin(p + "wo"),
                                    ffn_norm=vec(p + "ffn_norm.weight"), w_gate_up=lin(p + "w_gate_up"),
                                    w_down=lin(p + "w_down")))
        shape = (self.n_kv, self.max_seq, self.head_dim)
        self.k_cache = [torch.zeros(shape, dtype=torch.float16) for _ in range(self.n_layers)]
        self.v_cache = [torch.zeros(shape, dtype=torch.float16) for _ in range(self.n_layers)]
        self.pos = 0

    def reset(self) -> None:
        self.pos = 0

    def _rope(self, v: torch.Tensor) -> torch.Tensor:
        half = self.head_dim // 2
        ang = torch.tensor(float(self.pos), dtype=torch.float32) * self.inv_freq
        c, s = torch.cos(ang), torch.sin(ang)
        a, b = v[:, :half], v[:, half:]
        return torch.cat([a * c - b * s, b * c + a * s], dim=1)

    @torch.no_grad()
    def step(self, token: int) -> tuple[torch.Tensor, list[torch.Tensor]]:
        """Decode ``token`` at ``self.pos``; returns (logits fp32 [V], residuals [L+1] x fp32 [H])."""
        if self.pos >= self.max_seq:
            raise RuntimeError("sequence is full")
        NH, KV, D, pos = self.n_heads, self.n_kv, self.head_dim, self.pos
        g = NH // KV
        x = self.emb.row(int(token)).clone()
        res = [x.clone()]
        for li, L in enumerate(self.layers):
            qkv = L["wqkv"] @ rmsnorm(x, L["attn_norm"], self.eps)
            q = self._rope(qkv[:NH * D].view(NH, D))
            k = self._rope(qkv[NH * D:(NH + KV) * D].view(KV, D))
            v = qkv[(NH + KV) * D:].view(KV, D)
            self.k_cache[li][:, pos] = k.to(torch.float16)
            self.v_cache[li][:, pos] = v.to(torch.float16)
            K = self.k_cache[li][:, :pos + 1].float()
            V = self.v_cache[li][:, :pos + 1].float()
            att = torch.empty(NH, D, dtype=torch.float32)
            for h in range(NH):
                s = (K[h // g] @ q[h]) * 0.125
                p = torch.exp(s - s.max())
                att[h] = (p / p.sum()) @ V[h // g]
            x = x + L["wo"] @ att.view(-1)
            gu = L["w_gate_up"] @ rmsnorm(x, L["ffn_norm"], self.eps)
            x = x + L["w_down"] @ (silu(gu[:self.inter]) * gu[self.inter:])
            res.append(x.clone())
        logits = self.emb @ rmsnorm(x, self.final_norm, self.eps)
        self.pos += 1
        return logits, res

    def greedy(self, prompt: list[int], n_new: int) -> list[int]:
        """``python/cudallm/reference.py:160-171``."""
        self.reset()
        logits = None
        for t in prompt:
            logits, _ = self.step(t)
        out: list[int] = []
        while len(out) < n_new:
            out.append(int(torch.argmax(logits)))
            if len(out) < n_new:
                logits, _ = self.step(out[-1])
        return out
