"""float64 closed forms of the single-kernel operations (test infrastructure only).

These restate the numpy references of the reference's kernel tests
(``tests/test_kernels.py:19-207``) and the semantics of the kernels they test:

* matvec with fused RMSNorm prologue and STORE/ADD/SWIGLU epilogue
  (``src/kernels/matvec_opt.cu:129-156``; ``tests/test_kernels.py:53-96``)
* RMSNorm (``src/kernels/rmsnorm.cu:12-20``; ``tests/test_kernels.py:101-109``)
* RoPE + fp16 KV write (``src/kernels/rope_kv.cu:44-79``; ``tests/test_kernels.py:117-163``)
* decode attention with scale 1/8 (``src/kernels/attention_opt.cu:17-134``;
  ``tests/test_kernels.py:168-196``)
* silu(g)*u (``src/kernels/common.cuh:43``; ``tests/test_kernels.py:201-207``)
* argmax with ties to the lowest index (``src/kernels/argmax.cu:12-15``)
* the Llama-3 scaled RoPE inverse frequencies (``tests/test_kernels.py:29-38``,
  parameters from ``python/cudallm/export.py:35-41``)
"""
import numpy as np


def llama3_inv_freq(head_dim: int = 64, theta: float = 500000.0, factor: float = 32.0, low: float = 1.0,
                    high: float = 4.0, orig: int = 8192) -> np.ndarray:
    """Llama-3 frequency scaling, computed in float64 and stored as fp32."""
    i = np.arange(head_dim // 2, dtype=np.float64)
    base = 1.0 / theta ** (2 * i / head_dim)
    wavelen = 2 * np.pi / base
    smooth = (orig / wavelen - low) / (high - low)
    mid = (1 - smooth) * base / factor + smooth * base
    out = np.where(wavelen < orig / high, base, np.where(wavelen > orig / low, base / factor, mid))
    return out.astype(np.float32)


def rms_normalize(x, w, eps: float) -> np.ndarray:
    x64 = np.asarray(x, dtype=np.float64)
    return x64 / np.sqrt(np.mean(x64 * x64) + eps) * np.asarray(w, dtype=np.float64)


def silu(g):
    return g / (1.0 + np.exp(-g))


def matvec(w64: np.ndarray, x, epilogue: str = "store", norm_w=None, eps: float = 1e-5, y_init=None) -> np.ndarray:
    """``w64`` is the exact dequantised weight in float64, shape [rows, cols]."""
    x64 = np.asarray(x, dtype=np.float64)
    if norm_w is not None:
        x64 = rms_normalize(x64, norm_w, eps)
    d = w64 @ x64
    if epilogue == "swiglu":
        h = d.shape[0] // 2
        return silu(d[:h]) * d[h:]
    if epilogue == "add":
        return np.asarray(y_init, dtype=np.float64) + d
    return d


def rope(v64: np.ndarray, inv_freq: np.ndarray, pos: int) -> np.ndarray:
    """Rotate pairs (i, i+hd/2) by the fp32 angle fp32(pos)*inv_freq[i]; rotation in float64."""
    ang = (np.float32(pos) * np.asarray(inv_freq, dtype=np.float32)).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    half = v64.shape[-1] // 2
    a, b = v64[..., :half], v64[..., half:]
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)


def rope_kv(qkv, inv_freq, pos: int, k_cache, v_cache, nh: int, nkv: int, hd: int):
    """Expected outputs of the rope_kv hook.

    Returns (q_rot float64 [nh, hd], k_rot float64 [nkv, hd], k_cache fp16, v_cache fp16): the
    caches are the inputs with row ``pos`` of every kv head replaced by fp16(k_rot) and fp16(v).
    """
    qkv = np.asarray(qkv, dtype=np.float32)
    q = rope(qkv[:nh * hd].astype(np.float64).reshape(nh, hd), inv_freq, pos)
    k = rope(qkv[nh * hd:(nh + nkv) * hd].astype(np.float64).reshape(nkv, hd), inv_freq, pos)
    v = qkv[(nh + nkv) * hd:].reshape(nkv, hd)
    kc = np.array(k_cache, dtype=np.float16, copy=True)
    vc = np.array(v_cache, dtype=np.float16, copy=True)
    kc[:, pos, :] = k.astype(np.float16)
    vc[:, pos, :] = v.astype(np.float16)
    return q, k, kc, vc


def attention(q, k_cache, v_cache, ctx: int, nh: int, nkv: int, hd: int, scale: float = 0.125) -> np.ndarray:
    """softmax(scale * K q) V per query head, kv head = h // (nh/nkv), over tokens [0, ctx)."""
    q64 = np.asarray(q, dtype=np.float64).reshape(nh, hd)
    k64 = np.asarray(k_cache[:, :ctx], dtype=np.float64)
    v64 = np.asarray(v_cache[:, :ctx], dtype=np.float64)
    out = np.empty((nh, hd))
    g = nh // nkv
    for h in range(nh):
        s = (k64[h // g] @ q64[h]) * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v64[h // g]
    return out.reshape(-1)


def silu_mul(gu) -> np.ndarray:
    gu64 = np.asarray(gu, dtype=np.float64)
    h = gu64.size // 2
    return silu(gu64[:h]) * gu64[h:]


def argmax_lowest(v) -> int:
    """First index of the maximum (numpy's tie rule, which the reference kernel matches)."""
    return int(np.argmax(np.asarray(v)))
