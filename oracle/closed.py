"""float64 closed forms (test infrastructure only).

Independent, unfactored definitions in numpy float64 -- no int8/scale factoring, no online
softmax -- used to pin oracle/ref_cpu.py and the HIP kernels:

* ``gemv``        y = W x (+ b) (+ r) with W the exact dequantized weights
* ``rmsnorm``     x / sqrt(mean(x^2) + eps) * w                       (kernels.py:21-23)
* ``rope``        rotate-half on pairs (j, j + hd/2)                   (kernels.py:44-47)
* ``silu_mul``    g * sigmoid(g) * u                                   (kernels.py:73)
* ``attention``   softmax(q K^T * scale) V over positions < S, GQA head h -> kv h // group,
                  optional fp16 rounding of the output                 (kernels.py:98-126)
* ``causal_attention``  the prefill form (model.py:201-209)
* ``forward64``   an independent float64 forward of the whole dense model from the GGUF
                  tensors, looping over heads and positions (pins ref_cpu's composition).
"""

from __future__ import annotations

import numpy as np


def gemv(W, x, bias=None, residual=None):
    y = np.asarray(W, np.float64) @ np.asarray(x, np.float64)
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    if residual is not None:
        y = y + np.asarray(residual, np.float64)
    return y


def rmsnorm(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(w, np.float64)


def rope(x, cos, sin):
    """x (..., hd); cos/sin broadcastable to (..., hd/2)."""
    x = np.asarray(x, np.float64)
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    return np.concatenate([x1 * cos - x2 * sin, x1 * sin + x2 * cos], axis=-1)


def silu_mul(g, u):
    g = np.asarray(g, np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(u, np.float64)


def attention(q, k, v, S, scale=None, round_fp16=False):
    """q (Hq, hd); k, v (Hkv, cap, hd); positions < S valid."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    Hq, hd = q.shape
    Hkv = k.shape[0]
    g = Hq // Hkv
    scale = hd ** -0.5 if scale is None else scale
    out = np.empty((Hq, hd))
    for h in range(Hq):
        kv = h // g
        s = (k[kv, :S] @ q[h]) * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v[kv, :S]
    if round_fp16:
        out = out.astype(np.float16).astype(np.float64)
    return out


def causal_attention(q, k, v, pos0=0, scale=None):
    """q (L, Hq, hd) at positions pos0..; k, v (Hkv, cap, hd) -> (L, Hq, hd)."""
    q = np.asarray(q, np.float64)
    L, Hq, hd = q.shape
    out = np.empty((L, Hq, hd))
    for l in range(L):
        out[l] = attention(q[l], k, v, pos0 + l + 1, scale)
    return out


def forward64(weights: dict, cfg, ids, cos, sin):
    """Whole-model float64 forward over ``ids`` (prefill then nothing else), plain loops.

    ``weights``: name -> float64 array in logical (rows, cols) shape (dequantized GGUF tensors);
    returns the logits of the last position.
    """
    H, hd, nh, nkv = cfg.hidden, cfg.head_dim, cfg.n_head, cfg.n_kv
    L = len(ids)
    x = np.stack([weights["token_embd.weight"][i] for i in ids]).astype(np.float64)
    for layer in range(cfg.n_layers):
        p = f"blk.{layer}."
        h = rmsnorm(x, weights[p + "attn_norm.weight"], cfg.eps)
        q = h @ weights[p + "attn_q.weight"].T + weights[p + "attn_q.bias"]
        k = h @ weights[p + "attn_k.weight"].T + weights[p + "attn_k.bias"]
        v = h @ weights[p + "attn_v.weight"].T + weights[p + "attn_v.bias"]
        q = q.reshape(L, nh, hd)
        k = k.reshape(L, nkv, hd)
        v = v.reshape(L, nkv, hd)
        c = cos[:L][:, None, :]
        s = sin[:L][:, None, :]
        q = rope(q, c, s)
        k = rope(k, c, s)
        kc = np.transpose(k, (1, 0, 2))
        vc = np.transpose(v, (1, 0, 2))
        att = causal_attention(q, kc, vc).reshape(L, nh * hd)
        x = x + att @ weights[p + "attn_output.weight"].T
        h = rmsnorm(x, weights[p + "ffn_norm.weight"], cfg.eps)
        g = h @ weights[p + "ffn_gate.weight"].T
        u = h @ weights[p + "ffn_up.weight"].T
        x = x + silu_mul(g, u) @ weights[p + "ffn_down.weight"].T
    h = rmsnorm(x[-1], weights["output_norm.weight"], cfg.eps)
    return weights["output.weight"] @ h
