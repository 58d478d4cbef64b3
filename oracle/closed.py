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
                  tensors, looping over heads and positions (pins ref_cpu's composition);
                  ``fp16=True`` rounds where the reference's CUDA autocast prefill holds fp16
                  (pins ref_cpu's autocast mode).
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


def round16(a):
    """Round to fp16 (nearest even) and back."""
    return np.asarray(a, np.float64).astype(np.float16).astype(np.float64)


def causal_attention_f16(q, k, v, scale=None):
    """Causal attention as an fp16 flash-attention kernel forms it: per query l and head h,
    p = exp(s - max s) over positions <= l, output = (round16(p) V) / sum p, rounded to fp16.
    q (L, Hq, hd); k, v (Hkv, L, hd)."""
    q = np.asarray(q, np.float64)
    L, Hq, hd = q.shape
    g = Hq // k.shape[0]
    scale = hd ** -0.5 if scale is None else scale
    out = np.empty((L, Hq, hd))
    for l in range(L):
        for h in range(Hq):
            s = (np.asarray(k[h // g, :l + 1], np.float64) @ q[l, h]) * scale
            p = np.exp(s - s.max())
            out[l, h] = (round16(p) @ np.asarray(v[h // g, :l + 1], np.float64)) / p.sum()
    return round16(out)


def forward64(weights: dict, cfg, ids, cos, sin, fp16: bool = False, head_fp16: bool = False,
              return_hidden: bool = False):
    """Whole-model float64 forward over ``ids`` (prefill then nothing else), plain loops.

    ``weights``: name -> float64 array in logical (rows, cols) shape (dequantized GGUF tensors);
    returns the logits of the last position. ``fp16``: every value rounded to fp16 where the
    reference's CUDA prefill under fp16 autocast holds fp16 (model.py:147-151): the matrices
    and biases of each product, every product's result, the normed activations, RoPE output,
    attention (causal_attention_f16), SiLU product and the residual stream from the first
    o-projection on; ``head_fp16``: the LM head is an fp16 matmul too (an unquantized head),
    else it multiplies the fp16 normed vector in full precision (the Q8_0 GEMV).
    ``return_hidden``: (logits, the normed last row the LM head multiplies).
    """
    H, hd, nh, nkv = cfg.hidden, cfg.head_dim, cfg.n_head, cfg.n_kv
    L = len(ids)
    R = round16 if fp16 else (lambda a: a)
    W = lambda name: R(weights[name])
    x = np.stack([weights["token_embd.weight"][i] for i in ids]).astype(np.float64)
    for layer in range(cfg.n_layers):
        p = f"blk.{layer}."
        h = R(rmsnorm(x, weights[p + "attn_norm.weight"], cfg.eps))
        q = R(h @ W(p + "attn_q.weight").T + W(p + "attn_q.bias"))
        k = R(h @ W(p + "attn_k.weight").T + W(p + "attn_k.bias"))
        v = R(h @ W(p + "attn_v.weight").T + W(p + "attn_v.bias"))
        q = q.reshape(L, nh, hd)
        k = k.reshape(L, nkv, hd)
        v = v.reshape(L, nkv, hd)
        c = cos[:L][:, None, :]
        s = sin[:L][:, None, :]
        q = R(rope(q, c, s))
        k = R(rope(k, c, s))
        kc = np.transpose(k, (1, 0, 2))
        vc = np.transpose(v, (1, 0, 2))
        att = (causal_attention_f16(q, kc, vc) if fp16 else causal_attention(q, kc, vc)).reshape(L, nh * hd)
        x = R(R(x) + att @ W(p + "attn_output.weight").T)
        h = R(rmsnorm(x, weights[p + "ffn_norm.weight"], cfg.eps))
        g = R(h @ W(p + "ffn_gate.weight").T)
        u = R(h @ W(p + "ffn_up.weight").T)
        x = R(x + R(silu_mul(g, u)) @ W(p + "ffn_down.weight").T)
    h = R(rmsnorm(x[-1], weights["output_norm.weight"], cfg.eps))
    head = weights.get("output.weight", weights["token_embd.weight"])
    logits = R(R(head) @ h) if fp16 and head_fp16 else head @ h
    return (logits, h) if return_hidden else logits
