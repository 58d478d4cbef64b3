"""Host-side fp32 -> GGUF block quantizers (model preparation, not on the decode path).

Used to build the seeded synthetic GGUF models the benchmarks and parity tests run on. The
block layouts are the GGML ones the reference decodes (dequant.py:51-232); the choice of
scales is this file's own simple rule (absmax for Q8_0/Q5_0/Q6_K, min/max per sub-block for
Q4_K), not llama.cpp's search -- the produced file is the input of both the GPU path and the
CPU oracle, so only the layout has to be standard. Everything is vectorised numpy and
deterministic for a given input array.
"""

from __future__ import annotations

import numpy as np

from .dequant import GGML_F16, GGML_F32, GGML_Q4_K, GGML_Q5_0, GGML_Q6_K, GGML_Q8_0


def _f16(a: np.ndarray) -> np.ndarray:
    return a.astype(np.float16)


def _safe_inv(d: np.ndarray) -> np.ndarray:
    out = np.zeros_like(d, dtype=np.float32)
    nz = d != 0
    out[nz] = 1.0 / d[nz]
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """(n,) f32 -> Q8_0 blocks: d = absmax/127, q = round(x/d)."""
    b = x.reshape(-1, 32).astype(np.float32)
    d16 = _f16(np.abs(b).max(axis=1) / 127.0)
    q = np.clip(np.rint(b * _safe_inv(d16.astype(np.float32))[:, None]), -127, 127).astype(np.int8)
    out = np.empty((b.shape[0], 34), dtype=np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def quantize_q5_0(x: np.ndarray) -> np.ndarray:
    """(n,) f32 -> Q5_0 blocks: d = -(signed absmax)/16, code = clip(round(x/d)+16, 0, 31)."""
    b = x.reshape(-1, 32).astype(np.float32)
    idx = np.abs(b).argmax(axis=1)
    extreme = b[np.arange(b.shape[0]), idx]
    d16 = _f16(extreme / -16.0)
    code = np.clip(np.rint(b * _safe_inv(d16.astype(np.float32))[:, None]) + 16, 0, 31).astype(np.uint32)
    qs = (code[:, :16] & 0xF) | ((code[:, 16:] & 0xF) << 4)
    qh = ((code >> 4) & 1) << np.arange(32, dtype=np.uint32)
    qh = qh.sum(axis=1, dtype=np.uint64).astype(np.uint32)
    out = np.empty((b.shape[0], 22), dtype=np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:6] = qh.astype("<u4").view(np.uint8).reshape(-1, 4)
    out[:, 6:22] = qs.astype(np.uint8)
    return out.reshape(-1)


def pack_k4_scales(ls: np.ndarray, lm: np.ndarray) -> np.ndarray:
    """(nb,8) 6-bit scales and mins -> (nb,12) packed bytes, inverse of the unpacking in
    dequant.py:171-179 (j<4: low 6 bits of bytes j / j+4; j>=4: nibbles of byte j+4 and the
    top 2 bits of bytes j-4 / j)."""
    ls = ls.astype(np.uint32)
    lm = lm.astype(np.uint32)
    s = np.zeros((ls.shape[0], 12), dtype=np.uint32)
    for j in range(4):
        s[:, j] = ls[:, j] & 63
        s[:, j + 4] = lm[:, j] & 63
    for j in range(4, 8):
        s[:, j + 4] = (ls[:, j] & 0xF) | ((lm[:, j] & 0xF) << 4)
        s[:, j - 4] |= (ls[:, j] >> 4) << 6
        s[:, j] |= (lm[:, j] >> 4) << 6
    return s.astype(np.uint8)


def quantize_q4_k(x: np.ndarray) -> np.ndarray:
    """(n,) f32 -> Q4_K: per 32-sub-block affine (scale, -min), 6-bit scale/min codes."""
    b = x.reshape(-1, 8, 32).astype(np.float32)
    nb = b.shape[0]
    lo = np.minimum(b.min(axis=2), 0.0)
    hi = b.max(axis=2)
    scale = (hi - lo) / 15.0
    mins = -lo
    d16 = _f16(scale.max(axis=1) / 63.0)
    dmin16 = _f16(mins.max(axis=1) / 63.0)
    d = d16.astype(np.float32)
    dmin = dmin16.astype(np.float32)
    ls = np.clip(np.rint(scale * _safe_inv(d)[:, None]), 0, 63).astype(np.int32)
    lm = np.clip(np.rint(mins * _safe_inv(dmin)[:, None]), 0, 63).astype(np.int32)
    sc_eff = ls.astype(np.float32) * d[:, None]
    mn_eff = lm.astype(np.float32) * dmin[:, None]
    q = np.clip(np.rint((b + mn_eff[:, :, None]) * _safe_inv(sc_eff)[:, :, None]), 0, 15).astype(np.uint8)
    out = np.empty((nb, 144), dtype=np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = dmin16.view(np.uint8).reshape(-1, 2)
    out[:, 4:16] = pack_k4_scales(ls, lm)
    qs = np.empty((nb, 128), dtype=np.uint8)
    for c in range(4):  # chunk c: low nibble = sub-block 2c, high nibble = sub-block 2c+1
        qs[:, 32 * c:32 * c + 32] = q[:, 2 * c] | (q[:, 2 * c + 1] << 4)
    out[:, 16:] = qs
    return out.reshape(-1)


def quantize_q6_k(x: np.ndarray) -> np.ndarray:
    """(n,) f32 -> Q6_K: per 16-sub-block int8 scale (x d), 6-bit codes in -32..31."""
    b = x.reshape(-1, 16, 16).astype(np.float32)
    nb = b.shape[0]
    sub_scale = np.abs(b).max(axis=2) / 32.0                   # (nb,16) >= 0
    d16 = _f16(sub_scale.max(axis=1) / 127.0)
    d = d16.astype(np.float32)
    sc = np.clip(np.rint(sub_scale * _safe_inv(d)[:, None]), -128, 127).astype(np.int8)
    eff = sc.astype(np.float32) * d[:, None]
    code = (np.clip(np.rint(b * _safe_inv(eff)[:, :, None]), -32, 31) + 32).astype(np.uint8)
    code = code.reshape(nb, 256)
    ql = np.zeros((nb, 128), dtype=np.uint8)
    qh = np.zeros((nb, 64), dtype=np.uint8)
    for h in range(2):
        c = code[:, 128 * h:128 * h + 128]
        q0, q1, q2, q3 = c[:, 0:32], c[:, 32:64], c[:, 64:96], c[:, 96:128]
        ql[:, 64 * h:64 * h + 32] = (q0 & 0xF) | ((q2 & 0xF) << 4)
        ql[:, 64 * h + 32:64 * h + 64] = (q1 & 0xF) | ((q3 & 0xF) << 4)
        qh[:, 32 * h:32 * h + 32] = (q0 >> 4) | ((q1 >> 4) << 2) | ((q2 >> 4) << 4) | ((q3 >> 4) << 6)
    out = np.empty((nb, 210), dtype=np.uint8)
    out[:, 0:128] = ql
    out[:, 128:192] = qh
    out[:, 192:208] = sc.view(np.uint8)
    out[:, 208:210] = d16.view(np.uint8).reshape(-1, 2)
    return out.reshape(-1)


def quantize(ggml_type: int, x: np.ndarray) -> np.ndarray:
    """Quantize a flat f32 array (row-major, rows contiguous) to raw GGUF bytes."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    if ggml_type == GGML_F32:
        return x.view(np.uint8).copy()
    if ggml_type == GGML_F16:
        return x.astype(np.float16).view(np.uint8).copy()
    fn = {GGML_Q8_0: quantize_q8_0, GGML_Q5_0: quantize_q5_0,
          GGML_Q4_K: quantize_q4_k, GGML_Q6_K: quantize_q6_k}.get(ggml_type)
    if fn is None:
        raise NotImplementedError(f"quantize: ggml type {ggml_type}")
    return fn(x)
