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


# ---- the same quantizers on torch tensors (any device) --------------------------------------
# Used to build the large synthetic models on the GPU (the 7B configuration: 7.6e9 weights,
# minutes in numpy). Every step is the numpy quantizer's, op for op, in float32 with
# round-half-even (torch.round == np.rint) and float16 rounding (RNE in both), so on equal
# inputs the bytes are equal to quantize()'s.

def _t_inv(d):
    import torch
    return torch.where(d != 0, 1.0 / torch.where(d != 0, d, torch.ones_like(d)), torch.zeros_like(d))


def _t_f16_bytes(d16):
    import torch
    return d16.contiguous().view(torch.uint8).reshape(-1, 2)


def _t_q8_0(x):
    import torch
    b = x.reshape(-1, 32)
    d16 = (b.abs().amax(dim=1) / 127.0).half()
    q = torch.clamp(torch.round(b * _t_inv(d16.float())[:, None]), -127, 127).to(torch.int8)
    out = torch.empty(b.shape[0], 34, dtype=torch.uint8, device=x.device)
    out[:, 0:2] = _t_f16_bytes(d16)
    out[:, 2:] = q.view(torch.uint8)
    return out.reshape(-1)


def _t_q5_0(x):
    import torch
    b = x.reshape(-1, 32)
    idx = b.abs().argmax(dim=1)
    extreme = torch.gather(b, 1, idx[:, None])[:, 0]
    d16 = (extreme / -16.0).half()
    code = (torch.clamp(torch.round(b * _t_inv(d16.float())[:, None]) + 16, 0, 31)).to(torch.int64)
    qs = (code[:, :16] & 0xF) | ((code[:, 16:] & 0xF) << 4)
    qh = (((code >> 4) & 1) << torch.arange(32, device=x.device, dtype=torch.int64)).sum(dim=1)
    out = torch.empty(b.shape[0], 22, dtype=torch.uint8, device=x.device)
    out[:, 0:2] = _t_f16_bytes(d16)
    out[:, 2:6] = torch.stack([(qh >> (8 * i)) & 0xFF for i in range(4)], dim=1).to(torch.uint8)
    out[:, 6:22] = qs.to(torch.uint8)
    return out.reshape(-1)


def _t_pack_k4_scales(ls, lm):
    import torch
    s = torch.zeros(ls.shape[0], 12, dtype=torch.int64, device=ls.device)
    for j in range(4):
        s[:, j] = ls[:, j] & 63
        s[:, j + 4] = lm[:, j] & 63
    for j in range(4, 8):
        s[:, j + 4] = (ls[:, j] & 0xF) | ((lm[:, j] & 0xF) << 4)
        s[:, j - 4] |= (ls[:, j] >> 4) << 6
        s[:, j] |= (lm[:, j] >> 4) << 6
    return s.to(torch.uint8)


def _t_q4_k(x):
    import torch
    b = x.reshape(-1, 8, 32)
    nb = b.shape[0]
    lo = torch.clamp(b.amin(dim=2), max=0.0)
    hi = b.amax(dim=2)
    scale = (hi - lo) / 15.0
    mins = -lo
    d16 = (scale.amax(dim=1) / 63.0).half()
    dmin16 = (mins.amax(dim=1) / 63.0).half()
    d, dmin = d16.float(), dmin16.float()
    ls = torch.clamp(torch.round(scale * _t_inv(d)[:, None]), 0, 63).to(torch.int64)
    lm = torch.clamp(torch.round(mins * _t_inv(dmin)[:, None]), 0, 63).to(torch.int64)
    sc_eff = ls.float() * d[:, None]
    mn_eff = lm.float() * dmin[:, None]
    q = torch.clamp(torch.round((b + mn_eff[:, :, None]) * _t_inv(sc_eff)[:, :, None]), 0, 15).to(torch.uint8)
    out = torch.empty(nb, 144, dtype=torch.uint8, device=x.device)
    out[:, 0:2] = _t_f16_bytes(d16)
    out[:, 2:4] = _t_f16_bytes(dmin16)
    out[:, 4:16] = _t_pack_k4_scales(ls, lm)
    for c in range(4):
        out[:, 16 + 32 * c:48 + 32 * c] = q[:, 2 * c] | (q[:, 2 * c + 1] << 4)
    return out.reshape(-1)


def _t_q6_k(x):
    import torch
    b = x.reshape(-1, 16, 16)
    nb = b.shape[0]
    sub_scale = b.abs().amax(dim=2) / 32.0
    d16 = (sub_scale.amax(dim=1) / 127.0).half()
    d = d16.float()
    sc = torch.clamp(torch.round(sub_scale * _t_inv(d)[:, None]), -128, 127).to(torch.int8)
    eff = sc.float() * d[:, None]
    code = (torch.clamp(torch.round(b * _t_inv(eff)[:, :, None]), -32, 31) + 32).to(torch.uint8)
    code = code.reshape(nb, 256)
    out = torch.empty(nb, 210, dtype=torch.uint8, device=x.device)
    for h in range(2):
        c = code[:, 128 * h:128 * h + 128]
        q0, q1, q2, q3 = c[:, 0:32], c[:, 32:64], c[:, 64:96], c[:, 96:128]
        out[:, 64 * h:64 * h + 32] = (q0 & 0xF) | ((q2 & 0xF) << 4)
        out[:, 64 * h + 32:64 * h + 64] = (q1 & 0xF) | ((q3 & 0xF) << 4)
        out[:, 128 + 32 * h:160 + 32 * h] = (q0 >> 4) | ((q1 >> 4) << 2) | ((q2 >> 4) << 4) | ((q3 >> 4) << 6)
    out[:, 192:208] = sc.view(torch.uint8)
    out[:, 208:210] = _t_f16_bytes(d16)
    return out.reshape(-1)


def quantize_torch(ggml_type: int, x):
    """quantize() for a torch float32 tensor on any device -> flat uint8 tensor on that device."""
    import torch
    x = x.reshape(-1).to(torch.float32).contiguous()
    if ggml_type == GGML_F32:
        return x.view(torch.uint8).clone()
    if ggml_type == GGML_F16:
        return x.half().view(torch.uint8).clone()
    fn = {GGML_Q8_0: _t_q8_0, GGML_Q5_0: _t_q5_0, GGML_Q4_K: _t_q4_k, GGML_Q6_K: _t_q6_k}.get(ggml_type)
    if fn is None:
        raise NotImplementedError(f"quantize_torch: ggml type {ggml_type}")
    return fn(x)
