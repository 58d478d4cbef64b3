"""numpy restatement of the reference's GGML block decode (test infrastructure only).

Restates ``src/pico_engine/dequant.py`` of the reference:

* ``nbytes_for``                 -- dequant.py:27-48
* ``dequantize`` / per-format    -- dequant.py:51-76 (Q5_0, Q8_0), :182-201 (Q4_K),
                                    :204-232 (Q6_K), :235-240 (Q8_K), :243-260 (dispatch)
* ``scale_min_k4``               -- dequant.py:171-179
* ``unpack_q5_0/q8_0/q6_k/q4_k`` -- dequant.py:79-168 (the int8 + fp32-scale form the
                                    reference's Triton GEMVs read)

Pinned by: the reference's known-answer blocks (tests/test_dequant.py:21-72,
restated as fixtures in tests/golden/dequant_known_answers.json), hand-computed
bit-level blocks for the paths those leave open (Q4_K sub-blocks j>=4, Q6_K with
non-zero qh and mixed-sign scales, negative Q8_0 scales, fp16-subnormal scales),
an independent C restatement (oracle/dequant_ref.c) compared bit for bit on
random blocks, exhaustive sweeps of every code value, and the identity
unpack-form == dequant-form. See tests/test_oracle_dequant.py.

Block layouts (little-endian, one row = K/QK consecutive blocks):
  Q8_0 34 B : d f16 | qs i8[32]                    w = d*qs
  Q5_0 22 B : d f16 | qh u32 | qs u8[16]           w = d*(q5 - 16)
  Q4_K 144 B: d f16 | dmin f16 | scales u8[12] | qs u8[128]
  Q6_K 210 B: ql u8[128] | qh u8[64] | scales i8[16] | d f16   (d is LAST)
  Q8_K 292 B: d f32 | qs i8[256] | bsums i16[16]
"""

from __future__ import annotations

import numpy as np

F32, F16, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K = 0, 1, 6, 8, 12, 13, 14, 15

# (elements per block, bytes per block)
BLOCK = {F32: (1, 4), F16: (1, 2), Q5_0: (32, 22), Q8_0: (32, 34),
         Q4_K: (256, 144), Q6_K: (256, 210), Q8_K: (256, 292)}


def nbytes_for(ggml_type: int, n: int) -> int:
    """Bytes of ``n`` elements of ``ggml_type`` (dequant.py:27-48); asserts divisibility."""
    if ggml_type not in BLOCK:
        raise NotImplementedError(f"ggml type {ggml_type} not supported")
    qk, nbytes = BLOCK[ggml_type]
    assert n % qk == 0, f"type {ggml_type} needs n % {qk} == 0, got {n}"
    return (n // qk) * nbytes


def _blocks(raw, ggml_type: int, n: int) -> np.ndarray:
    qk, nbytes = BLOCK[ggml_type]
    arr = np.frombuffer(raw, dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw.view(np.uint8).reshape(-1)
    nb = n // qk
    return arr[: nb * nbytes].reshape(nb, nbytes)


def _f16_field(blk: np.ndarray, off: int) -> np.ndarray:
    """Little-endian fp16 at byte ``off`` of every block, widened to f32 (exact)."""
    return np.ascontiguousarray(blk[:, off:off + 2]).view(np.float16).astype(np.float32).reshape(-1)


def q5_0_codes(blk: np.ndarray) -> np.ndarray:
    """(nb, 32) 5-bit codes 0..31 of Q5_0 blocks (dequant.py:54-63)."""
    qh = np.ascontiguousarray(blk[:, 2:6]).view("<u4").astype(np.uint32)  # (nb,1)
    qs = blk[:, 6:22].astype(np.uint32)                                     # (nb,16)
    bit = np.arange(32, dtype=np.uint32)
    high = (qh >> bit) & 1                                                  # (nb,32)
    nib = np.concatenate([qs & 0xF, qs >> 4], axis=1)                       # (nb,32)
    return (nib | (high << 4)).astype(np.int32)


def scale_min_k4(scales: np.ndarray, j: int) -> tuple[np.ndarray, np.ndarray]:
    """6-bit scale and min of sub-block ``j`` from the 12 packed bytes (dequant.py:171-179)."""
    s = scales.astype(np.int32)
    if j < 4:
        return s[:, j] & 63, s[:, j + 4] & 63
    sc = (s[:, j + 4] & 0x0F) | ((s[:, j - 4] >> 6) << 4)
    mn = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    return sc, mn


def q4_k_parts(blk: np.ndarray):
    """Q4_K -> (d, dmin, sc (nb,8), mn (nb,8), nibbles (nb,256)) in element order."""
    d, dmin = _f16_field(blk, 0), _f16_field(blk, 2)
    scales = blk[:, 4:16]
    qs = blk[:, 16:144]
    sc = np.stack([scale_min_k4(scales, j)[0] for j in range(8)], axis=1)
    mn = np.stack([scale_min_k4(scales, j)[1] for j in range(8)], axis=1)
    nib = np.empty((blk.shape[0], 256), dtype=np.int32)
    for c in range(4):                       # 32-byte chunk c feeds sub-blocks 2c (lo), 2c+1 (hi)
        seg = qs[:, 32 * c:32 * c + 32].astype(np.int32)
        nib[:, 64 * c:64 * c + 32] = seg & 0xF
        nib[:, 64 * c + 32:64 * c + 64] = seg >> 4
    return d, dmin, sc, mn, nib


def q6_k_parts(blk: np.ndarray):
    """Q6_K -> (d, scales (nb,16) int, codes (nb,256) in -32..31) in element order (dequant.py:204-232)."""
    ql = blk[:, 0:128].astype(np.int32)
    qh = blk[:, 128:192].astype(np.int32)
    sc = np.ascontiguousarray(blk[:, 192:208]).view(np.int8).astype(np.int32)
    d = _f16_field(blk, 208)
    q = np.empty((blk.shape[0], 256), dtype=np.int32)
    for h in range(2):
        lo_a = ql[:, 64 * h:64 * h + 32]
        lo_b = ql[:, 64 * h + 32:64 * h + 64]
        hb = qh[:, 32 * h:32 * h + 32]
        base = 128 * h
        q[:, base + 0:base + 32] = ((lo_a & 0xF) | ((hb & 3) << 4)) - 32
        q[:, base + 32:base + 64] = ((lo_b & 0xF) | (((hb >> 2) & 3) << 4)) - 32
        q[:, base + 64:base + 96] = ((lo_a >> 4) | (((hb >> 4) & 3) << 4)) - 32
        q[:, base + 96:base + 128] = ((lo_b >> 4) | (((hb >> 6) & 3) << 4)) - 32
    return d, sc, q


def q6_k_scale_index() -> np.ndarray:
    """Scale slot (0..15) used by each of the 256 Q6_K elements: 8h + l//16 + 2*quarter."""
    idx = np.empty(256, dtype=np.int64)
    for e in range(256):
        h, r = divmod(e, 128)
        quarter, l = divmod(r, 32)
        idx[e] = 8 * h + l // 16 + 2 * quarter
    return idx


def dequantize(ggml_type: int, raw, n: int) -> np.ndarray:
    """Dequantize ``n`` elements to float32, bit-exact (dequant.py:243-260)."""
    if ggml_type == F32:
        return np.frombuffer(raw, dtype="<f4")[:n].astype(np.float32)
    if ggml_type == F16:
        return np.frombuffer(raw, dtype="<f2")[:n].astype(np.float32)
    blk = _blocks(raw, ggml_type, n)
    if ggml_type == Q8_0:
        d = _f16_field(blk, 0)
        q = np.ascontiguousarray(blk[:, 2:34]).view(np.int8).astype(np.float32)
        return (q * d[:, None]).reshape(-1)
    if ggml_type == Q5_0:
        d = _f16_field(blk, 0)
        return ((q5_0_codes(blk) - 16).astype(np.float32) * d[:, None]).reshape(-1)
    if ggml_type == Q4_K:
        d, dmin, sc, mn, nib = q4_k_parts(blk)
        sub = np.arange(256) // 32
        scale = (sc.astype(np.float32) * d[:, None])[:, sub]      # exact: <= 17 significant bits
        offset = (mn.astype(np.float32) * dmin[:, None])[:, sub]  # exact
        return (scale * nib.astype(np.float32) - offset).astype(np.float32).reshape(-1)
    if ggml_type == Q6_K:
        d, sc, q = q6_k_parts(blk)
        s = sc[:, q6_k_scale_index()].astype(np.float64)
        # the reference multiplies in float64 then stores f32; every product is exact
        return (q.astype(np.float64) * d[:, None].astype(np.float64) * s).astype(np.float32).reshape(-1)
    if ggml_type == Q8_K:
        d = np.ascontiguousarray(blk[:, 0:4]).view("<f4").reshape(-1)
        q = np.ascontiguousarray(blk[:, 4:260]).view(np.int8).astype(np.float32)
        return (q * d[:, None]).reshape(-1)
    raise NotImplementedError(f"dequantize for ggml type {ggml_type} not implemented")


# --- the reference's unpacked kernel form (dequant.py:79-168) ---------------------------

def unpack_q8_0(raw, n: int):
    """-> (qs int8 (n,), d f32 (n/32,))  (dequant.py:98-104)."""
    blk = _blocks(raw, Q8_0, n)
    return np.ascontiguousarray(blk[:, 2:34]).view(np.int8).reshape(-1).copy(), _f16_field(blk, 0)


def unpack_q5_0(raw, n: int):
    """-> (q5 int8 0..31 (n,), d f32 (n/32,)) without the -16 offset (dequant.py:79-95)."""
    blk = _blocks(raw, Q5_0, n)
    return q5_0_codes(blk).astype(np.int8).reshape(-1), _f16_field(blk, 0)


def unpack_q6_k(raw, n: int):
    """-> (q int8 -32..31 (n,), dsc = d*scale f32 (n/16,)) (dequant.py:107-137)."""
    blk = _blocks(raw, Q6_K, n)
    d, sc, q = q6_k_parts(blk)
    return q.astype(np.int8).reshape(-1), (sc.astype(np.float32) * d[:, None]).astype(np.float32).reshape(-1)


def unpack_q4_k(raw, n: int):
    """-> (q int8 0..15 (n,), sc*d f32 (n/32,), mn*dmin f32 (n/32,)) (dequant.py:140-168)."""
    blk = _blocks(raw, Q4_K, n)
    d, dmin, sc, mn, nib = q4_k_parts(blk)
    return (nib.astype(np.int8).reshape(-1),
            (sc.astype(np.float32) * d[:, None]).astype(np.float32).reshape(-1),
            (mn.astype(np.float32) * dmin[:, None]).astype(np.float32).reshape(-1))
