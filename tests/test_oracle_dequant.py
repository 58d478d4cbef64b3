"""Pins the oracle's block decode (oracle/dequant.py) before it is used to judge the GPU.

Checks: the reference's known-answer blocks and hand-derived blocks (golden JSON), bit-exact
agreement with the independent C restatement on random blocks of every format (random
bytes, so every code value, sign and fp16 pattern incl. subnormals/inf/nan occurs), the fp16
decode over all 65536 patterns against numpy, the unpacked kernel form against the dequant
form, and quantize -> dequantize round trips of the host quantizer.
"""

import ctypes
import json

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import dequant as dq

KA = json.loads((GOLDEN / "dequant_known_answers.json").read_text())


def c_dequant(lib, t, raw: bytes, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    buf = np.frombuffer(raw, np.uint8).copy()
    assert lib.oracle_dequantize(t, buf.ctypes.data, n, out.ctypes.data) == 0
    return out


def random_blocks(t: int, nblk: int, seed: int) -> bytes:
    qk, size = dq.BLOCK[t]
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=nblk * size, dtype=np.uint8).reshape(nblk, size)
    # keep the fp16 scales finite so values compare with ==
    offs = {8: [0], 6: [0], 12: [0, 2], 14: [208]}.get(t, [])
    for o in offs:
        raw[:, o + 1] &= 0x7B  # exponent < 31
    if t == 15:  # Q8_K f32 d: finite
        raw[:, 3] &= 0x3F
    return raw.tobytes()


@pytest.mark.parametrize("c", KA["cases"], ids=[c["name"] for c in KA["cases"]])
def test_known_answers_numpy(c):
    out = dq.dequantize(c["type"], bytes.fromhex(c["block_hex"]), c["n"])
    np.testing.assert_array_equal(out, np.array(c["expected"], np.float32))


@pytest.mark.parametrize("c", KA["cases"], ids=[c["name"] for c in KA["cases"]])
def test_known_answers_c(oracle_clib, c):
    out = c_dequant(oracle_clib, c["type"], bytes.fromhex(c["block_hex"]), c["n"])
    np.testing.assert_array_equal(out, np.array(c["expected"], np.float32))


def test_nbytes_for():
    for t, n, nbytes in KA["nbytes_for"]:
        assert dq.nbytes_for(t, n) == nbytes
    with pytest.raises(AssertionError):
        dq.nbytes_for(dq.Q4_K, 896)
    with pytest.raises(NotImplementedError):
        dq.nbytes_for(99, 32)


@pytest.mark.parametrize("t", [dq.Q8_0, dq.Q5_0, dq.Q4_K, dq.Q6_K, dq.Q8_K, dq.F16])
def test_numpy_matches_c_on_random_blocks(oracle_clib, t):
    qk, size = dq.BLOCK[t]
    nblk = 4096 if qk == 32 else 512
    if t == dq.F16:
        rng = np.random.default_rng(3)
        raw = rng.standard_normal(4096).astype(np.float16).tobytes()
        n = 4096
    else:
        raw = random_blocks(t, nblk, seed=t)
        n = nblk * qk
    a = dq.dequantize(t, raw, n)
    b = c_dequant(oracle_clib, t, raw, n)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))


def test_fp16_decode_all_patterns(oracle_clib):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle_clib.oracle_half_to_float(int(b)) for b in bits], np.float32)
    finite = np.isfinite(ref)
    np.testing.assert_array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    assert np.all(got[np.isinf(ref)] == ref[np.isinf(ref)])


def test_q5_0_every_code():
    """Every 5-bit code at every position: qs nibbles 0..15 x qh bit 0/1 -> value code-16."""
    for hb in (0, 1):
        for nib in range(16):
            qs = bytes([nib | (nib << 4)] * 16)
            qh = 0xFFFFFFFF if hb else 0
            blk = np.float16(1.0).tobytes() + int(qh).to_bytes(4, "little") + qs
            out = dq.dequantize(dq.Q5_0, blk, 32)
            assert np.all(out == (nib | (hb << 4)) - 16)


def test_q6_k_every_code():
    """Every 6-bit code in every quarter: ql nibble x qh 2-bit field -> value code-32."""
    for hi2 in range(4):
        for nib in range(16):
            ql = bytes([nib | (nib << 4)] * 128)
            qh = bytes([hi2 | (hi2 << 2) | (hi2 << 4) | (hi2 << 6)] * 64)
            blk = ql + qh + bytes([1] * 16) + np.float16(1.0).tobytes()
            out = dq.dequantize(dq.Q6_K, blk, 256)
            assert np.all(out == (nib | (hi2 << 4)) - 32)


def test_unpack_forms_match_dequant():
    """The reference's int8+scale kernel form reproduces the dequantized weights."""
    for t in (dq.Q8_0, dq.Q5_0, dq.Q4_K, dq.Q6_K):
        qk, _ = dq.BLOCK[t]
        nblk = 64 if qk == 256 else 512
        raw = random_blocks(t, nblk, seed=100 + t)
        n = nblk * qk
        w = dq.dequantize(t, raw, n).astype(np.float64)
        if t == dq.Q8_0:
            q, d = dq.unpack_q8_0(raw, n)
            rec = q.reshape(-1, 32) * d[:, None].astype(np.float64)
        elif t == dq.Q5_0:
            q, d = dq.unpack_q5_0(raw, n)
            rec = (q.reshape(-1, 32).astype(np.float64) - 16) * d[:, None]
        elif t == dq.Q6_K:
            q, dsc = dq.unpack_q6_k(raw, n)
            rec = q.reshape(-1, 16) * dsc[:, None].astype(np.float64)
        else:
            q, sc, mn = dq.unpack_q4_k(raw, n)
            rec = q.reshape(-1, 32) * sc[:, None].astype(np.float64) - mn[:, None]
        np.testing.assert_allclose(rec.reshape(-1), w, rtol=2e-7, atol=0)


def test_q4_k_scale_pack_is_inverse_of_unpack():
    """pico_hip's K4 scale packer and the oracle's unpacker agree on all 64x64 (sc, m) pairs
    in every sub-block slot."""
    from pico_hip.quantize import pack_k4_scales
    vals = np.arange(64)
    for j in range(8):
        ls = np.zeros((4096, 8), np.int32)
        lm = np.zeros((4096, 8), np.int32)
        ls[:, j] = np.repeat(vals, 64)
        lm[:, j] = np.tile(vals, 64)
        packed = pack_k4_scales(ls, lm)
        sc, mn = dq.scale_min_k4(packed, j)
        np.testing.assert_array_equal(sc, ls[:, j])
        np.testing.assert_array_equal(mn, lm[:, j])


@pytest.mark.parametrize("t,tol", [(dq.Q8_0, 1 / 127), (dq.Q5_0, 1 / 16), (dq.Q4_K, 1 / 8),
                                   (dq.Q6_K, 1 / 24)])
def test_quantize_roundtrip(t, tol):
    """quantize -> dequantize reproduces the input within the format's step (relative to the
    block's range); a wrong bit position or scale index would blow far past it."""
    from pico_hip.quantize import quantize
    qk, _ = dq.BLOCK[t]
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(qk * 256) * 0.02).astype(np.float32)
    w = dq.dequantize(t, quantize(t, x).tobytes(), x.size)
    blocks = x.reshape(-1, qk)
    err = np.abs(w.reshape(-1, qk) - blocks).max(axis=1)
    rng_ = np.abs(blocks).max(axis=1)
    assert np.all(err <= tol * rng_ * 1.05 + 1e-9), float((err / rng_).max())
