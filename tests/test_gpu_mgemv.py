"""Decode GEMVs on the integer matrix cores (pe_mgemv, from the MFMA layout) against float64
on the dequantized weights (1e-3 relative, the decode bound; fp32-level in practice) and
against the tiled GEMVs."""

import numpy as np
import pytest
import torch

from helpers import dequant_rows, quantized_normal, random_quant, rel_err
from oracle import closed
from oracle import dequant as dq

pytestmark = pytest.mark.gpu
TOL = 1e-3
DEV = "cuda"


@pytest.fixture(scope="module")
def K():
    from pico_hip import kernels
    return kernels


def mweight(K, t, raw, n, k):
    blocks = torch.from_numpy(np.frombuffer(raw, np.uint8).copy()).to(DEV)
    return K.pack_weight(blocks, t, n, k, mfma=True)


# (type, k, n): one super-block, row counts that leave a partial row group, the 7B inner
# sizes, a workgroup looping over several tiles (n / 16 > CUs)
SHAPES = [(dq.Q4_K, 256, 16), (dq.Q6_K, 256, 40), (dq.Q4_K, 3584, 1000), (dq.Q6_K, 3584, 520),
          (dq.Q4_K, 18944, 64), (dq.Q6_K, 18944, 96), (dq.Q6_K, 4864, 4608), (dq.Q4_K, 1024, 9000)]


@pytest.mark.parametrize("t,k,n", SHAPES, ids=[f"{t}-{k}x{n}" for t, k, n in SHAPES])
def test_mgemv_matches_closed_form(K, t, k, n):
    raw = quantized_normal(t, n, k, seed=k + 3 * n + t)
    w = mweight(K, t, raw, n, k)
    W = dequant_rows(t, raw, n, k)
    rng = np.random.default_rng(k + n)
    x = rng.standard_normal(k).astype(np.float32)
    r = rng.standard_normal(n).astype(np.float32)
    xt, rt = torch.from_numpy(x).to(DEV), torch.from_numpy(r).to(DEV)
    y = K.mgemv(xt, w).cpu().numpy()
    assert rel_err(y, closed.gemv(W, x)) < 1e-5
    yr = K.mgemv(xt, w, residual=rt)
    assert rel_err(yr.cpu().numpy(), closed.gemv(W, x, residual=r)) < TOL
    assert torch.equal(K.mgemv(xt, w, residual=rt), yr)  # fixed reduction order
    if n % 32 == 0:
        ut = K.mgemv(K.to_ut(xt), w, residual=K.to_ut(rt), layout=K.LAYOUT_X_UT | K.LAYOUT_Y_UT)
        assert torch.equal(K.from_ut(ut), yr)  # the layouts only move elements


@pytest.mark.parametrize("t,k,n", [(dq.Q4_K, 3584, 512), (dq.Q6_K, 4864, 256), (dq.Q4_K, 18944, 96)])
def test_mgemv_rmsnorm_and_silu(K, t, k, n):
    """RMSNorm (sum of squares factored out) and the [gate; up] SiLU pair of 2n rows."""
    raw = quantized_normal(t, 2 * n, k, seed=n + k)
    w = mweight(K, t, raw, 2 * n, k)
    W = dequant_rows(t, raw, 2 * n, k)
    rng = np.random.default_rng(n)
    x = rng.standard_normal(k).astype(np.float32)
    nw = (rng.standard_normal(k) * 0.5).astype(np.float32)
    xt, nt = torch.from_numpy(x).to(DEV), torch.from_numpy(nw).to(DEV)
    h = closed.rmsnorm(x, nw, 1e-6)
    y = K.mgemv(xt, w, norm_w=nt, eps=1e-6).cpu().numpy()
    assert rel_err(y, closed.gemv(W, h)) < 1e-5
    act = K.mgemv(xt, w, norm_w=nt, eps=1e-6, silu=True)
    gu = closed.gemv(W, h)
    assert rel_err(act.cpu().numpy(), closed.silu_mul(gu[:n], gu[n:])) < 1e-5
    ut = K.mgemv(K.to_ut(xt), w, norm_w=K.to_ut(nt), eps=1e-6, silu=True, layout=K.LAYOUT_X_UT)
    assert torch.equal(ut, act)
    act_plain = K.mgemv(xt, w, silu=True).cpu().numpy()  # without the norm
    g2 = closed.gemv(W, x)
    assert rel_err(act_plain, closed.silu_mul(g2[:n], g2[n:])) < 1e-5


def _pow2_blocks(t, codes):
    """GGUF blocks (rows of 256-element super-blocks) with d = 1/16, unit scales, zero mins and
    the given unsigned codes (Q4_K: 0..15; Q6_K: 0..63, weight (code - 32) / 16): every weight
    is code / 16 or (code - 32) / 16, exact in fp16 products."""
    n, k = codes.shape
    out = bytearray()
    d = np.float16(1 / 16).tobytes()
    for r in range(n):
        for s in range(k // 256):
            c = codes[r, 256 * s:256 * (s + 1)]
            if t == dq.Q4_K:
                b = bytearray(144)
                b[0:2] = d
                b[4:16] = bytes([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1])  # sc = 1, m = 0
                for e in range(256):
                    j, l = divmod(e, 32)
                    b[16 + 32 * (j // 2) + l] |= int(c[e]) << (4 if j % 2 else 0)
            else:
                b = bytearray(210)
                for e in range(256):
                    h, rest = divmod(e, 128)
                    qt, l = divmod(rest, 32)
                    b[64 * h + l + 32 * (qt & 1)] |= (int(c[e]) & 15) << (4 if qt >> 1 else 0)
                    b[128 + 32 * h + l] |= (int(c[e]) >> 4) << (2 * qt)
                b[192:208] = bytes([1] * 16)
                b[208:210] = d
            out += b
    return bytes(out)


@pytest.mark.parametrize("t", [dq.Q4_K, dq.Q6_K])
def test_mgemv_low_planes_and_tiny_sub_blocks(K, t):
    """A single activation v whose low bits sit in plane 1, 2 or 3 (v = 1 + 2^-8, 1 + 2^-15,
    1 + 2^-22) or whose sub-block maximum is tiny (3 * 2^-30 (1 + 2^-9)), against power-of-two
    weights: Q4_K returns W[:, j] * v exactly (every product and the plane sum are exact), Q6_K
    (whose -32 offset is subtracted after rounding) to 2^-18, which a dropped plane 1 or 2 fails."""
    n, k = 32, 512
    rng = np.random.default_rng(7)
    vals = np.array([0, 1, 2, 4, 8])
    codes = vals[rng.integers(0, 5, (n, k))] + (0 if t == dq.Q4_K else 32)
    raw = _pow2_blocks(t, codes)
    w = mweight(K, t, raw, n, k)
    W = dequant_rows(t, raw, n, k).astype(np.float64)
    vs = [1 + 2.0 ** -8, 1 + 2.0 ** -15, 3 * 2.0 ** -30 * (1 + 2.0 ** -9)]
    if t == dq.Q4_K:
        vs.append(1 + 2.0 ** -22)
    for j in (0, 33, 300, k - 1):
        for v in vs:
            x = torch.zeros(k, device=DEV)
            x[j] = v
            y = K.mgemv(x, w).double().cpu().numpy()
            ref = W[:, j] * np.float64(np.float32(v))
            if t == dq.Q4_K:
                np.testing.assert_array_equal(y, ref)
            else:
                np.testing.assert_allclose(y, ref, rtol=2.0 ** -18, atol=0)


@pytest.mark.parametrize("t", [dq.Q4_K, dq.Q6_K])
def test_mgemv_one_hot_columns(K, t):
    """x = e_j returns column j of W: exactly for Q4_K (d sc q - dmin m with the dequantizer's
    one rounding), to one rounding of d sc (q - 32) for Q6_K. Pins the code and row layout."""
    n, k = 48, 2048
    raw = random_quant(t, n, k, seed=21 + t)
    w = mweight(K, t, raw, n, k)
    W = dequant_rows(t, raw, n, k)
    for j in (0, 1, 7, 8, 15, 16, 31, 32, 100, 255, 256, 1000, k - 1):
        x = torch.zeros(k, device=DEV)
        x[j] = 1.0
        y = K.mgemv(x, w).cpu().numpy()
        if t == dq.Q4_K:
            np.testing.assert_array_equal(y, W[:, j])
        else:
            np.testing.assert_allclose(y, W[:, j], rtol=2 ** -22, atol=0)


def test_mgemv_nonfinite_activation_gives_nan(K):
    t, n, k = dq.Q4_K, 32, 512
    raw = quantized_normal(t, n, k, seed=4)
    w = mweight(K, t, raw, n, k)
    x = torch.randn(k, device=DEV)
    x[300] = float("inf")
    assert torch.isnan(K.mgemv(x, w)).all()


def test_mgemv_is_the_decode_path_for_large_matrices(K):
    """pack_weight keeps an MFMA copy of large Q4_K / Q6_K matrices only; qgemv, qgemv_norm and
    qgemv_norm_silu then run pe_mgemv, within fp32 rounding of the tiled kernels."""
    t, k, ffn = dq.Q4_K, 3584, 4736
    assert not K.mfma_eligible(dq.Q4_K, 896, 4864) and not K.mfma_eligible(dq.Q5_0, 37888, 3584)
    assert not K.mfma_eligible(dq.Q4_K, 3584, 3584)  # the 7B o-projection stays tiled
    assert K.mfma_eligible(t, 2 * ffn, k)
    raw = quantized_normal(t, 2 * ffn, k, seed=8)
    blocks = torch.from_numpy(np.frombuffer(raw, np.uint8).copy()).to(DEV)
    w = K.pack_weight(blocks, t, 2 * ffn, k)
    assert w.mfma is not None and w.mfma.numel() == K.lib.pe_mfma_bytes(t, 2 * ffn, k)
    rng = np.random.default_rng(5)
    x = torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(DEV)
    nw = torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(DEV)
    r = torch.from_numpy(rng.standard_normal(2 * ffn).astype(np.float32)).to(DEV)
    runs = {}
    for on in (True, False):
        K.use_mfma_gemv = on
        try:
            runs[on] = (K.qgemv(x, w, residual=r), K.qgemv_norm(x, nw, w, 1e-6),
                        K.qgemv_norm_silu(x, nw, w, 1e-6))
        finally:
            K.use_mfma_gemv = True
    for a, b in zip(runs[True], runs[False]):
        assert rel_err(a.cpu().numpy(), b.cpu().numpy()) < 1e-5


def test_mgemv_rejects_bad_arguments(K):
    """Status codes (no launch): another type, k not a multiple of 256, the SiLU pair with a
    residual, a unit-transposed y of n % 32 != 0."""
    t, n, k = dq.Q4_K, 48, 512
    raw = quantized_normal(t, n, k, seed=4)
    w = mweight(K, t, raw, n, k)
    x, y = torch.zeros(k, device=DEV), torch.zeros(n, device=DEV)
    call = lambda ty, nn, kk, res, silu, layout: K.lib.pe_mgemv(
        ty, w.mfma.data_ptr(), nn, kk, x.data_ptr(), None, 0.0, res, y.data_ptr(), silu, layout, None)
    assert call(dq.Q8_0, n, k, None, 0, 0) == 2
    assert call(t, n, 500, None, 0, 0) == 3
    assert call(t, n // 2, k, y.data_ptr(), 1, 0) == 3
    assert call(t, n, k, None, 0, K.LAYOUT_Y_UT) == 3
    assert call(t, n, k, None, 0, 0) == 0
    torch.cuda.synchronize()
