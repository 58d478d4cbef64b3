"""GPU parity of every kernel against the oracle (bit-exact dequant, 1e-3 relative GEMV and
attention, as the decode path requires). Run on an MI355X: pytest -m gpu."""

import json

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from helpers import dequant_rows, quantized_normal, random_quant, rel_err
from oracle import closed
from oracle import dequant as dq

pytestmark = pytest.mark.gpu
TOL = 1e-3  # relative, fp32 accumulate

KA = json.loads((GOLDEN / "dequant_known_answers.json").read_text())
DEV = "cuda"


@pytest.fixture(scope="module")
def K():
    from pico_hip import kernels
    return kernels


def dev_bytes(raw: bytes) -> torch.Tensor:
    return torch.from_numpy(np.frombuffer(raw, np.uint8).copy()).to(DEV)


def qweight(K, t, raw, n, k):
    return K.pack_weight(dev_bytes(raw), t, n, k)


# ---- dequantization (bit-exact) ----------------------------------------------------------

@pytest.mark.parametrize("c", KA["cases"], ids=[c["name"] for c in KA["cases"]])
def test_dequant_known_answers(K, c):
    out = K.dequantize(c["type"], dev_bytes(bytes.fromhex(c["block_hex"])), c["n"]).cpu().numpy()
    np.testing.assert_array_equal(out, np.array(c["expected"], np.float32))


@pytest.mark.parametrize("t", [dq.Q8_0, dq.Q5_0, dq.Q4_K, dq.Q6_K])
def test_dequant_random_blocks_bitexact(K, t):
    qk = dq.BLOCK[t][0]
    raw = random_quant(t, 64, 8 * qk, seed=11 + t)
    n = 64 * 8 * qk
    gpu = K.dequantize(t, dev_bytes(raw), n).cpu().numpy()
    ref = dq.dequantize(t, raw, n)
    np.testing.assert_array_equal(gpu.view(np.uint32), ref.view(np.uint32))


def test_dequant_f16_f32_q8k(K):
    rng = np.random.default_rng(1)
    h = rng.standard_normal(1000).astype(np.float16)
    h[:5] = np.array([0x0001, 0x03FF, 0x8001, 0x7BFF, 0x0400], np.uint16).view(np.float16)
    np.testing.assert_array_equal(K.dequantize(dq.F16, dev_bytes(h.tobytes()), 1000).cpu().numpy(),
                                  h.astype(np.float32))
    f = rng.standard_normal(999).astype(np.float32)
    np.testing.assert_array_equal(K.dequantize(dq.F32, dev_bytes(f.tobytes()), 999).cpu().numpy(), f)
    raw = rng.integers(0, 256, size=(8, 292), dtype=np.uint8)
    raw[:, 0:4] = (rng.standard_normal(8).astype(np.float32) * 0.01).view(np.uint8).reshape(-1, 4)
    out = K.dequantize(dq.Q8_K, dev_bytes(raw.tobytes()), 2048).cpu().numpy()
    np.testing.assert_array_equal(out, dq.dequantize(dq.Q8_K, raw.tobytes(), 2048))


@pytest.mark.parametrize("t,n,k", [(dq.Q8_0, 96, 896), (dq.Q5_0, 96, 896), (dq.Q4_K, 40, 4864),
                                   (dq.Q6_K, 40, 4864), (dq.Q5_0, 8, 4864), (dq.Q8_0, 8, 256)])
def test_tiled_decode_bitexact(K, t, n, k):
    """pe_repack + the GEMV kernels' own unit decode reproduce the oracle bit for bit."""
    raw = random_quant(t, n, k, seed=n + k + t)
    w = qweight(K, t, raw, n, k)
    gpu = K.dequantize_weight(w).cpu().numpy()
    ref = dequant_rows(t, raw, n, k)
    np.testing.assert_array_equal(gpu.view(np.uint32), ref.view(np.uint32))


def test_embed_gather(K):
    raw = random_quant(dq.Q8_0, 50, 896, seed=3)
    table = K.RawTensor(dev_bytes(raw), dq.Q8_0, (50, 896))
    ids = torch.tensor([0, 49, 7, 7, -1, 50], device=DEV)
    out = K.embed_gather(table, ids).cpu().numpy()
    ref = dequant_rows(dq.Q8_0, raw, 50, 896)
    np.testing.assert_array_equal(out[:4], ref[[0, 49, 7, 7]])
    assert np.all(np.isnan(out[4:]))  # out-of-range ids give NaN rows, no OOB read


# ---- dequant-GEMV -------------------------------------------------------------------------

GEMV_SHAPES = [  # (type, K_in, N_out): the config-1 microbench shapes + 7B shapes
    (dq.Q5_0, 896, 1152), (dq.Q5_0, 896, 896), (dq.Q5_0, 896, 9728), (dq.Q5_0, 4864, 896),
    (dq.Q8_0, 896, 1152), (dq.Q8_0, 896, 896), (dq.Q8_0, 896, 9728), (dq.Q8_0, 4864, 896),
    (dq.Q4_K, 4864, 896), (dq.Q6_K, 4864, 896),
    (dq.Q4_K, 3584, 512), (dq.Q6_K, 3584, 512), (dq.Q4_K, 18944, 256), (dq.Q6_K, 18944, 256),
    (dq.Q8_0, 1024, 100), (dq.Q5_0, 2048, 64),
]


@pytest.mark.parametrize("t,k,n", GEMV_SHAPES, ids=[f"{dq.BLOCK[t][0]}-{t}-{k}x{n}" for t, k, n in GEMV_SHAPES])
def test_qgemv_matches_closed_form(K, t, k, n):
    raw = quantized_normal(t, n, k, seed=k + n + t)
    w = qweight(K, t, raw, n, k)
    rng = np.random.default_rng(k * 7 + n)
    x = rng.standard_normal(k).astype(np.float32)
    y = K.qgemv(torch.from_numpy(x).to(DEV), w).cpu().numpy()
    ref = closed.gemv(dequant_rows(t, raw, n, k), x)
    assert rel_err(y, ref) < TOL


def test_qgemv_lm_head_rows(K):
    """896 -> 151936 Q8_0 (the LM head); a seeded subset of rows checked in float64."""
    n, k = 151936, 896
    raw = quantized_normal(dq.Q8_0, n, k, seed=42)
    w = qweight(K, dq.Q8_0, raw, n, k)
    x = np.random.default_rng(0).standard_normal(k).astype(np.float32)
    y = K.qgemv(torch.from_numpy(x).to(DEV), w).cpu().numpy()
    rows = np.sort(np.random.default_rng(1).choice(n, 4096, replace=False))
    rows = np.concatenate([rows, [0, n - 1]])
    blk = np.frombuffer(raw, np.uint8).reshape(n, -1)[rows]
    ref = closed.gemv(dequant_rows(dq.Q8_0, blk.tobytes(), len(rows), k), x)
    assert rel_err(y[rows], ref) < TOL


@pytest.mark.parametrize("t,k", [(dq.Q8_0, 896), (dq.Q5_0, 896), (dq.Q4_K, 4864), (dq.Q6_K, 4864),
                                 (dq.Q6_K, 18944)])
def test_qgemv_one_hot_is_exact_column(K, t, k):
    """x = e_j gives column j of W exactly: pins row/column indexing and the unit layout."""
    n = 64
    raw = random_quant(t, n, k, seed=5 + t)
    w = qweight(K, t, raw, n, k)
    W = dequant_rows(t, raw, n, k)
    for j in (0, 1, 31, 32, 255, 256, k // 2 + 17, k - 1):
        x = torch.zeros(k, device=DEV)
        x[j] = 1.0
        y = K.qgemv(x, w).cpu().numpy()
        np.testing.assert_array_equal(y, W[:, j])


def test_qgemv_residual_bias_and_determinism(K):
    t, k, n = dq.Q5_0, 896, 1152
    raw = quantized_normal(t, n, k, seed=9)
    w = qweight(K, t, raw, n, k)
    rng = np.random.default_rng(2)
    x, r, b = (rng.standard_normal(s).astype(np.float32) for s in (k, n, n))
    X, R, B = (torch.from_numpy(v).to(DEV) for v in (x, r, b))
    y1 = K.qgemv(X, w, residual=R, bias=B)
    y2 = K.qgemv(X, w, residual=R, bias=B)
    assert torch.equal(y1, y2)  # fixed reduction order: bitwise repeatable
    ref = closed.gemv(dequant_rows(t, raw, n, k), x, bias=b, residual=r)
    assert rel_err(y1.cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("t,k,n", [(dq.Q5_0, 896, 9728), (dq.Q8_0, 896, 4096), (dq.Q4_K, 3584, 1024)])
def test_qgemv_rmsnorm(K, t, k, n):
    raw = quantized_normal(t, n, k, seed=t + k)
    w = qweight(K, t, raw, n, k)
    rng = np.random.default_rng(4)
    x = rng.standard_normal(k).astype(np.float32)
    nw = (rng.standard_normal(k) * 0.5).astype(np.float32)
    y = K.qgemv_norm(torch.from_numpy(x).to(DEV), torch.from_numpy(nw).to(DEV), w, 1e-6).cpu().numpy()
    ref = closed.gemv(dequant_rows(t, raw, n, k), closed.rmsnorm(x, nw, 1e-6))
    assert rel_err(y, ref) < TOL


@pytest.mark.parametrize("t,k,ffn", [(dq.Q5_0, 896, 4864), (dq.Q4_K, 3584, 512)])
def test_qgemv_rmsnorm_silu(K, t, k, ffn):
    raw = quantized_normal(t, 2 * ffn, k, seed=ffn)
    w = qweight(K, t, raw, 2 * ffn, k)
    rng = np.random.default_rng(6)
    x = rng.standard_normal(k).astype(np.float32)
    nw = rng.standard_normal(k).astype(np.float32)
    act = K.qgemv_norm_silu(torch.from_numpy(x).to(DEV), torch.from_numpy(nw).to(DEV), w, 1e-6).cpu().numpy()
    gu = closed.gemv(dequant_rows(t, raw, 2 * ffn, k), closed.rmsnorm(x, nw, 1e-6))
    assert rel_err(act, closed.silu_mul(gu[:ffn], gu[ffn:])) < TOL


@pytest.mark.parametrize("m", [1, 5, 8, 13, 17, 64, 100, 129])
@pytest.mark.parametrize("t,k,n", [(dq.Q5_0, 896, 1152), (dq.Q6_K, 4864, 896), (dq.Q8_0, 896, 300)])
def test_qgemm_prefill(K, m, t, k, n):
    raw = quantized_normal(t, n, k, seed=m + n)
    w = qweight(K, t, raw, n, k)
    rng = np.random.default_rng(m)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    r = rng.standard_normal((m, n)).astype(np.float32)
    out = torch.full((m, n + 7), float("nan"), device=DEV)  # strided destination
    K.qgemm(torch.from_numpy(x).to(DEV), w, bias=torch.from_numpy(b).to(DEV),
            residual=torch.from_numpy(r).to(DEV), out=out[:, 3:3 + n])
    got = out.cpu().numpy()
    W = dequant_rows(t, raw, n, k).astype(np.float64)
    ref = x.astype(np.float64) @ W.T + b + r
    assert rel_err(got[:, 3:3 + n], ref) < TOL
    assert np.all(np.isnan(got[:, :3])) and np.all(np.isnan(got[:, 3 + n:]))


# Launches of more than 2048 blocks at one task per group run the looped form (capped grid,
# several tasks per group, next chunk's loads in flight): plain with residual in both layouts,
# RMSNorm, and the SiLU pair, one shape per lane-group width.
LOOP_SHAPES = [(dq.Q8_0, 896, 20000), (dq.Q4_K, 3584, 6016), (dq.Q5_0, 4864, 2100),
               (dq.Q6_K, 18944, 2112)]


@pytest.mark.parametrize("t,k,n", LOOP_SHAPES, ids=[f"{t}-{k}x{n}" for t, k, n in LOOP_SHAPES])
def test_qgemv_looped_form(K, t, k, n):
    raw = quantized_normal(t, n, k, seed=k + 5 * n)
    w = qweight(K, t, raw, n, k)
    W = dequant_rows(t, raw, n, k)
    rng = np.random.default_rng(n)
    x = rng.standard_normal(k).astype(np.float32)
    r = rng.standard_normal(n).astype(np.float32)
    xt, rt = torch.from_numpy(x).to(DEV), torch.from_numpy(r).to(DEV)
    nat = K.qgemv(xt, w, residual=rt)
    assert rel_err(nat.cpu().numpy(), closed.gemv(W, x, residual=r)) < TOL
    if n % 32 == 0:
        ut = K.qgemv(K.to_ut(xt), w, residual=K.to_ut(rt), layout=K.LAYOUT_X_UT | K.LAYOUT_Y_UT)
        assert rel_err(K.from_ut(ut).cpu().numpy(), nat.cpu().numpy()) < 1e-6
    if k <= 8192:
        nw = (rng.standard_normal(k) * 0.5).astype(np.float32)
        y = K.qgemv_norm(xt, torch.from_numpy(nw).to(DEV), w, 1e-6).cpu().numpy()
        assert rel_err(y, closed.gemv(W, closed.rmsnorm(x, nw, 1e-6))) < TOL
    assert torch.equal(K.qgemv(xt, w, residual=rt), nat)  # deterministic


def test_qgemv_rmsnorm_silu_looped_form(K):
    t, k, ffn = dq.Q4_K, 3584, 4200
    raw = quantized_normal(t, 2 * ffn, k, seed=ffn)
    w = qweight(K, t, raw, 2 * ffn, k)
    rng = np.random.default_rng(6)
    x = rng.standard_normal(k).astype(np.float32)
    nw = rng.standard_normal(k).astype(np.float32)
    xt, nt = torch.from_numpy(x).to(DEV), torch.from_numpy(nw).to(DEV)
    act = K.qgemv_norm_silu(xt, nt, w, 1e-6).cpu().numpy()
    gu = closed.gemv(dequant_rows(t, raw, 2 * ffn, k), closed.rmsnorm(x, nw, 1e-6))
    assert rel_err(act, closed.silu_mul(gu[:ffn], gu[ffn:])) < TOL
    ut = K.qgemv_norm_silu(K.to_ut(xt), K.to_ut(nt), w, 1e-6, layout=K.LAYOUT_X_UT)
    assert rel_err(ut.cpu().numpy(), act) < 1e-6


# ---- attention ----------------------------------------------------------------------------

def _kv(rng, n_kv, cap, hd):
    return (rng.standard_normal((n_kv, cap, hd)).astype(np.float32),
            rng.standard_normal((n_kv, cap, hd)).astype(np.float32))


@pytest.mark.parametrize("hd,n_head,n_kv", [(64, 14, 2), (128, 28, 4), (64, 4, 4)])
# capacities <= 256: one pass per head; up to 512 (hd 128) / 1024 (hd 64): one 1024-thread
# workgroup per head; beyond: split chunks + merge launch
@pytest.mark.parametrize("S,cap", [(1, 8), (17, 77), (64, 64), (65, 130), (130, 130), (512, 600),
                                   (4096, 4096), (257, 300), (1, 400), (300, 512), (512, 512),
                                   (1000, 1024), (700, 1100)])
def test_decode_attn(K, hd, n_head, n_kv, S, cap):
    rng = np.random.default_rng(S + hd)
    q = rng.standard_normal((n_head, hd)).astype(np.float32)
    k, v = _kv(rng, n_kv, cap, hd)
    out = K.decode_attn(torch.from_numpy(q).to(DEV), torch.from_numpy(k).to(DEV),
                        torch.from_numpy(v).to(DEV), S=torch.tensor([S], device=DEV)).cpu().numpy()
    ref = closed.attention(q, k, v, S, round_fp16=False)
    assert rel_err(out, ref) < TOL
    # the stored values are fp16-representable (kernels.py:126 rounding)
    np.testing.assert_array_equal(out, out.astype(np.float16).astype(np.float32))


def test_decode_attn_long_context_and_len_forms(K):
    """32768-long cache (config 2), S given as int, int32, int64 tensor, and with an offset."""
    rng = np.random.default_rng(0)
    n_head, n_kv, hd, cap = 14, 2, 64, 32768
    q = rng.standard_normal((n_head, hd)).astype(np.float32)
    k, v = _kv(rng, n_kv, cap, hd)
    Q, Kc, Vc = (torch.from_numpy(a).to(DEV) for a in (q, k, v))
    ref = closed.attention(q, k, v, 32768)
    for S in (32768, torch.tensor([32768], device=DEV, dtype=torch.int32),
              torch.tensor([32767], device=DEV)):
        kw = {"S_offset": 1} if isinstance(S, torch.Tensor) and S.dtype == torch.int64 else {}
        out = K.decode_attn(Q, Kc, Vc, S=S, **kw).cpu().numpy()
        assert rel_err(out, ref) < TOL
    out = K.decode_attn(Q, Kc, Vc, S=None).cpu().numpy()  # default S = capacity
    assert rel_err(out, ref) < TOL


# single pass (100), split + merge launch (10 and 24 chunks of 64 positions)
@pytest.mark.parametrize("cap", [100, 600, 1500])
def test_decode_attn_unrounded_and_clamp(K, cap):
    rng = np.random.default_rng(8)
    q = rng.standard_normal((14, 64)).astype(np.float32)
    k, v = _kv(rng, 2, cap, 64)
    Q, Kc, Vc = (torch.from_numpy(a).to(DEV) for a in (q, k, v))
    out = K.decode_attn(Q, Kc, Vc, S=90, round_fp16=False).cpu().numpy()
    assert rel_err(out, closed.attention(q, k, v, 90)) < 1e-5
    over = K.decode_attn(Q, Kc, Vc, S=cap + 900).cpu().numpy()  # S > capacity clamps (kernels.py:110)
    assert rel_err(over, closed.attention(q, k, v, cap)) < TOL
    empty = K.decode_attn(Q, Kc, Vc, S=0).cpu().numpy()   # S = 0: 0/0 like the reference
    assert np.all(np.isnan(empty))


@pytest.mark.parametrize("cap", [100, 1500, 32768])  # single pass / split + merge launch
def test_decode_attn_fp16_rounding_is_nearest_even(K, cap):
    """The stored output is the kernel's own unrounded fp32 result converted to fp16 with
    round-to-nearest-even (Triton's default for acc.to(tl.float16), kernels.py:126; numpy's
    astype(float16)): fp16 subnormals kept, values past 65504 to infinity. A truncating,
    flushing or saturating conversion fails this bit for bit."""
    rng = np.random.default_rng(cap)
    q = rng.standard_normal((14, 64)).astype(np.float32)
    k, v = _kv(rng, 2, cap, 64)
    Q, Kc = torch.from_numpy(q).to(DEV), torch.from_numpy(k).to(DEV)
    # normal, fp16-subnormal and overflowing outputs (a mean of 3e4 * (3 + N(0,1)) values)
    for vscale, shift in ((1.0, 0.0), (3e-6, 0.0), (3e4, 3.0)):
        Vc = torch.from_numpy((v + np.float32(shift)) * np.float32(vscale)).to(DEV)
        u = K.decode_attn(Q, Kc, Vc, S=cap - 3, round_fp16=False).cpu().numpy()
        r = K.decode_attn(Q, Kc, Vc, S=cap - 3).cpu().numpy()
        with np.errstate(over="ignore"):
            want = u.astype(np.float16).astype(np.float32)
        np.testing.assert_array_equal(r, want)
        assert not np.array_equal(r, u)
        if vscale > 1:
            assert np.isinf(r).any()
        if vscale < 1:
            assert (np.abs(r[r != 0]) < 6.1e-5).any()


@pytest.mark.parametrize("cap", [200, 300, 1500])  # single pass / split + merge launch
def test_decode_attn_workspace_reuse_and_graph(K, cap):
    """One workspace across many in-order calls and across graph replays with a device S."""
    rng = np.random.default_rng(9)
    n_head, n_kv, hd = 14, 2, 64
    q = rng.standard_normal((n_head, hd)).astype(np.float32)
    k, v = _kv(rng, n_kv, cap, hd)
    Q, Kc, Vc = (torch.from_numpy(a).to(DEV) for a in (q, k, v))
    ws = K.decode_attn_workspace(n_head, n_kv, hd, cap, DEV)
    pos = torch.zeros(1, dtype=torch.int64, device=DEV)
    out = torch.empty(n_head, hd, device=DEV)
    for S in (5, cap - 1, 64, 129, cap):
        pos.fill_(S - 1)
        K.decode_attn(Q, Kc, Vc, S=pos, S_offset=1, workspace=ws, out=out)
        assert rel_err(out.cpu().numpy(), closed.attention(q, k, v, S)) < TOL
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        K.decode_attn(Q, Kc, Vc, S=pos, S_offset=1, workspace=ws, out=out)
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(g):
        K.decode_attn(Q, Kc, Vc, S=pos, S_offset=1, workspace=ws, out=out)
    for S in (1, 200, 64, cap, 65):
        pos.fill_(S - 1)
        g.replay()
        torch.cuda.synchronize()
        graph_out = out.clone()
        eager = K.decode_attn(Q, Kc, Vc, S=pos, S_offset=1, workspace=ws)
        assert torch.equal(graph_out, eager)
        assert rel_err(graph_out.cpu().numpy(), closed.attention(q, k, v, S)) < TOL


@pytest.mark.parametrize("L,pos0,hd", [(1, 0, 64), (13, 0, 64), (40, 5, 64), (300, 0, 64), (9, 0, 128)])
def test_prefill_attn(K, L, pos0, hd):
    rng = np.random.default_rng(L)
    n_head, n_kv, cap = (14, 2, pos0 + L + 3) if hd == 64 else (28, 4, pos0 + L)
    q = rng.standard_normal((L, n_head, hd)).astype(np.float32)
    k, v = _kv(rng, n_kv, cap, hd)
    out = K.prefill_attn(torch.from_numpy(q).to(DEV), torch.from_numpy(k).to(DEV),
                         torch.from_numpy(v).to(DEV), pos0=pos0).cpu().numpy()
    ref = closed.causal_attention(q, k, v, pos0).reshape(L, n_head * hd)
    assert rel_err(out, ref) < TOL


# ---- element-wise (reference tests/test_kernels.py:16-70) ---------------------------------

@pytest.mark.parametrize("L", [1, 5])
def test_rmsnorm(K, L):
    rng = np.random.default_rng(L)
    x = rng.standard_normal((L, 896)).astype(np.float32)
    w = rng.standard_normal(896).astype(np.float32)
    out = K.rmsnorm(torch.from_numpy(x).to(DEV), torch.from_numpy(w).to(DEV), 1e-6).cpu().numpy()
    assert np.abs(out - closed.rmsnorm(x, w, 1e-6)).max() < 1e-5


def test_rope_contiguous_and_strided_view(K):
    """The reference's non-contiguous prefill regression (test_kernels.py:40-59)."""
    rng = np.random.default_rng(0)
    L, nh, nkv, hd = 5, 14, 2, 64
    qkv = torch.from_numpy(rng.standard_normal((L, nh * hd + 2 * nkv * hd)).astype(np.float32)).to(DEV)
    q, k, _ = qkv.split([nh * hd, nkv * hd, nkv * hd], dim=-1)
    q, k = q.view(L, nh, hd), k.view(L, nkv, hd)
    assert not q.is_contiguous()
    c = rng.standard_normal((L, hd // 2)).astype(np.float32)
    s = rng.standard_normal((L, hd // 2)).astype(np.float32)
    C, S = torch.from_numpy(c).to(DEV), torch.from_numpy(s).to(DEV)
    for x in (q, k, q.contiguous()):
        ref = closed.rope(x.cpu().numpy(), c[:, None, :], s[:, None, :])
        assert np.abs(K.rope(x, C, S).cpu().numpy() - ref).max() < 1e-5


@pytest.mark.parametrize("L", [1, 5])
def test_silu_mul(K, L):
    gu = np.random.default_rng(L).standard_normal((L, 2 * 4864)).astype(np.float32)
    out = K.silu_mul(torch.from_numpy(gu).to(DEV), 4864).cpu().numpy()
    assert np.abs(out - closed.silu_mul(gu[:, :4864], gu[:, 4864:])).max() < 1e-4


def test_kv_write(K):
    rng = np.random.default_rng(3)
    L, nkv, hd, cap = 7, 2, 64, 20
    kk = rng.standard_normal((L, nkv, hd)).astype(np.float32)
    vv = rng.standard_normal((L, nkv, hd)).astype(np.float32)
    kc = torch.zeros(nkv, cap, hd, device=DEV)
    vc = torch.zeros(nkv, cap, hd, device=DEV)
    K.kv_write(torch.from_numpy(kk).to(DEV), torch.from_numpy(vv).to(DEV), kc, vc, pos0=4)
    kc, vc = kc.cpu().numpy(), vc.cpu().numpy()
    np.testing.assert_array_equal(kc[:, 4:11], kk.transpose(1, 0, 2))
    np.testing.assert_array_equal(vc[:, 4:11], vv.transpose(1, 0, 2))
    assert not kc[:, :4].any() and not kc[:, 11:].any()


# ---- fused QKV prologue -------------------------------------------------------------------

# The 0.5B shapes (one row pair per 32-lane group) and the 7B shape (hidden 3584, 128-lane
# groups) and hidden 2048 (64-lane groups), in both activation layouts; one without biases.
@pytest.mark.parametrize("types,hidden,nh,nkv,hd,ut,bias", [
    ((dq.Q5_0, dq.Q5_0, dq.Q8_0), 896, 14, 2, 64, False, True),
    ((dq.Q5_0, dq.Q5_0, dq.Q5_0), 896, 14, 2, 64, True, True),
    ((dq.Q4_K, dq.Q4_K, dq.Q6_K), 3584, 28, 4, 128, False, True),
    ((dq.Q4_K, dq.Q4_K, dq.Q6_K), 3584, 28, 4, 128, True, True),
    ((dq.Q5_0, dq.Q8_0, dq.Q8_0), 2048, 32, 8, 64, True, False),
])
def test_qkv_rmsnorm_rope(K, types, hidden, nh, nkv, hd, ut, bias):
    rng = np.random.default_rng(hidden)
    cap, pos, theta = 40, 23, 1e6
    rows = (nh * hd, nkv * hd, nkv * hd)
    raws = [quantized_normal(t, r, hidden, seed=i + 1) for i, (t, r) in enumerate(zip(types, rows))]
    ws = [qweight(K, t, raw, r, hidden) for t, raw, r in zip(types, raws, rows)]
    bs = [rng.standard_normal(r).astype(np.float32) * 0.1 for r in rows]
    x = rng.standard_normal(hidden).astype(np.float32)
    nw = rng.standard_normal(hidden).astype(np.float32)
    inv = 1.0 / (theta ** (np.arange(0, hd, 2) / hd))
    ang = (np.arange(64)[:, None] * inv[None, :]).astype(np.float32)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    kc = torch.zeros(nkv, cap, hd, device=DEV)
    vc = torch.zeros(nkv, cap, hd, device=DEV)
    T = lambda a: torch.from_numpy(a).to(DEV)
    xin, nin = (K.to_ut(T(x)), K.to_ut(T(nw))) if ut else (T(x), T(nw))
    dbias = [T(b) for b in bs] if bias else [None, None, None]
    q = K.qkv_rmsnorm_rope(xin, nin, 1e-6, *ws, *dbias, T(cos), T(sin), torch.tensor([pos], device=DEV),
                           kc, vc, nh, layout=K.LAYOUT_X_UT if ut else K.LAYOUT_NATURAL).cpu().numpy()
    if not bias:
        bs = [None, None, None]
    h = closed.rmsnorm(x, nw, 1e-6)
    outs = [closed.gemv(dequant_rows(t, raw, r, hidden), h, bias=b)
            for t, raw, r, b in zip(types, raws, rows, bs)]
    rq = closed.rope(outs[0].reshape(nh, hd), cos[pos], sin[pos])
    rk = closed.rope(outs[1].reshape(nkv, hd), cos[pos], sin[pos])
    assert rel_err(q, rq) < TOL
    kc, vc = kc.cpu().numpy(), vc.cpu().numpy()
    assert rel_err(kc[:, pos], rk) < TOL
    assert rel_err(vc[:, pos], outs[2].reshape(nkv, hd)) < TOL
    kc[:, pos] = 0
    vc[:, pos] = 0
    assert not kc.any() and not vc.any()  # nothing else written


# ---- unit-transposed activation layout (the decode path's vectors) ------------------------

@pytest.mark.parametrize("t,k,n", [(dq.Q5_0, 896, 896), (dq.Q6_K, 4864, 896), (dq.Q8_0, 896, 1152),
                                   (dq.Q4_K, 3584, 512)])
def test_qgemv_ut_layouts_match_natural(K, t, k, n):
    raw = quantized_normal(t, n, k, seed=k + 3 * n)
    w = qweight(K, t, raw, n, k)
    rng = np.random.default_rng(11)
    x = torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(DEV)
    r = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(DEV)
    nat = K.qgemv(x, w, residual=r)
    ut = K.qgemv(K.to_ut(x), w, residual=K.to_ut(r), layout=K.LAYOUT_X_UT | K.LAYOUT_Y_UT)
    assert rel_err(K.from_ut(ut).cpu().numpy(), nat.cpu().numpy()) < 1e-6
    xo = K.qgemv(K.to_ut(x), w, layout=K.LAYOUT_X_UT)          # ut in, natural out
    assert rel_err(xo.cpu().numpy(), closed.gemv(dequant_rows(t, raw, n, k), x.cpu().numpy())) < TOL


def test_norm_silu_and_lm_head_ut(K):
    rng = np.random.default_rng(12)
    k, ffn = 896, 4864
    raw = quantized_normal(dq.Q5_0, 2 * ffn, k, seed=77)
    w = qweight(K, dq.Q5_0, raw, 2 * ffn, k)
    x = torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(DEV)
    nw = torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(DEV)
    nat = K.qgemv_norm_silu(x, nw, w, 1e-6)
    ut = K.qgemv_norm_silu(K.to_ut(x), K.to_ut(nw), w, 1e-6, layout=K.LAYOUT_X_UT | K.LAYOUT_Y_UT)
    assert rel_err(K.from_ut(ut).cpu().numpy(), nat.cpu().numpy()) < 1e-5
    rawo = quantized_normal(dq.Q8_0, 4096, k, seed=78)
    wo = qweight(K, dq.Q8_0, rawo, 4096, k)
    a = K.qgemv_norm(x, nw, wo, 1e-6)
    b = K.qgemv_norm(K.to_ut(x), K.to_ut(nw), wo, 1e-6, layout=K.LAYOUT_X_UT)
    assert rel_err(b.cpu().numpy(), a.cpu().numpy()) < 1e-5


def test_embed_and_attention_ut_outputs(K):
    raw = random_quant(dq.Q8_0, 20, 896, seed=4)
    table = K.RawTensor(dev_bytes(raw), dq.Q8_0, (20, 896))
    ids = torch.tensor([3, 19], device=DEV)
    nat = K.embed_gather(table, ids)
    ut = K.embed_gather(table, ids, layout=K.LAYOUT_Y_UT)
    for r in range(2):
        assert torch.equal(K.from_ut(ut[r]), nat[r])
    rng = np.random.default_rng(5)
    q = torch.from_numpy(rng.standard_normal((14, 64)).astype(np.float32)).to(DEV)
    kc = torch.from_numpy(rng.standard_normal((2, 2000, 64)).astype(np.float32)).to(DEV)
    vc = torch.from_numpy(rng.standard_normal((2, 2000, 64)).astype(np.float32)).to(DEV)
    for cap, S in ((100, 77), (2000, 1500)):   # single-pass and split kernels
        a = K.decode_attn(q, kc[:, :cap].contiguous(), vc[:, :cap].contiguous(), S=S)
        b = K.decode_attn(q, kc[:, :cap].contiguous(), vc[:, :cap].contiguous(), S=S, layout=K.LAYOUT_Y_UT)
        assert torch.equal(K.from_ut(b.reshape(-1)), a.reshape(-1))


# ---- device-side greedy pick (LM head + argmax) -------------------------------------------

def _const_rows_q8(vals, k):
    """Q8_0 rows whose weights are all vals[r] (exactly representable: d = vals[r] / 127)."""
    from pico_hip.quantize import quantize
    W = np.repeat(np.asarray(vals, np.float32)[:, None], k, axis=1)
    return quantize(dq.Q8_0, W)


# (Q8_0, 3584, 20000): rows of 112 units on a launch large enough for the looped form
@pytest.mark.parametrize("t,k,n", [(dq.Q8_0, 896, 151936), (dq.Q5_0, 896, 1000), (dq.Q6_K, 4864, 300),
                                   (dq.Q8_0, 896, 1), (dq.Q8_0, 3584, 20000)])
def test_argmax_matches_torch_argmax(K, t, k, n):
    raw = quantized_normal(t, n, k, seed=n + t)
    w = qweight(K, t, raw, n, k)
    rng = np.random.default_rng(n)
    x = torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(DEV)
    nw = torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(DEV)
    g = K.GreedyState(n, 4, DEV)
    g.reset(7, 41, 0)
    logits = K.qgemv_norm_argmax(x, nw, w, 1e-6, g)
    ref = K.qgemv_norm(x, nw, w, 1e-6)
    assert torch.equal(logits, ref)          # same logits as the plain LM head
    want = int(torch.argmax(ref))
    st = g.state.tolist()
    assert st == [want, 42, 1]
    assert int(g.log[0]) == want


def test_argmax_ties_nan_and_state_chain(K):
    """Lowest row wins among equal maxima (torch.argmax), NaN beats numbers, the state
    advances over consecutive calls and the log stops at its capacity."""
    k, n = 896, 20000
    vals = np.linspace(-0.5, 0.4, n).astype(np.float32)
    vals[[1234, 5678, 19999]] = 0.9                      # three tied maxima
    w = K.pack_weight(dev_bytes(_const_rows_q8(vals, k)), dq.Q8_0, n, k)
    x = torch.ones(k, device=DEV)
    nw = torch.ones(k, device=DEV)
    g = K.GreedyState(n, 2, DEV)
    g.reset(0, 5, 0)
    for step in range(3):
        logits = K.qgemv_norm_argmax(x, nw, w, 1e-6, g)
        assert int(torch.argmax(logits)) == 1234
        assert g.state.tolist() == [1234, 6 + step, step + 1]
    assert g.log.tolist() == [1234, 1234]                # capacity 2: the third pick is not logged
    xn = x.clone()
    xn[3] = float("nan")                                 # every logit NaN -> row 0 (first NaN)
    K.qgemv_norm_argmax(xn, nw, w, 1e-6, g)
    assert int(g.state[0]) == 0
    neg = torch.full((k,), -1.0, device=DEV)             # all logits negative: argmax = min |vals|
    logits = K.qgemv_norm_argmax(neg, nw, w, 1e-6, g)
    assert int(g.state[0]) == int(torch.argmax(logits))


def test_argmax_in_graph_replays(K):
    n, k = 151936, 896
    raw = quantized_normal(dq.Q8_0, n, k, seed=5)
    w = qweight(K, dq.Q8_0, raw, n, k)
    rng = np.random.default_rng(3)
    xs = [torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(DEV) for _ in range(4)]
    nw = torch.ones(k, device=DEV)
    x = xs[0].clone()
    g = K.GreedyState(n, 8, DEV)
    g.reset(0, 0, 0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        K.qgemv_norm_argmax(x, nw, w, 1e-6, g)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = K.qgemv_norm_argmax(x, nw, w, 1e-6, g)
    g.reset(0, 100, 0)
    want = []
    for xi in xs:
        x.copy_(xi)
        graph.replay()
        torch.cuda.synchronize()
        want.append(int(torch.argmax(K.qgemv_norm(xi, nw, w, 1e-6))))
        assert int(torch.argmax(out)) == want[-1]
    assert g.log[:4].tolist() == want
    assert g.state.tolist() == [want[-1], 104, 4]


@pytest.mark.parametrize("n", [14, 5, 4, 2, 1])
def test_qgemv_sum_rmsnorm_silu(K, n):
    """silu(g) * u of rmsnorm(x + sum of parts); the stored sum equals the float32 sum taken
    in part order, bit for bit. Up to 4 parts are loaded with x, more after the weights."""
    t, k, ffn = dq.Q5_0, 896, 4864
    raw = quantized_normal(t, 2 * ffn, k, seed=31)
    w = qweight(K, t, raw, 2 * ffn, k)
    rng = np.random.default_rng(31)
    x = rng.standard_normal(k).astype(np.float32)
    parts = (rng.standard_normal((n, k)) * 0.3).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    T = lambda a: torch.from_numpy(a).to(DEV)
    act, xs = K.qgemv_sum_norm_silu(T(x), T(parts), T(nw), w, 1e-6)
    want = x.copy()
    for p in parts:
        want = (want + p).astype(np.float32)
    np.testing.assert_array_equal(xs.cpu().numpy(), want)
    Wd = dequant_rows(t, raw, 2 * ffn, k)
    h = closed.rmsnorm(want, nw, 1e-6)
    ref = closed.silu_mul(closed.gemv(Wd[:ffn], h), closed.gemv(Wd[ffn:], h))
    assert rel_err(act.cpu().numpy(), ref) < TOL
    # no parts: the plain fused gate/up
    plain = K.qgemv_norm_silu(T(want), T(nw), w, 1e-6)
    act0, _ = K.qgemv_sum_norm_silu(T(want), T(parts[:0].copy()), T(nw), w, 1e-6)
    assert torch.equal(plain, act0)
    # unit-transposed x, parts, norm weight and sum, unit-transposed act: the same sum, and the
    # plain fused gate/up of that sum in the same layout bit for bit (the RMSNorm sum of
    # squares is reduced in a layout-dependent order, so only to rounding across layouts)
    UT = K.LAYOUT_X_UT | K.LAYOUT_Y_UT
    pu = torch.stack([K.to_ut(T(pp)) for pp in parts])
    act_u, xs_u = K.qgemv_sum_norm_silu(K.to_ut(T(x)), pu, K.to_ut(T(nw)), w, 1e-6, layout=UT)
    assert torch.equal(K.from_ut(xs_u), xs)
    assert torch.equal(act_u, K.qgemv_norm_silu(K.to_ut(T(want)), K.to_ut(T(nw)), w, 1e-6, layout=UT))
    assert rel_err(K.from_ut(act_u).cpu().numpy(), act.cpu().numpy()) < 1e-6


# ---- attention of a kv group + its o-projection share in one launch (attn_gproj) -----------

GPROJ_CASES = [
    (dq.Q5_0, 14, 2, 77, [1, 17, 61, 64, 65, 77]),   # config 0 shapes, both 64-position passes
    (dq.Q5_0, 14, 2, 128, [127, 128]),               # largest cache
    (dq.Q8_0, 8, 1, 64, [3, 40]),                    # MQA: one group of 8 query heads
    (dq.Q4_K, 8, 2, 100, [33, 100]),                 # K-quant o-projection (512 columns)
    (dq.Q6_K, 16, 4, 50, [7, 50]),                   # four groups (four parts)
]


@pytest.mark.parametrize("t,nh,nkv,cap,Ss", GPROJ_CASES,
                         ids=[f"t{t}-{nh}x{nkv}-cap{cap}" for t, nh, nkv, cap, _ in GPROJ_CASES])
def test_attn_gproj_matches_closed_form(K, t, nh, nkv, cap, Ss):
    """Part j = Wo[:, columns of group j] . attention of group j's heads; x + the parts in
    order is the o-projection with its residual."""
    hd, hidden = 64, 896
    rng = np.random.default_rng(nh * cap + t + 7)
    q = rng.standard_normal((nh, hd)).astype(np.float32)
    k, v = _kv(rng, nkv, cap, hd)
    x = rng.standard_normal(hidden).astype(np.float32)
    raw = quantized_normal(t, hidden, nh * hd, seed=cap + t)
    wo = qweight(K, t, raw, hidden, nh * hd)
    W = dequant_rows(t, raw, hidden, nh * hd)
    T = lambda a: torch.from_numpy(a).to(DEV)
    G = nh // nkv
    assert K.attn_gproj_supported(nh, nkv, hd, cap, wo)
    for S in Ss:
        parts = K.attn_gproj(T(q), T(k), T(v), wo, S=torch.tensor([S - 1], device=DEV),
                             S_offset=1).cpu().numpy()
        assert parts.shape == (nkv, hidden)
        attn = closed.attention(q, k, v, S, round_fp16=True).reshape(-1)
        for j in range(nkv):
            cols = slice(j * G * hd, (j + 1) * G * hd)
            assert rel_err(parts[j], closed.gemv(W[:, cols], attn[cols])) < TOL, f"S={S} j={j}"
        y = x.copy()
        for pp in parts:
            y = (y + pp).astype(np.float32)
        assert rel_err(y, closed.gemv(W, attn, residual=x)) < TOL, f"S={S}"


def test_attn_gproj_layout_empty_and_limits(K):
    hd, nh, nkv, cap, hidden = 64, 14, 2, 77, 896
    rng = np.random.default_rng(6)
    q = torch.from_numpy(rng.standard_normal((nh, hd)).astype(np.float32)).to(DEV)
    k, v = (torch.from_numpy(a).to(DEV) for a in _kv(rng, nkv, cap, hd))
    wo = qweight(K, dq.Q5_0, quantized_normal(dq.Q5_0, hidden, nh * hd, seed=6), hidden, nh * hd)
    nat = K.attn_gproj(q, k, v, wo, S=40)
    ut = K.attn_gproj(q, k, v, wo, S=40, layout=K.LAYOUT_Y_UT)
    for j in range(nkv):
        assert torch.equal(K.from_ut(ut[j]), nat[j])
    # the same attention as decode_attn, whatever the o-projection split
    a2 = K.decode_attn(q, k, v, S=40)
    y2 = K.qgemv(a2.reshape(-1), wo)
    assert rel_err(nat.sum(0).cpu().numpy(), y2.cpu().numpy()) < TOL
    assert torch.isnan(K.attn_gproj(q, k, v, wo, S=0)).all()
    assert not K.attn_gproj_supported(nh, nkv, 128, cap, wo)      # head_dim 128
    assert not K.attn_gproj_supported(nh, nkv, hd, 129, wo)       # capacity past 128
    assert not K.attn_gproj_supported(28, 2, hd, cap, wo)         # 14 query heads per group
    assert not K.attn_gproj_supported(10, 5, hd, cap, wo)         # 5 kv heads


# attn_split_gproj: the split attention's records merged per kv group with that group's Wo
# columns (long caches; any capacity)
SPLIT_GPROJ_CASES = [
    (dq.Q5_0, 14, 2, 2048, [1, 64, 65, 1000, 2047, 2048]),  # config 3 heads: one chunk, ragged, full
    (dq.Q5_0, 14, 2, 8200, [8193, 8200]),                   # config 3 decode context
    (dq.Q8_0, 8, 1, 1500, [3, 1500]),                       # MQA: one group of 8 query heads
    (dq.Q4_K, 8, 2, 1100, [700, 1100]),                     # K-quant o-projection (512 columns)
    (dq.Q6_K, 16, 4, 300, [129, 300]),                      # four groups (four parts)
]


@pytest.mark.parametrize("t,nh,nkv,cap,Ss", SPLIT_GPROJ_CASES,
                         ids=[f"t{t}-{nh}x{nkv}-cap{cap}" for t, nh, nkv, cap, _ in SPLIT_GPROJ_CASES])
def test_attn_split_gproj_matches_closed_form(K, t, nh, nkv, cap, Ss):
    """Part j = Wo[:, columns of group j] . attention of group j's heads over S positions of a
    long cache (fp16-rounded attention output); x + the parts in order is the o-projection
    with its residual."""
    hd, hidden = 64, 896
    rng = np.random.default_rng(nh * cap + t + 11)
    q = rng.standard_normal((nh, hd)).astype(np.float32)
    k, v = _kv(rng, nkv, cap, hd)
    x = rng.standard_normal(hidden).astype(np.float32)
    raw = quantized_normal(t, hidden, nh * hd, seed=cap + t + 1)
    wo = qweight(K, t, raw, hidden, nh * hd)
    W = dequant_rows(t, raw, hidden, nh * hd)
    T = lambda a: torch.from_numpy(a).to(DEV)
    G = nh // nkv
    assert K.attn_split_gproj_supported(nh, nkv, hd, cap, wo)
    ws = K.decode_attn_workspace(nh, nkv, hd, cap, DEV)
    kd, vd = T(k), T(v)
    for S in Ss:
        parts = K.attn_split_gproj(T(q), kd, vd, wo, S=torch.tensor([S - 1], device=DEV), S_offset=1,
                                   workspace=ws).cpu().numpy()
        assert parts.shape == (nkv, hidden)
        attn = closed.attention(q, k, v, S, round_fp16=True).reshape(-1)
        for j in range(nkv):
            cols = slice(j * G * hd, (j + 1) * G * hd)
            assert rel_err(parts[j], closed.gemv(W[:, cols], attn[cols])) < TOL, f"S={S} j={j}"
        y = x.copy()
        for pp in parts:
            y = (y + pp).astype(np.float32)
        assert rel_err(y, closed.gemv(W, attn, residual=x)) < TOL, f"S={S}"


def test_attn_split_gproj_layout_empty_and_limits(K):
    """Unit-transposed parts equal the natural ones; the same attention as decode_attn + the
    o-projection GEMV; S = 0 gives NaN; shape limits."""
    hd, nh, nkv, cap, hidden = 64, 14, 2, 3000, 896
    rng = np.random.default_rng(16)
    q = torch.from_numpy(rng.standard_normal((nh, hd)).astype(np.float32)).to(DEV)
    k, v = (torch.from_numpy(a).to(DEV) for a in _kv(rng, nkv, cap, hd))
    wo = qweight(K, dq.Q5_0, quantized_normal(dq.Q5_0, hidden, nh * hd, seed=16), hidden, nh * hd)
    ws = K.decode_attn_workspace(nh, nkv, hd, cap, DEV)
    nat = K.attn_split_gproj(q, k, v, wo, S=2500, workspace=ws)
    ut = K.attn_split_gproj(q, k, v, wo, S=2500, workspace=ws, layout=K.LAYOUT_Y_UT)
    for j in range(nkv):
        assert torch.equal(K.from_ut(ut[j]), nat[j])
    a2 = K.decode_attn(q, k, v, S=2500, workspace=ws)
    y2 = K.qgemv(a2.reshape(-1), wo)
    assert rel_err(nat.sum(0).cpu().numpy(), y2.cpu().numpy()) < TOL
    assert torch.isnan(K.attn_split_gproj(q, k, v, wo, S=0, workspace=ws)).all()
    assert not K.attn_split_gproj_supported(nh, nkv, 128, cap, wo)   # head_dim 128
    assert not K.attn_split_gproj_supported(28, 2, hd, cap, wo)      # 14 query heads per group
    small = torch.zeros(64, dtype=torch.uint8, device=DEV)
    with pytest.raises(RuntimeError):
        K.attn_split_gproj(q, k, v, wo, S=10, workspace=small)       # workspace too small


# ---- prompt-prefill GEMM on the matrix cores (fp16 operands, fp32 accumulate) --------------

@pytest.mark.parametrize("t,n,k", [(dq.Q5_0, 96, 896), (dq.Q8_0, 64, 896), (dq.Q4_K, 40, 4864),
                                   (dq.Q6_K, 40, 4864)])
def test_dequant_tiled_f16_is_rounded_exact_value(K, t, n, k):
    """fp16 weights = the exact dequantized value rounded to nearest even, bit for bit."""
    raw = random_quant(t, n, k, seed=n + k + t + 1)
    w = qweight(K, t, raw, n, k)
    gpu = K.dequantize_weight_f16(w).cpu().numpy()
    ref = dequant_rows(t, raw, n, k).astype(np.float16)
    np.testing.assert_array_equal(gpu.view(np.uint16), ref.view(np.uint16))


GEMM16_CASES = [  # (M, N, K, bias, residual, a_row_stride_extra)
    (1, 128, 896, False, False, 0), (13, 1152, 896, True, False, 0), (128, 896, 896, False, True, 0),
    (300, 9728, 896, False, False, 0), (257, 896, 4864, False, True, 0), (77, 200, 96, True, True, 32),
    (8192, 1152, 896, True, False, 0),
    # 256 x 128 workgroup tiles (>= 512 of them), ragged edges included
    (4096, 4096, 96, True, True, 0), (4000, 4000, 64, False, False, 32),
    # 64 x 128 workgroup tiles (the 128 x 128 grid would have < 512 workgroups)
    (8192, 896, 256, False, True, 0), (4100, 1000, 64, True, False, 0),
]


@pytest.mark.parametrize("M,N,Kd,bias,res,extra", GEMM16_CASES)
def test_gemm_f16_matches_fp16_operand_reference(K, M, N, Kd, bias, res, extra):
    """C = A W^T (+ bias) (+ residual) against float64 on the same fp16-rounded operands
    (fp32 accumulation: only the summation order differs)."""
    rng = np.random.default_rng(M + N + Kd)
    a = rng.standard_normal((M, Kd + extra)).astype(np.float32)
    w16 = (rng.standard_normal((N, Kd)) * 0.05).astype(np.float16)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    r = rng.standard_normal((M, N)).astype(np.float32) if res else None
    T = lambda v: None if v is None else torch.from_numpy(v).to(DEV)
    A = T(a)[:, :Kd]  # row stride Kd + extra
    c = K.gemm_f16(A, T(w16), bias=T(b), residual=T(r)).cpu().numpy()
    ref = a[:, :Kd].astype(np.float16).astype(np.float64) @ w16.astype(np.float64).T
    if b is not None:
        ref = ref + b
    if r is not None:
        ref = ref + r
    assert c.shape == (M, N)
    assert rel_err(c, ref) < 1e-5


LT_CASES = [  # (M, N, K, bias, residual, a_row_stride_extra): the config-3 prefill products + edges
    (1, 128, 896, False, False, 0), (13, 1152, 896, True, False, 0), (128, 896, 896, False, True, 0),
    (257, 896, 4864, False, True, 0), (77, 200, 96, True, True, 32), (8192, 1152, 896, True, False, 0),
    (8192, 896, 896, False, True, 0), (8192, 896, 4864, False, True, 0),
]


@pytest.mark.parametrize("M,N,Kd,bias,res,extra", LT_CASES)
def test_gemm_lt_matches_fp16_operand_reference(K, M, N, Kd, bias, res, extra):
    """pe_gemm_lt (hipBLASLt) against float64 on the same fp16 operands (fp32 accumulation:
    only the summation order differs), with the bias, the residual, and the residual added in
    place (residual == out); a strided A included."""
    rng = np.random.default_rng(M + N + Kd + 7)
    a = rng.standard_normal((M, Kd + extra)).astype(np.float16)
    w16 = (rng.standard_normal((N, Kd)) * 0.05).astype(np.float16)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    r = rng.standard_normal((M, N)).astype(np.float32) if res else None
    T = lambda v: None if v is None else torch.from_numpy(v).to(DEV)
    A = T(a)[:, :Kd]
    ws = K.gemm_lt_workspace(DEV)
    c = K.gemm_lt(A, T(w16), bias=T(b), residual=T(r), workspace=ws).cpu().numpy()
    ref = a[:, :Kd].astype(np.float64) @ w16.astype(np.float64).T
    if b is not None:
        ref = ref + b
    if r is not None:
        ref = ref + r
    assert c.shape == (M, N)
    assert rel_err(c, ref) < 1e-5
    if res:
        x = T(r)
        K.gemm_lt(A, T(w16), bias=T(b), residual=x, out=x, workspace=ws)
        assert rel_err(x.cpu().numpy(), ref) < 1e-5


def _rmsnorm_f32_emulated(x, w, eps):
    """The device row norm's float32 arithmetic in its order: thread t = 64 w + l of a 256-wide
    row sweep sums x[t + 256 j]^2 over j ascending; each wave's partials are added by the DPP /
    permlane butterfly (partner lanes l^1, l^2, the half-row mirror, the row mirror, l^16, l^32;
    every lane ends with the same bits), the four wave sums in wave order; rstd by IEEE division
    and square root."""
    f32 = np.float32
    n = x.shape[0]
    waves = []
    for wv in range(4):
        part = np.zeros(64, f32)
        for ln in range(64):
            acc = f32(0)
            for i in range(64 * wv + ln, n, 256):
                acc = f32(acc + f32(x[i] * x[i]))
            part[ln] = acc
        lanes = np.arange(64)
        for p in (lanes ^ 1, lanes ^ 2, (lanes & ~7) | (7 - (lanes & 7)), (lanes & ~15) | (15 - (lanes & 15)),
                  lanes ^ 16, lanes ^ 32):
            part = (part + part[p]).astype(f32)
        waves.append(part[0])
    tot = f32(f32(f32(waves[0] + waves[1]) + waves[2]) + waves[3])
    rstd = f32(f32(1) / np.sqrt(f32(f32(tot / f32(n)) + f32(eps))))
    return ((x * rstd).astype(f32) * w).astype(f32)


@pytest.mark.parametrize("n", [64, 896, 1000, 3584, 4096, 5000])
def test_rmsnorm_bits_follow_the_summation_order(K, n):
    """Both row-norm kernels (one wave per row up to 4096 elements, one workgroup per row
    beyond) give the bits of the float32 emulation of their common summation order, in fp32
    and rounded to fp16."""
    rng = np.random.default_rng(n)
    x = rng.standard_normal((3, n)).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    X, Wt = torch.from_numpy(x).to(DEV), torch.from_numpy(w).to(DEV)
    got32 = K.rmsnorm(X, Wt, 1e-6).cpu().numpy()
    got16 = K.rmsnorm(X, Wt, 1e-6, half=True).cpu().numpy()
    for r in range(3):
        want = _rmsnorm_f32_emulated(x[r], w, 1e-6)
        np.testing.assert_array_equal(got32[r].view(np.uint32), want.view(np.uint32))
        np.testing.assert_array_equal(got16[r].view(np.uint16), want.astype(np.float16).view(np.uint16))


def test_rmsnorm_and_flash_half_outputs_are_rounded_fp32_outputs(K):
    """pe_rmsnorm_h16 and pe_flash_prefill_h16 store the fp32 kernels' values rounded to fp16
    (nearest even), bit for bit: the operands the prefill GEMMs would round as they read them."""
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal((300, 896)).astype(np.float32)).to(DEV)
    w = torch.from_numpy(rng.standard_normal(896).astype(np.float32)).to(DEV)
    h16 = K.rmsnorm(x, w, 1e-6, half=True)
    assert h16.dtype == torch.float16
    assert torch.equal(h16, K.rmsnorm(x, w, 1e-6).half())
    L, nh, nkv, hd = 300, 14, 2, 64
    q = torch.from_numpy(rng.standard_normal((L, nh, hd)).astype(np.float32)).to(DEV)
    kc = torch.from_numpy(rng.standard_normal((nkv, L + 5, hd)).astype(np.float32)).to(DEV)
    vc = torch.from_numpy(rng.standard_normal((nkv, L + 5, hd)).astype(np.float32)).to(DEV)
    o16 = K.flash_prefill(q, kc, vc, half=True)
    assert o16.dtype == torch.float16
    assert torch.equal(o16, K.flash_prefill(q, kc, vc).half())


@pytest.mark.parametrize("M,ffn,Kd", [(300, 4864, 896), (13, 512, 3584), (129, 48, 96), (1, 16, 32),
                                      (4096, 2048, 64)])
def test_gemm_f16_silu_equals_gemm_then_silu(K, M, ffn, Kd):
    """The SiLU-fused gate/up GEMM (interleaved rows) gives silu_mul(gemm_f16(A, [gate; up]))
    bit for bit: the same MFMA accumulation per column and the same SiLU formula."""
    rng = np.random.default_rng(M + ffn)
    a = torch.from_numpy(rng.standard_normal((M, Kd)).astype(np.float32)).to(DEV)
    w16 = torch.from_numpy((rng.standard_normal((2 * ffn, Kd)) * 0.05).astype(np.float16)).to(DEV)
    ref = K.silu_mul(K.gemm_f16(a, w16), ffn)
    got = K.gemm_f16_silu(a, K.interleave_gate_up_f16(w16))
    assert got.shape == (M, ffn)
    assert torch.equal(got, ref)


@pytest.mark.parametrize("M,N,Kd,bias,res,extra", GEMM16_CASES)
def test_gemm_h16_equals_gemm_f16_on_fp16_values(K, M, N, Kd, bias, res, extra):
    """pe_gemm_h16 (A stored in fp16) gives pe_gemm_f16's bits on the same values: A rounded to
    fp16 before or as it is read is the same operand (row strides with padding included)."""
    rng = np.random.default_rng(M + N + Kd + 1)
    a = rng.standard_normal((M, Kd + extra)).astype(np.float16)
    w16 = (rng.standard_normal((N, Kd)) * 0.05).astype(np.float16)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    r = rng.standard_normal((M, N)).astype(np.float32) if res else None
    T = lambda v: None if v is None else torch.from_numpy(v).to(DEV)
    A16 = T(a)[:, :Kd]  # fp16, row stride Kd + extra
    ref = K.gemm_f16(A16.float(), T(w16), bias=T(b), residual=T(r))
    got = K.gemm_f16(A16, T(w16), bias=T(b), residual=T(r))
    assert torch.equal(got, ref)


@pytest.mark.parametrize("M,N,Kd,bias,res,extra", [
    (8192, 896, 4864, False, True, 0), (8192, 896, 896, False, True, 0), (8192, 1152, 896, True, False, 0),
    (1100, 160, 128, True, True, 64), (1024, 4000, 64, False, True, 0), (2049, 896, 896, True, True, 0),
    (1023, 896, 896, False, True, 0)])
def test_gemm_h16_long_prompt_kernel(K, M, N, Kd, bias, res, extra):
    """Products with M >= 1024, K % 64 == 0 and N % 16 == 0 run on pe_gemm_h16's direct-to-LDS
    kernel (256-row tiles, ragged M and N included; M = 1023 stays on the other kernel): the
    bits of the fp32-A kernel on the same fp16 values (the same MFMA accumulation order), also
    with the residual added in place (residual is out)."""
    rng = np.random.default_rng(M + N + Kd + 11)
    a = rng.standard_normal((M, Kd + extra)).astype(np.float16)
    w16 = (rng.standard_normal((N, Kd)) * 0.05).astype(np.float16)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    r = rng.standard_normal((M, N)).astype(np.float32) if res else None
    T = lambda v: None if v is None else torch.from_numpy(v).to(DEV)
    A16 = T(a)[:, :Kd]
    ref = K.gemm_f16(A16.float(), T(w16), bias=T(b), residual=T(r))
    got = K.gemm_f16(A16, T(w16), bias=T(b), residual=T(r))
    assert torch.equal(got, ref)
    if res:
        x = T(r)
        K.gemm_f16(A16, T(w16), bias=T(b), residual=x, out=x)
        assert torch.equal(x, ref)
    if M * N * Kd <= 2 ** 31:
        want = a[:, :Kd].astype(np.float64) @ w16.astype(np.float64).T
        if b is not None:
            want = want + b
        if r is not None:
            want = want + r
        assert rel_err(got.cpu().numpy(), want) < 1e-5


@pytest.mark.parametrize("M,ffn,Kd", [(300, 4864, 896), (13, 512, 3584), (129, 48, 96), (1, 16, 32),
                                      (4096, 2048, 64), (8192, 256, 64)])
def test_gemm_f16_silu_half_output_and_down_product(K, M, ffn, Kd):
    """The fp16-output SiLU GEMM stores the fp32 result rounded to nearest even, and the down
    product on it equals the fp32 path's (whose A is rounded the same way as it is read)."""
    rng = np.random.default_rng(M + ffn + 1)
    a = torch.from_numpy(rng.standard_normal((M, Kd)).astype(np.float32)).to(DEV)
    w16 = torch.from_numpy((rng.standard_normal((2 * ffn, Kd)) * 0.05).astype(np.float16)).to(DEV)
    wil = K.interleave_gate_up_f16(w16)
    act32 = K.gemm_f16_silu(a, wil)
    act16 = K.gemm_f16_silu(a, wil, half=True)
    assert act16.dtype == torch.float16 and act16.shape == (M, ffn)
    assert torch.equal(act16, act32.half())
    if ffn % 32:  # the down product's K must be a multiple of 32
        return
    wd = torch.from_numpy((rng.standard_normal((96, ffn)) * 0.05).astype(np.float16)).to(DEV)
    res = torch.from_numpy(rng.standard_normal((M, 96)).astype(np.float32)).to(DEV)
    assert torch.equal(K.gemm_f16(act16, wd, residual=res), K.gemm_f16(act32, wd, residual=res))


@pytest.mark.parametrize("M,ffn,Kd", [(300, 4864, 896), (13, 512, 3584), (129, 48, 96), (8192, 256, 64),
                                      (8192, 4864, 896), (1100, 48, 128), (2048, 1008, 64),
                                      (8000, 1008, 128), (7937, 16, 192), (9000, 2448, 896), (7936, 4864, 896)])
def test_gemm_h16_silu_equals_fp32_operand_path(K, M, ffn, Kd):
    """The SiLU GEMM on an fp16 A (pe_gemm_h16_silu_h) gives the bits of the fp32-A GEMM on the
    A those fp16 values came from (the fp32 path rounds A the same way as it reads it), and so
    does an fp16 A from rmsnorm(half=True) against the fp32 norm. From M = 7937 with K % 64 == 0
    and K >= 128 the fp16 product runs on the 256 x 256 tile kernel (ragged row and column tiles
    here, K at its minimum 128 and an odd multiple of 64), below that and for the fp32 A on the
    128 x 128 one."""
    rng = np.random.default_rng(M + ffn + 5)
    a = torch.from_numpy(rng.standard_normal((M, Kd)).astype(np.float32)).to(DEV)
    w16 = torch.from_numpy((rng.standard_normal((2 * ffn, Kd)) * 0.05).astype(np.float16)).to(DEV)
    wil = K.interleave_gate_up_f16(w16)
    assert torch.equal(K.gemm_f16_silu(a.half(), wil, half=True), K.gemm_f16_silu(a, wil, half=True))
    nw = torch.from_numpy(rng.standard_normal(Kd).astype(np.float32)).to(DEV)
    h32, h16 = K.rmsnorm(a, nw, 1e-6), K.rmsnorm(a, nw, 1e-6, half=True)
    assert torch.equal(K.gemm_f16_silu(h16, wil, half=True), K.gemm_f16_silu(h32, wil, half=True))
    with pytest.raises(ValueError):
        K.gemm_f16_silu(a.half(), wil)  # an fp16 A stores fp16 output


@pytest.mark.parametrize("L,nh,nkv,hd,pos0", [(1, 14, 2, 64, 0), (77, 14, 2, 64, 5), (300, 28, 4, 128, 0),
                                              (8, 4, 4, 64, 3)])
def test_rope_kv_write_equals_rope_then_kv_write(K, L, nh, nkv, hd, pos0):
    """One pass of RoPE on the q and k heads plus the cache write of k and v gives the bits of
    rope followed by kv_write; nothing else in the caches is touched."""
    rng = np.random.default_rng(L + nh + hd)
    cap = pos0 + L + 4
    qkv = torch.from_numpy(rng.standard_normal((L, (nh + 2 * nkv) * hd)).astype(np.float32)).to(DEV)
    ang = rng.standard_normal((L, hd // 2)).astype(np.float32)
    cos, sin = torch.from_numpy(np.cos(ang)).to(DEV), torch.from_numpy(np.sin(ang)).to(DEV)
    k1 = torch.full((nkv, cap, hd), 7.0, device=DEV)
    v1 = torch.full((nkv, cap, hd), 7.0, device=DEV)
    k2, v2 = k1.clone(), v1.clone()
    q = K.rope_kv_write(qkv, cos, sin, nh, k1, v1, pos0=pos0)
    qk = K.rope(qkv[:, :(nh + nkv) * hd].view(L, nh + nkv, hd), cos, sin)
    K.kv_write(qk[:, nh:], qkv[:, (nh + nkv) * hd:].view(L, nkv, hd), k2, v2, pos0=pos0)
    assert torch.equal(q, qk[:, :nh])
    assert torch.equal(k1, k2) and torch.equal(v1, v2)


def _kv16_layout_ref(k, v, length):
    """numpy restatement of the fp16 key blocks (pe_rope_kv_write_blocks): per kv head and
    64-key block, K [key][dim] then V^T [dim][key slot] as 64 rows of 8 chunks of 8 halves,
    chunk c of row r at chunk position c ^ (r & 7); slot 8 g + i of a 32-key slab holds key
    4 g + i (i < 4) or 16 + 4 g + (i - 4)."""
    n_kv, _, hd = k.shape
    nblk = (length + 63) // 64
    out = np.zeros((n_kv, nblk, 2, 64, 8, 8), np.float16)
    slot_key = np.zeros(64, np.int64)
    for key in range(64):
        kw = key % 32
        g, i = (kw // 4, kw % 4) if kw < 16 else ((kw - 16) // 4, 4 + (kw - 16) % 4)
        slot_key[32 * (key // 32) + 8 * g + i] = key
    for h in range(n_kv):
        for b in range(nblk):
            kb = np.zeros((64, 64), np.float16)
            vb = np.zeros((64, 64), np.float16)
            n = min(64, length - 64 * b)
            kb[:n] = k[h, 64 * b:64 * b + n].astype(np.float16)
            vb[:n] = v[h, 64 * b:64 * b + n].astype(np.float16)
            vt = vb[slot_key].T  # [dim][slot]
            for r in range(64):
                for c in range(8):
                    out[h, b, 0, r, c ^ (r & 7)] = kb[r, 8 * c:8 * c + 8]
                    out[h, b, 1, r, c ^ (r & 7)] = vt[r, 8 * c:8 * c + 8]
    return out.view(np.uint8).reshape(n_kv, nblk, 16384)


@pytest.mark.parametrize("splits", [(37, 100), (64, 64, 9), (1, 5, 130)])
def test_rope_kv_write_blocks_in_pieces(K, splits):
    """Key blocks written by several calls at increasing pos0 (blocks shared by two calls: the
    V^T chunks a call only partly covers keep the other call's keys) equal the numpy layout of
    the caches the calls wrote, and the fp32 caches equal one call over the whole prompt."""
    rng = np.random.default_rng(sum(splits))
    nh, nkv, hd = 14, 2, 64
    L = sum(splits)
    qkv = torch.from_numpy(rng.standard_normal((L, (nh + 2 * nkv) * hd)).astype(np.float32)).to(DEV)
    ang = rng.standard_normal((L, hd // 2)).astype(np.float32)
    cos, sin = torch.from_numpy(np.cos(ang)).to(DEV), torch.from_numpy(np.sin(ang)).to(DEV)
    k1, v1 = torch.zeros(nkv, L, hd, device=DEV), torch.zeros(nkv, L, hd, device=DEV)
    k2, v2 = k1.clone(), v1.clone()
    K.rope_kv_write(qkv, cos, sin, nh, k1, v1)
    kv16 = K.kv16_blocks(nkv, L, DEV)
    pos = 0
    for n in splits:
        K.rope_kv_write(qkv[pos:pos + n], cos[pos:pos + n], sin[pos:pos + n], nh, k2, v2, pos0=pos, kv16=kv16)
        pos += n
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    np.testing.assert_array_equal(kv16.cpu().numpy(), _kv16_layout_ref(k1.cpu().numpy(), v1.cpu().numpy(), L))


@pytest.mark.parametrize("L", [1, 64, 77, 300, 1000])
@pytest.mark.parametrize("n_head,n_kv", [(14, 2), (8, 8), (16, 1), (9, 3), (4, 2), (16, 2)])
def test_flash_prefill_blocks_equals_fp32_cache_path(K, L, n_head, n_kv):
    """The RoPE pass writing the fp16 key blocks (pe_rope_kv_write_blocks) leaves the caches and
    q as pe_rope_kv_write does and fills the blocks as the numpy restatement of their layout
    says; flash attention from the blocks (pe_flash_prefill_blocks: two 16-query tiles per wave,
    direct-to-LDS copies, q rounded after its scale * log2 e scaling) stays within 1e-3 relative
    of pe_flash_prefill_h16 on the fp32 caches (the two roundings of q), and up to 300 positions
    within 2e-3 of float64 attention on the fp16-rounded operands. Groups of 1,
    2 and 3 query heads per kv head put 4, 2 and 2 sets of 32 queries in a workgroup (waves
    whose unmasked prefixes differ), 7 the 0.5B model's shape, 8 and 16 the eight loading
    waves."""
    rng = np.random.default_rng(L + 31 * n_head + n_kv)
    hd, cap = 64, L + 5
    qkv = torch.from_numpy(rng.standard_normal((L, (n_head + 2 * n_kv) * hd)).astype(np.float32)).to(DEV)
    ang = rng.standard_normal((L, hd // 2)).astype(np.float32)
    cos, sin = torch.from_numpy(np.cos(ang)).to(DEV), torch.from_numpy(np.sin(ang)).to(DEV)
    k1, v1 = torch.zeros(n_kv, cap, hd, device=DEV), torch.zeros(n_kv, cap, hd, device=DEV)
    k2, v2 = k1.clone(), v1.clone()
    q1 = K.rope_kv_write(qkv, cos, sin, n_head, k1, v1)
    kv16 = K.kv16_blocks(n_kv, L, DEV)
    q2 = K.rope_kv_write(qkv, cos, sin, n_head, k2, v2, kv16=kv16)
    assert torch.equal(q1, q2) and torch.equal(k1, k2) and torch.equal(v1, v2)
    if L <= 300:
        want = _kv16_layout_ref(k1.cpu().numpy(), v1.cpu().numpy(), L)
        np.testing.assert_array_equal(kv16.cpu().numpy(), want)
    ref = K.flash_prefill(q1, k1, v1, half=True)
    got = K.flash_prefill_blocks(q2, kv16, split=False)
    assert rel_err(got.float().cpu().numpy(), ref.float().cpu().numpy()) < 1e-3
    if L <= 300:
        h16 = lambda t: t.cpu().numpy().astype(np.float16).astype(np.float32)
        want = closed.causal_attention(h16(q1), h16(k1), h16(v1), 0).reshape(L, n_head * hd)
        assert rel_err(got.float().cpu().numpy(), want) < 2e-3
    if L <= 4096:  # nothing to split: the default schedule is the same
        assert K.flash_prefill_blocks_workspace(n_head, n_kv, L) == 0
        assert torch.equal(K.flash_prefill_blocks(q2, kv16), got)


def test_flash_prefill_blocks_full_length(K):
    """The block path at the config-3 length (8192 positions, 14/2 heads), unsplit, against the
    fp32-cache kernel."""
    test_flash_prefill_blocks_equals_fp32_cache_path(K, 8192, 14, 2)


def _blocks_case(K, L, n_head, n_kv, seed):
    rng = np.random.default_rng(seed)
    hd = 64
    qkv = torch.from_numpy(rng.standard_normal((L, (n_head + 2 * n_kv) * hd)).astype(np.float32)).to(DEV)
    ang = rng.standard_normal((L, hd // 2)).astype(np.float32)
    cos, sin = torch.from_numpy(np.cos(ang)).to(DEV), torch.from_numpy(np.sin(ang)).to(DEV)
    kc, vc = torch.zeros(n_kv, L, hd, device=DEV), torch.zeros(n_kv, L, hd, device=DEV)
    kv16 = K.kv16_blocks(n_kv, L, DEV)
    q = K.rope_kv_write(qkv, cos, sin, n_head, kc, vc, kv16=kv16)
    return q, kc, vc, kv16


@pytest.mark.parametrize("L,n_head,n_kv", [(4097, 14, 2), (4200, 8, 8), (5000, 9, 3), (6001, 4, 2),
                                           (9000, 14, 2), (8192, 16, 1)])
def test_flash_prefill_blocks_split_merge(K, L, n_head, n_kv):
    """Past 4096 positions the long query sets run as several key ranges merged by a second
    launch: the queries below 4096 (unsplit sets) keep the unsplit bits, the others stay within
    two fp16 ulps of them, plus 2^-14 where the sum cancels (the same sums in another fp32
    order); the workspace's prior contents
    do not matter, and one byte too few is refused."""
    q, _, _, kv16 = _blocks_case(K, L, n_head, n_kv, L + n_head)
    need = K.flash_prefill_blocks_workspace(n_head, n_kv, L)
    assert need > 0
    un = K.flash_prefill_blocks(q, kv16, split=False)
    ws = torch.full((need,), 0xFF, device=DEV, dtype=torch.uint8)  # NaN bit patterns
    sp = K.flash_prefill_blocks(q, kv16, workspace=ws)
    assert torch.equal(sp[:4096], un[:4096])
    a, b = un.float(), sp.float()
    ulp = torch.exp2(torch.floor(torch.log2(a.abs().clamp_min(2.0 ** -14))) - 10)
    excess = ((a - b).abs() - 2 * ulp).max().item()  # plus 2^-14 absolute near cancellation
    assert excess <= 2.0 ** -14, excess
    assert torch.equal(K.flash_prefill_blocks(q, kv16, workspace=ws), sp)  # deterministic
    with pytest.raises(RuntimeError):
        K.flash_prefill_blocks(q, kv16, workspace=ws[:need - 1])


def test_flash_prefill_blocks_split_matches_closed_form(K):
    """The split schedule (4608 positions, 4 heads on one kv head: sets of up to 72 key blocks
    in two ranges) against float64 attention on the same fp16-rounded q, k, v."""
    L, n_head, n_kv = 4608, 4, 1
    q, kc, vc, kv16 = _blocks_case(K, L, n_head, n_kv, 77)
    assert K.flash_prefill_blocks_workspace(n_head, n_kv, L) > 0
    out = K.flash_prefill_blocks(q, kv16).float().cpu().numpy()
    h16 = lambda t: t.cpu().numpy().astype(np.float16).astype(np.float32)
    ref = closed.causal_attention(h16(q), h16(kc), h16(vc), 0).reshape(L, n_head * 64)
    assert rel_err(out, ref) < 2e-3


@pytest.mark.parametrize("L,pos0", [(1, 0), (5, 0), (64, 0), (100, 7), (130, 0), (513, 0)])
@pytest.mark.parametrize("n_head,n_kv", [(14, 2), (8, 8), (16, 4), (16, 1), (9, 3)])
def test_flash_prefill_matches_closed_form(K, L, pos0, n_head, n_kv):
    """Causal GQA attention on the matrix cores against float64 on the same fp16-rounded q, k,
    v (the probabilities are rounded to fp16 inside: 2e-3 relative), for group sizes 7, 1, 4,
    16 and 3 (query blocks of 32, 256, 64, 16 and 80 per workgroup)."""
    rng = np.random.default_rng(L + pos0)
    hd, cap = 64, pos0 + L + 3
    q = rng.standard_normal((L, n_head, hd)).astype(np.float32)
    k, v = _kv(rng, n_kv, cap, hd)
    out = K.flash_prefill(torch.from_numpy(q).to(DEV), torch.from_numpy(k).to(DEV),
                          torch.from_numpy(v).to(DEV), pos0=pos0).cpu().numpy()
    h16 = lambda a: a.astype(np.float16).astype(np.float32)
    ref = closed.causal_attention(h16(q), h16(k), h16(v), pos0).reshape(L, n_head * hd)
    assert rel_err(out, ref) < 2e-3
    fp32 = K.prefill_attn(torch.from_numpy(q).to(DEV), torch.from_numpy(k).to(DEV),
                          torch.from_numpy(v).to(DEV), pos0=pos0).cpu().numpy()
    assert rel_err(out, fp32) < 5e-3  # the fp32 path, to fp16-operand accuracy
