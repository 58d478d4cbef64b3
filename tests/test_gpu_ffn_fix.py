"""GPU parity of the fused decode FFN (pe_ffn_fix) and its consumer (pe_qkv_fix_rmsnorm_rope):

* the down-slice layout byte for byte against a numpy restatement (random blocks: every code
  value, subnormal scales);
* the FFN output (the sum of the fixed-point replicas) against float64 closed forms over the
  oracle's dequantized weights (1e-3 relative), and against the two-launch path it replaces
  (pe_qgemv_fix_rmsnorm_silu + pe_qgemv, 1e-5), for every ffn_down format, both gate/up
  formats, the config-0 shape and a hidden of 2048;
* x_sum bit for bit: x + (float)(2^-32 acc_in);
* the replica count (1, 2, 4, 8) leaves the summed accumulator unchanged bit for bit, runs
  are deterministic, natural and unit-transposed layouts agree, an unrepresentable addend is
  counted and turns the consumer's vector into NaN;
* the staged QKV launch over x + the replicas against the direct QKV launch over the same
  sum computed on the host (1e-5) and against float64 (1e-3), its x_sum bit for bit.
"""

import numpy as np
import pytest
import torch

from helpers import dequant_rows, quantized_normal, random_quant, rel_err
from oracle import closed
from oracle import dequant as dq

pytestmark = pytest.mark.gpu
TOL = 1e-3
DEV = "cuda"
FIX = 2.0 ** 32


@pytest.fixture(scope="module")
def K():
    from pico_hip import kernels
    return kernels


def dev_bytes(raw: bytes) -> torch.Tensor:
    return torch.from_numpy(np.frombuffer(raw, np.uint8).copy()).to(DEV)


def T(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _f16(b: np.ndarray) -> np.float32:
    return np.float32(np.frombuffer(bytes(b), np.float16)[0])


def _k4_scale_min(s: np.ndarray, j: int) -> tuple[int, int]:
    if j < 4:
        return int(s[j]) & 63, int(s[j + 4]) & 63
    return (int(s[j + 4]) & 15) | ((int(s[j - 4]) >> 6) << 4), (int(s[j + 4]) >> 4) | ((int(s[j]) >> 6) << 4)


def down_slice_ref(t: int, raw: bytes, n: int, k: int) -> np.ndarray:
    """numpy restatement of the down-slice layout (include/pico_hip.h, pe_repack_down_slices)."""
    qk, size = dq.BLOCK[t]
    blocks = np.frombuffer(raw, np.uint8).reshape(n, k // qk, size)
    U = k // 32
    ka, ks = {dq.Q4_K: (16, 8), dq.Q6_K: (16, 16), dq.Q5_0: (16, 8), dq.Q8_0: (32, 4)}[t]
    A = np.zeros((U, n, ka), np.uint8)
    S = np.zeros((U, n, ks), np.uint8)
    nu = n // 32
    ut_pos = lambda r: ((r % 32) // 4 * nu + r // 32) * 4 + r % 4   # records in this row order
    for u in range(U):
        for rr in range(n):
            r, pos = rr, ut_pos(rr)
            if t == dq.Q4_K:
                b = blocks[r, u // 8]
                j = u % 8
                chunk = b[16 + 32 * (j // 2):48 + 32 * (j // 2)]
                code = (chunk >> 4) if j & 1 else (chunk & 15)
                A[u, pos] = code[:16] | (code[16:] << 4)
                sc, mn = _k4_scale_min(b[4:16], j)
                S[u, pos] = np.array([_f16(b[0:2]) * np.float32(sc), _f16(b[2:4]) * np.float32(mn)],
                                   np.float32).view(np.uint8)
            elif t == dq.Q6_K:
                b = blocks[r, u // 8]
                hf, q = (u % 8) // 4, u % 4
                ql = b[64 * hf + 32 * (q & 1):64 * hf + 32 * (q & 1) + 32]
                lo = (ql >> 4) if q >= 2 else (ql & 15)
                hi = (b[128 + 32 * hf:160 + 32 * hf] >> (2 * q)) & 3
                A[u, pos] = lo[:16] | (lo[16:] << 4)
                S[u, pos, :8] = hi[:8] | (hi[8:16] << 2) | (hi[16:24] << 4) | (hi[24:] << 6)
                d = _f16(b[208:210])
                sc = b[192 + 8 * hf + 2 * q:194 + 8 * hf + 2 * q].view(np.int8).astype(np.float32)
                S[u, pos, 8:] = (d * sc).astype(np.float32).view(np.uint8)
            elif t == dq.Q5_0:
                b = blocks[r, u]
                A[u, pos] = b[6:22]
                S[u, pos, :4] = b[2:6]
                S[u, pos, 4:] = np.array([_f16(b[0:2])], np.float32).view(np.uint8)
            else:
                b = blocks[r, u]
                A[u, pos] = b[2:34]
                S[u, pos] = np.array([_f16(b[0:2])], np.float32).view(np.uint8)
    return np.concatenate([A.reshape(-1), S.reshape(-1)])


@pytest.mark.parametrize("t,n,k", [(dq.Q4_K, 64, 512), (dq.Q6_K, 64, 512), (dq.Q5_0, 64, 96),
                                   (dq.Q8_0, 96, 96), (dq.Q6_K, 32, 256)])
def test_down_slice_layout_bytes(K, t, n, k):
    raw = random_quant(t, n, k, seed=n + k + t)
    got = K.repack_down_slices(dev_bytes(raw), t, n, k).cpu().numpy()
    np.testing.assert_array_equal(got, down_slice_ref(t, raw, n, k))
    with pytest.raises(ValueError):
        K.repack_down_slices(dev_bytes(raw), t, n, k - 16)
    if n > 32:
        with pytest.raises(ValueError):   # rows are stored in the unit-transposed order: n % 32
            K.repack_down_slices(dev_bytes(raw[:len(raw) * 16 // n]), t, 16, k)


class Ffn:
    """One FFN layer: [gate; up] and ffn_down quantized N(0, 0.02), their float64 forms."""

    def __init__(self, K, t_gu, t_down, hidden, ffn, seed):
        self.hidden, self.ffn = hidden, ffn
        gu_raw = quantized_normal(t_gu, 2 * ffn, hidden, seed=seed)
        dn_raw = quantized_normal(t_down, hidden, ffn, seed=seed + 1)
        self.w_gu = K.pack_weight(dev_bytes(gu_raw), t_gu, 2 * ffn, hidden)
        self.w_down = K.pack_weight(dev_bytes(dn_raw), t_down, hidden, ffn, slices=True)
        assert self.w_down.slices is not None
        self.gu64 = dequant_rows(t_gu, gu_raw, 2 * ffn, hidden).astype(np.float64)
        self.dn64 = dequant_rows(t_down, dn_raw, hidden, ffn).astype(np.float64)

    def inputs(self, seed):
        rng = np.random.default_rng(seed)
        h = self.hidden
        x = rng.standard_normal(h).astype(np.float32)
        nw = (1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32)
        acc = np.zeros(h + 2, np.int64)
        acc[:h] = np.rint(rng.standard_normal(h) * 0.5 * FIX).astype(np.int64)
        return x, nw, acc

    def reference(self, x, nw, acc):
        """(x_sum as the kernel forms it, the down product in float64)."""
        h = self.hidden
        xs = (x + (acc[:h].astype(np.float64) / FIX).astype(np.float32)).astype(np.float32)
        hn = closed.rmsnorm(xs.astype(np.float64), nw, 1e-6)
        gu = self.gu64 @ hn
        act = closed.silu_mul(gu[:self.ffn], gu[self.ffn:])
        return xs, self.dn64 @ act


def run_ffn(K, f: Ffn, x, nw, acc, replicas=4, ut=True):
    h = f.hidden
    xin, nin, ain = T(x), T(nw), T(acc)
    if ut:
        xin, nin = K.to_ut(xin), K.to_ut(nin)
        ain = ain.clone()
        ain[:h] = K.to_ut(ain[:h])
    out = torch.zeros(replicas, K.fix_stride(h), device=DEV, dtype=torch.int64)
    xs = K.ffn_fix(xin, ain, nin, f.w_gu, f.w_down, 1e-6, out,
                   layout=(K.LAYOUT_X_UT | K.LAYOUT_Y_UT) if ut else K.LAYOUT_NATURAL)
    tot = out.sum(0)
    if ut:
        xs = K.from_ut(xs)
        tot = torch.cat([K.from_ut(tot[:h]), tot[h:]])
    return xs.cpu().numpy(), tot.cpu().numpy(), out


SHAPES = [  # (gate/up type, ffn_down type, hidden, ffn)
    (dq.Q5_0, dq.Q6_K, 896, 4864),
    (dq.Q5_0, dq.Q4_K, 896, 4864),
    (dq.Q8_0, dq.Q6_K, 256, 512),
    (dq.Q5_0, dq.Q5_0, 256, 96),
    (dq.Q8_0, dq.Q8_0, 128, 160),
    (dq.Q5_0, dq.Q4_K, 2048, 1024),
]


@pytest.mark.parametrize("t_gu,t_down,hidden,ffn", SHAPES)
def test_ffn_fix_matches_float64_and_two_launch_path(K, t_gu, t_down, hidden, ffn):
    f = Ffn(K, t_gu, t_down, hidden, ffn, seed=hidden + ffn + t_down)
    x, nw, acc = f.inputs(seed=hidden)
    xs_ref, y_ref = f.reference(x, nw, acc)
    xs, tot, _ = run_ffn(K, f, x, nw, acc)
    np.testing.assert_array_equal(xs, xs_ref)              # x + (float)(2^-32 acc), bit for bit
    assert tot[hidden] == 0
    y = tot[:hidden].astype(np.float64) / FIX
    assert rel_err(y, y_ref) < TOL
    # the two launches it replaces: fixed-point gate/up GEMV, then the ffn_down GEMV
    act, xs2 = K.qgemv_fix_norm_silu(T(x), T(acc), T(nw), f.w_gu, 1e-6)
    y2 = K.qgemv(act, f.w_down).cpu().numpy()
    np.testing.assert_array_equal(xs2.cpu().numpy(), xs)
    assert rel_err(y, y2) < 1e-5


def test_ffn_fix_replicas_layouts_determinism(K):
    f = Ffn(K, dq.Q5_0, dq.Q6_K, 896, 4864, seed=5)
    x, nw, acc = f.inputs(seed=6)
    base = run_ffn(K, f, x, nw, acc, replicas=4)[1]
    for reps in (1, 2, 8):
        np.testing.assert_array_equal(run_ffn(K, f, x, nw, acc, replicas=reps)[1], base)
    np.testing.assert_array_equal(run_ffn(K, f, x, nw, acc, replicas=4)[1], base)     # deterministic
    np.testing.assert_array_equal(run_ffn(K, f, x, nw, acc, replicas=4, ut=False)[1], base)
    # replica q holds the blocks b with b % 4 == q: every replica is non-zero
    out = run_ffn(K, f, x, nw, acc, replicas=4)[2]
    assert all(bool(out[q, :896].ne(0).any()) for q in range(4))


def test_ffn_fix_adds_to_existing_replicas_and_counts_unrepresentable(K):
    f = Ffn(K, dq.Q5_0, dq.Q4_K, 256, 512, seed=9)
    x, nw, acc = f.inputs(seed=10)
    once = run_ffn(K, f, x, nw, acc)[1]
    # a second launch into the same replicas adds the same sums again
    out = torch.zeros(4, K.fix_stride(256), device=DEV, dtype=torch.int64)
    for _ in range(2):
        K.ffn_fix(K.to_ut(T(x)), torch.cat([K.to_ut(T(acc[:256])), T(acc[256:])]), K.to_ut(T(nw)),
                  f.w_gu, f.w_down, 1e-6, out, layout=K.LAYOUT_X_UT | K.LAYOUT_Y_UT)
    tot = out.sum(0)
    np.testing.assert_array_equal(torch.cat([K.from_ut(tot[:256]), tot[256:]]).cpu().numpy(), 2 * once)
    # an addend at or beyond the bound is counted instead of added
    bound = K.ffn_fix_bound(512)
    assert bound == 2.0 ** 27   # 16 units: the largest power of two with 16 * b <= 2^31
    xb = x.copy()
    xb[3] = 1e30
    nwb = nw.copy()
    nwb[:] = 1e30
    _, tot, _ = run_ffn(K, f, xb, nwb, acc)
    assert tot[256] > 0
    # ... and the consumer turns every element into NaN
    q, xs = qkv_fix_case(K, dq.Q5_0, 256, 4, 2, acc_replicas=out.clone().fill_(0), poison=True)
    assert np.isnan(xs).all() and np.isnan(q).all()


def qkv_fix_case(K, t, hidden, nh, nkv, acc_replicas=None, poison=False, seed=3):
    """Run the staged QKV launch; returns (q, x_sum) (host arrays)."""
    hd, cap, pos = 64, 24, 17
    rows = (nh * hd, nkv * hd, nkv * hd)
    raws = [quantized_normal(t, r, hidden, seed=seed + i) for i, r in enumerate(rows)]
    ws = [K.pack_weight(dev_bytes(raw), t, r, hidden) for raw, r in zip(raws, rows)]
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(hidden).astype(np.float32)
    nw = rng.standard_normal(hidden).astype(np.float32)
    inv = 1.0 / (1e6 ** (np.arange(0, hd, 2) / hd))
    ang = (np.arange(64)[:, None] * inv[None, :]).astype(np.float32)
    cos, sin = T(np.cos(ang).astype(np.float32)), T(np.sin(ang).astype(np.float32))
    acc = acc_replicas
    if poison:
        acc[2, hidden] = 1
    kc = torch.zeros(nkv, cap, hd, device=DEV)
    vc = torch.zeros(nkv, cap, hd, device=DEV)
    q, xs = K.qkv_fix_rmsnorm_rope(K.to_ut(T(x)), acc, K.to_ut(T(nw)), 1e-6, *ws, None, None, None,
                                   cos, sin, torch.tensor([pos], device=DEV), kc, vc, nh,
                                   layout=K.LAYOUT_X_UT)
    return q.cpu().numpy(), (None if xs is None else K.from_ut(xs).cpu().numpy())


@pytest.mark.parametrize("t,hidden,nh,nkv,replicas", [(dq.Q5_0, 896, 14, 2, 4), (dq.Q8_0, 896, 14, 2, 0),
                                                      (dq.Q4_K, 512, 8, 2, 4), (dq.Q6_K, 2048, 16, 4, 4)])
def test_qkv_fix_matches_direct_qkv_over_the_sum(K, t, hidden, nh, nkv, replicas):
    hd, cap, pos = 64, 40, 29
    rows = (nh * hd, nkv * hd, nkv * hd)
    raws = [quantized_normal(t, r, hidden, seed=hidden + i) for i, r in enumerate(rows)]
    ws = [K.pack_weight(dev_bytes(raw), t, r, hidden) for raw, r in zip(raws, rows)]
    rng = np.random.default_rng(hidden + replicas)
    bs = [rng.standard_normal(r).astype(np.float32) * 0.1 for r in rows]
    x = rng.standard_normal(hidden).astype(np.float32)
    nw = rng.standard_normal(hidden).astype(np.float32)
    stride = K.fix_stride(hidden)
    acc = np.zeros((max(replicas, 1), stride), np.int64)
    if replicas:
        acc[:, :hidden] = np.rint(rng.standard_normal((replicas, hidden)) * 0.3 * FIX).astype(np.int64)
    tot = acc.sum(0)[:hidden]
    xs_ref = (x + (tot.astype(np.float64) / FIX).astype(np.float32)).astype(np.float32) if replicas else x
    inv = 1.0 / (1e6 ** (np.arange(0, hd, 2) / hd))
    ang = (np.arange(64)[:, None] * inv[None, :]).astype(np.float32)
    cos_np, sin_np = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    cos, sin = T(cos_np), T(sin_np)
    UT = K.LAYOUT_X_UT
    dacc = None
    if replicas:
        dacc = T(acc)
        for q_ in range(replicas):
            dacc[q_, :hidden] = K.to_ut(dacc[q_, :hidden])
    kc, vc = torch.zeros(nkv, cap, hd, device=DEV), torch.zeros(nkv, cap, hd, device=DEV)
    q, xs = K.qkv_fix_rmsnorm_rope(K.to_ut(T(x)), dacc, K.to_ut(T(nw)), 1e-6, *ws, *[T(b) for b in bs],
                                   cos, sin, torch.tensor([pos], device=DEV), kc, vc, nh, layout=UT)
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    q2 = K.qkv_rmsnorm_rope(K.to_ut(T(xs_ref)), K.to_ut(T(nw)), 1e-6, *ws, *[T(b) for b in bs], cos, sin,
                            torch.tensor([pos], device=DEV), kc2, vc2, nh, layout=UT)
    if replicas:
        np.testing.assert_array_equal(K.from_ut(xs).cpu().numpy(), xs_ref)
    else:
        assert xs is None
    assert rel_err(q.cpu().numpy(), q2.cpu().numpy()) < 1e-5
    assert rel_err(kc.cpu().numpy(), kc2.cpu().numpy()) < 1e-5
    assert rel_err(vc.cpu().numpy(), vc2.cpu().numpy()) < 1e-5
    # float64 closed forms
    h = closed.rmsnorm(xs_ref.astype(np.float64), nw, 1e-6)
    outs = [closed.gemv(dequant_rows(t, raw, r, hidden), h, bias=b) for raw, r, b in zip(raws, rows, bs)]
    assert rel_err(q.cpu().numpy(), closed.rope(outs[0].reshape(nh, hd), cos_np[pos], sin_np[pos])) < TOL
    kcn, vcn = kc.cpu().numpy(), vc.cpu().numpy()
    assert rel_err(kcn[:, pos], closed.rope(outs[1].reshape(nkv, hd), cos_np[pos], sin_np[pos])) < TOL
    assert rel_err(vcn[:, pos], outs[2].reshape(nkv, hd)) < TOL
    kcn[:, pos] = 0
    vcn[:, pos] = 0
    assert not kcn.any() and not vcn.any()


def test_abi_rejects_bad_ffn_fix_arguments(K):
    from pico_hip._lib import FfnFixArgs, lib
    import ctypes
    f = Ffn(K, dq.Q5_0, dq.Q8_0, 128, 64, seed=1)
    x = torch.zeros(128, device=DEV)
    acc = torch.zeros(130, device=DEV, dtype=torch.int64)
    out = torch.zeros(4, K.fix_stride(128), device=DEV, dtype=torch.int64)

    def call(**kw):
        a = dict(type_gu=f.w_gu.ggml_type, w_gu=f.w_gu.data.data_ptr(), type_down=f.w_down.ggml_type,
                 w_down=f.w_down.slices.data_ptr(), hidden=128, ffn=64, x=x.data_ptr(), acc_in=acc.data_ptr(),
                 norm_w=x.data_ptr(), eps=1e-6, x_sum=None, acc_out=out.data_ptr(), replicas=4,
                 acc_stride=K.fix_stride(128), layout=0)
        a.update(kw)
        return lib.pe_ffn_fix(ctypes.byref(FfnFixArgs(**a)), None)

    assert call() == 0
    assert call(replicas=3) == 3
    assert call(acc_stride=128) == 3
    assert call(type_gu=dq.Q4_K) == 2
    assert call(hidden=4096) == 3
    assert call(acc_out=None) == 1
    assert call(x=x.data_ptr() + 4) == 4
    torch.cuda.synchronize()


# ---- the first layer's QKV launch over the token's embedding row ---------------------------

@pytest.mark.parametrize("t,et,hidden,nh,nkv,vocab", [(dq.Q5_0, dq.Q8_0, 896, 14, 2, 300),
                                                      (dq.Q8_0, dq.F16, 896, 14, 2, 100),
                                                      (dq.Q4_K, dq.Q4_K, 512, 8, 2, 64),
                                                      (dq.Q6_K, dq.Q6_K, 2048, 16, 4, 40)])
def test_qkv_embed_matches_gather_then_staged_qkv(K, t, et, hidden, nh, nkv, vocab):
    """pe_qkv_embed_rmsnorm_rope == pe_embed_gather followed by the staged launch over that
    row (the same bits: the same decode and the same staged arithmetic), x_out == the gathered
    row, and the clear range zeroed (the words after it untouched)."""
    hd, cap, pos = 64, 40, 29
    rows = (nh * hd, nkv * hd, nkv * hd)
    raws = [quantized_normal(t, r, hidden, seed=hidden + i) for i, r in enumerate(rows)]
    ws = [K.pack_weight(dev_bytes(raw), t, r, hidden) for raw, r in zip(raws, rows)]
    rng = np.random.default_rng(hidden)
    traw = ((rng.standard_normal(vocab * hidden) * 0.02).astype(np.float16).tobytes() if et == dq.F16
            else random_quant(et, vocab, hidden, seed=hidden))
    table = K.RawTensor(dev_bytes(traw), et, (vocab, hidden))
    bs = [T(rng.standard_normal(r).astype(np.float32) * 0.1) for r in rows]
    nw = K.to_ut(T(rng.standard_normal(hidden).astype(np.float32)))
    inv = 1.0 / (1e6 ** (np.arange(0, hd, 2) / hd))
    ang = (np.arange(64)[:, None] * inv[None, :]).astype(np.float32)
    cos, sin = T(np.cos(ang).astype(np.float32)), T(np.sin(ang).astype(np.float32))
    UT = K.LAYOUT_X_UT
    tok = torch.tensor([vocab - 3], device=DEV)
    pos_t = torch.tensor([pos], device=DEV)
    clear = torch.full((3, 4, K.fix_stride(hidden)), -7, dtype=torch.int64, device=DEV)
    guard = torch.full((64,), 5, dtype=torch.int64, device=DEV)
    block = torch.cat([clear.reshape(-1), guard])   # the clear range, then words it must not touch
    xo = torch.empty(hidden, device=DEV)
    kc, vc = torch.zeros(nkv, cap, hd, device=DEV), torch.zeros(nkv, cap, hd, device=DEV)
    q = K.qkv_embed_rmsnorm_rope(table, tok, nw, 1e-6, *ws, *bs, cos, sin, pos_t, kc, vc, nh, x_out=xo,
                                 clear=block[:clear.numel()], layout=UT)
    row = K.embed_gather(table, tok, layout=K.LAYOUT_Y_UT).reshape(-1)
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    q2, _ = K.qkv_fix_rmsnorm_rope(row, None, nw, 1e-6, *ws, *bs, cos, sin, pos_t, kc2, vc2, nh, layout=UT)
    assert torch.equal(xo, row)
    assert torch.equal(q, q2) and torch.equal(kc, kc2) and torch.equal(vc, vc2)
    assert not block[:clear.numel()].any()
    assert (block[clear.numel():] == 5).all()
    # an id outside the table: NaN activation (as pe_embed_gather gives)
    bad = torch.tensor([vocab], device=DEV)
    q3 = K.qkv_embed_rmsnorm_rope(table, bad, nw, 1e-6, *ws, *bs, cos, sin, pos_t, kc, vc, nh, x_out=xo,
                                  layout=UT)
    assert torch.isnan(xo).all() and torch.isnan(q3).all()
