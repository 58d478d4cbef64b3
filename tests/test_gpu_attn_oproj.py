"""GPU parity of the per-head attention + o-projection launch (pe_attn_oproj_fix) and its
consumer (pe_qgemv_fix_rmsnorm_silu): the o-projection layout byte for byte against a numpy
restatement, the attention over the cache with the fp16 output rounding times each head's
columns of Wo against float64 closed forms (1e-3 relative), the fixed-point accumulator's
determinism, layouts and poison count, and the gate/up GEMV over x + 2^-32 acc bit for bit
against the same GEMV over x + parts."""

import numpy as np
import pytest
import torch

from helpers import dequant_rows, quantized_normal, rel_err
from oracle import closed
from oracle import dequant as dq

pytestmark = pytest.mark.gpu
TOL = 1e-3
DEV = "cuda"
FIX = 2.0 ** 32
NAME = {dq.Q5_0: "Q5_0", dq.Q8_0: "Q8_0"}


@pytest.fixture(scope="module")
def K():
    from pico_hip import kernels
    return kernels


def dev_bytes(raw: bytes) -> torch.Tensor:
    return torch.from_numpy(np.frombuffer(raw, np.uint8).copy()).to(DEV)


def oproj_layout_ref(t: int, raw: bytes, n: int, k: int) -> np.ndarray:
    """numpy restatement of the o-projection layout (include/pico_hip.h, pe_repack_oproj)."""
    size = 22 if t == dq.Q5_0 else 34
    blocks = np.frombuffer(raw, np.uint8).reshape(n, k // 32, size)
    tiles, heads = (n + 15) // 16, k // 64
    bsz = 704 if t == dq.Q5_0 else 1088
    dofs = 640 if t == dq.Q5_0 else 1024
    out = np.zeros((heads, tiles, bsz), np.uint8)
    for hh in range(heads):
        for ti in range(tiles):
            ob = out[hh, ti]
            for lane in range(64):
                row, g = 16 * ti + (lane & 15), lane >> 4
                if row >= n:
                    continue
                units = [blocks[row, 2 * hh + u] for u in range(2)]
                if t == dq.Q5_0:
                    hb = 0
                    for u, b in enumerate(units):
                        ob[8 * lane + 4 * u:8 * lane + 4 * u + 4] = b[6 + 4 * g:10 + 4 * g]
                        qh = int.from_bytes(bytes(b[2:6]), "little")
                        for c in range(2):
                            for i in range(4):
                                hb |= ((qh >> (16 * c + 4 * g + i)) & 1) << (4 * (2 * u + c) + i)
                    ob[512 + 2 * lane:514 + 2 * lane] = np.frombuffer(hb.to_bytes(2, "little"), np.uint8)
                else:
                    for u, b in enumerate(units):
                        ob[16 * lane + 8 * u:16 * lane + 8 * u + 4] = b[2 + 4 * g:6 + 4 * g]
                        ob[16 * lane + 8 * u + 4:16 * lane + 8 * u + 8] = b[18 + 4 * g:22 + 4 * g]
                if lane < 32:
                    ob[dofs + 2 * lane:dofs + 2 * lane + 2] = units[lane >> 4][0:2]
    return out.reshape(-1)


@pytest.mark.parametrize("t,n,k", [(dq.Q5_0, 40, 128), (dq.Q8_0, 40, 128), (dq.Q5_0, 16, 896),
                                   (dq.Q8_0, 33, 192)])
def test_oproj_layout_bytes(K, t, n, k):
    raw = quantized_normal(t, n, k, seed=n + k + t)
    got = K.repack_oproj(dev_bytes(raw), t, n, k).cpu().numpy()
    np.testing.assert_array_equal(got, oproj_layout_ref(t, raw, n, k))
    with pytest.raises(ValueError):
        K.repack_oproj(dev_bytes(raw), t, n, k - 32)   # k % 64


def make_wo(K, t, hidden, nh, seed):
    raw = quantized_normal(t, hidden, nh * 64, seed=seed)
    wo = K.pack_weight(dev_bytes(raw), t, hidden, nh * 64, oproj=True)
    assert wo.oproj is not None
    return wo, dequant_rows(t, raw, hidden, nh * 64)


CASES = [
    # the config-0 layer (Q5_0 Wo), 14/2 heads, capacity 77
    (dq.Q5_0, 896, 14, 2, 77, [0, 12, 44, 76]),
    (dq.Q8_0, 896, 14, 2, 128, [1, 63, 64, 127]),   # a full cache: both score passes
    (dq.Q8_0, 512, 8, 8, 64, [30]),                  # one query head per kv head
    (dq.Q5_0, 1024, 16, 2, 100, [99]),               # 8 heads per group
    (dq.Q5_0, 256, 4, 2, 16, [5]),                   # the tiny test model
    (dq.Q8_0, 160, 2, 1, 20, [17]),                  # 10 row tiles: a partial second workgroup
]


@pytest.mark.parametrize("t,hidden,nh,nkv,cap,positions", CASES,
                         ids=[f"h{h}-{nh}x{nkv}-cap{c}-{NAME[t]}" for t, h, nh, nkv, c, _ in CASES])
def test_attn_oproj_matches_closed_form(K, t, hidden, nh, nkv, cap, positions):
    hd = 64
    rng = np.random.default_rng(hidden + nh + cap)
    wo, Wo = make_wo(K, t, hidden, nh, seed=hidden + cap)
    assert K.attn_oproj_supported(nh, nkv, hd, cap, wo)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    for pos in positions:
        q = rng.standard_normal((nh, hd)).astype(np.float32)
        kc = rng.standard_normal((nkv, cap, hd)).astype(np.float32)
        vc = rng.standard_normal((nkv, cap, hd)).astype(np.float32)
        acc = K.fix_acc(hidden, DEV)[0]
        K.attn_oproj_fix(T(q), T(kc), T(vc), wo, torch.tensor([pos], device=DEV), acc)
        attn = closed.attention(q, kc, vc, pos + 1, round_fp16=True).reshape(-1)
        ref = closed.gemv(Wo, attn)
        a = acc.cpu().numpy()
        assert a[hidden] == 0, f"pos={pos}: unrepresentable-value count {a[hidden]}"
        assert rel_err(a[:hidden].astype(np.float64) / FIX, ref) < TOL, f"pos={pos}"
        # integer sums: a second launch gives the same bits
        acc2 = K.fix_acc(hidden, DEV)[0]
        K.attn_oproj_fix(T(q), T(kc), T(vc), wo, torch.tensor([pos], device=DEV), acc2)
        assert torch.equal(acc, acc2)


def test_attn_oproj_accumulates_layouts_position_limits(K):
    """acc is added to (two launches = twice the sums); the unit-transposed accumulator holds
    the natural one's sums; a position outside the cache only counts as unrepresentable;
    shape limits."""
    hd, hidden, nh, nkv, cap = 64, 896, 14, 2, 77
    rng = np.random.default_rng(5)
    wo, _ = make_wo(K, dq.Q5_0, hidden, nh, seed=5)
    q = torch.from_numpy(rng.standard_normal((nh, hd)).astype(np.float32)).to(DEV)
    kc = torch.from_numpy(rng.standard_normal((nkv, cap, hd)).astype(np.float32)).to(DEV)
    vc = torch.from_numpy(rng.standard_normal((nkv, cap, hd)).astype(np.float32)).to(DEV)
    pos = torch.tensor([40], device=DEV)
    nat = K.fix_acc(hidden, DEV)[0]
    K.attn_oproj_fix(q, kc, vc, wo, pos, nat)
    twice = nat.clone()
    K.attn_oproj_fix(q, kc, vc, wo, pos, twice)
    assert torch.equal(twice[:hidden], 2 * nat[:hidden]) and int(twice[hidden]) == 0
    ut = K.fix_acc(hidden, DEV)[0]
    K.attn_oproj_fix(q, kc, vc, wo, pos, ut, layout=K.LAYOUT_Y_UT)
    assert torch.equal(K.from_ut(ut[:hidden]), nat[:hidden])
    assert int(ut[hidden]) == 0
    for bad_pos in (cap, -1):
        bad = K.fix_acc(hidden, DEV)[0]
        K.attn_oproj_fix(q, kc, vc, wo, torch.tensor([bad_pos], device=DEV), bad)
        assert int(bad[hidden]) > 0 and not bad[:hidden].any(), bad_pos
    assert not K.attn_oproj_supported(nh, nkv, hd, 129, wo)        # capacity past 128
    assert not K.attn_oproj_supported(nh, nkv, 128, cap, wo)       # head_dim 128
    plain = K.pack_weight(dev_bytes(quantized_normal(dq.Q5_0, hidden, nh * hd, seed=1)), dq.Q5_0,
                          hidden, nh * hd)
    assert plain.oproj is None and not K.attn_oproj_supported(nh, nkv, hd, cap, plain)
    with pytest.raises(ValueError):
        K.attn_oproj_fix(q, kc, vc, plain, pos, nat)


@pytest.mark.parametrize("t", [dq.Q5_0, dq.Q8_0])
def test_qgemv_fix_norm_silu_equals_parts_path(K, t):
    """x + 2^-32 acc with acc holding exact images of fp32 values equals x + that one part,
    bit for bit (gate/up output and the stored sum); a non-zero poison count gives NaN."""
    hidden, ffn, eps = 896, 4864, 1e-6
    rng = np.random.default_rng(t)
    raw = quantized_normal(t, 2 * ffn, hidden, seed=t + 3)
    w = K.pack_weight(dev_bytes(raw), t, 2 * ffn, hidden)
    x = torch.from_numpy(rng.standard_normal(hidden).astype(np.float32)).to(DEV)
    nw = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)).to(DEV)
    # parts of magnitude >= 2^-8 have no bits below 2^-32: p 2^32 is an exact integer
    p = (rng.choice([-1.0, 1.0], hidden) * rng.uniform(2.0 ** -8, 4.0, hidden)).astype(np.float32)
    fixv = np.zeros(hidden + 2, np.int64)
    fixv[:hidden] = (p.astype(np.float64) * FIX).astype(np.int64)
    assert np.array_equal(fixv[:hidden].astype(np.float64) / FIX, p.astype(np.float64))
    fix = torch.from_numpy(fixv).to(DEV)
    parts = torch.from_numpy(p[None]).to(DEV)
    for layout in (0, K.LAYOUT_X_UT | K.LAYOUT_Y_UT):
        xx, nn, pp = (K.to_ut(v) for v in (x, nw, parts[0])) if layout else (x, nw, parts[0])
        ff = fix
        if layout:
            ff = fix.clone()
            ff[:hidden] = K.to_ut(fix[:hidden])
        a1, s1 = K.qgemv_fix_norm_silu(xx, ff, nn, w, eps, layout=layout)
        a2, s2 = K.qgemv_sum_norm_silu(xx, pp[None], nn, w, eps, layout=layout)
        assert torch.equal(a1, a2) and torch.equal(s1, s2), f"layout {layout}"
    fix[hidden] = 1
    a3, s3 = K.qgemv_fix_norm_silu(x, fix, nw, w, eps)
    assert torch.isnan(s3).all() and torch.isnan(a3).all()
