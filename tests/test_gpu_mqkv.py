"""Decode QKV on the integer matrix cores (pe_mqkv_rmsnorm_rope, from the RoPE-pair MFMA
layouts) against float64 on the dequantized weights (1e-3 relative, the decode bound) and
against the tiled QKV launch (fp32-level), its cache writes, the invalid-position rule,
determinism and graph replay."""

import dataclasses

import numpy as np
import pytest
import torch

from helpers import dequant_rows, quantized_normal, rel_err
from oracle import closed
from oracle import dequant as dq

pytestmark = pytest.mark.gpu
TOL = 1e-3
DEV = "cuda"


@pytest.fixture(scope="module")
def K():
    from pico_hip import kernels
    return kernels


def T(a):
    return torch.from_numpy(np.array(a)).to(DEV)


class Qkv:
    """A random QKV problem: weights (with their RoPE-pair layouts), biases, norm, x, tables."""

    def __init__(self, K, types, hidden, nh, nkv, hd, bias=True, seed=0, cap=40):
        rng = np.random.default_rng(seed + hidden)
        self.types, self.hidden, self.nh, self.nkv, self.hd, self.cap = types, hidden, nh, nkv, hd, cap
        self.rows = (nh * hd, nkv * hd, nkv * hd)
        self.raws = [quantized_normal(t, r, hidden, seed=seed + i + 1) for i, (t, r) in enumerate(zip(types, self.rows))]
        self.ws = [K.pack_weight(T(np.frombuffer(raw, np.uint8)), t, r, hidden, pairs_hd=hd)
                   for t, raw, r in zip(types, self.raws, self.rows)]
        self.bs = [rng.standard_normal(r).astype(np.float32) * 0.1 for r in self.rows] if bias else None
        self.x = rng.standard_normal(hidden).astype(np.float32)
        self.nw = rng.standard_normal(hidden).astype(np.float32)
        inv = 1.0 / (1e6 ** (np.arange(0, hd, 2) / hd))
        ang = (np.arange(64)[:, None] * inv[None, :]).astype(np.float32)
        self.cos, self.sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)

    def run(self, K, pos, ut=False, tiled=False, caches=None):
        ws = [dataclasses.replace(w, pairs=None) for w in self.ws] if tiled else self.ws
        assert K.mqkv_ok(*ws) != tiled
        kc, vc = caches if caches is not None else (torch.zeros(self.nkv, self.cap, self.hd, device=DEV),
                                                    torch.zeros(self.nkv, self.cap, self.hd, device=DEV))
        x, nw = T(self.x), T(self.nw)
        if ut:
            x, nw = K.to_ut(x), K.to_ut(nw)
        b = [T(v) for v in self.bs] if self.bs is not None else [None] * 3
        q = K.qkv_rmsnorm_rope(x, nw, 1e-6, *ws, *b, T(self.cos), T(self.sin),
                               torch.tensor([pos], device=DEV), kc, vc, self.nh,
                               layout=K.LAYOUT_X_UT if ut else K.LAYOUT_NATURAL)
        return q, kc, vc

    def expected(self, pos):
        h = closed.rmsnorm(self.x, self.nw, 1e-6)
        bs = self.bs if self.bs is not None else [None] * 3
        outs = [closed.gemv(dequant_rows(t, raw, r, self.hidden), h, bias=b)
                for t, raw, r, b in zip(self.types, self.raws, self.rows, bs)]
        rq = closed.rope(outs[0].reshape(self.nh, self.hd), self.cos[pos], self.sin[pos])
        rk = closed.rope(outs[1].reshape(self.nkv, self.hd), self.cos[pos], self.sin[pos])
        return rq, rk, outs[2].reshape(self.nkv, self.hd)


# The 7B shape (Q4_K q/k, Q6_K v) in both activation layouts; the other format pairings; head
# sizes 16 (one group of 8 pairs per head), 64 and 128; one workgroup wave (hidden 256) to
# eight (hidden 3840 and up)
CASES = [
    ((dq.Q4_K, dq.Q4_K, dq.Q6_K), 3584, 28, 4, 128, False, True),
    ((dq.Q4_K, dq.Q4_K, dq.Q6_K), 3584, 28, 4, 128, True, True),
    ((dq.Q6_K, dq.Q6_K, dq.Q4_K), 512, 4, 2, 64, False, False),
    ((dq.Q4_K, dq.Q4_K, dq.Q4_K), 256, 2, 1, 16, True, True),
    ((dq.Q6_K, dq.Q6_K, dq.Q6_K), 1024, 8, 2, 128, False, True),
    ((dq.Q4_K, dq.Q4_K, dq.Q6_K), 3840, 6, 2, 64, False, True),
]


@pytest.mark.parametrize("types,hidden,nh,nkv,hd,ut,bias", CASES,
                         ids=[f"{c[1]}-{c[2]}x{c[4]}-{'ut' if c[5] else 'nat'}{'-nobias' if not c[6] else ''}" for c in CASES])
def test_mqkv_matches_closed_form_and_tiled(K, types, hidden, nh, nkv, hd, ut, bias):
    p = Qkv(K, types, hidden, nh, nkv, hd, bias=bias)
    pos = 23
    q, kc, vc = p.run(K, pos, ut=ut)
    rq, rk, rv = p.expected(pos)
    qn, kn, vn = q.cpu().numpy(), kc.cpu().numpy(), vc.cpu().numpy()
    assert rel_err(qn, rq) < TOL
    assert rel_err(kn[:, pos], rk) < TOL
    assert rel_err(vn[:, pos], rv) < TOL
    kn[:, pos] = 0
    vn[:, pos] = 0
    assert not kn.any() and not vn.any()  # nothing else written
    # the tiled launch on the same problem: the same values to fp32 rounding
    q2, kc2, vc2 = p.run(K, pos, ut=ut, tiled=True)
    assert rel_err(qn, q2.cpu().numpy()) < 1e-5
    assert rel_err(kc.cpu().numpy(), kc2.cpu().numpy()) < 1e-5
    assert rel_err(vc.cpu().numpy(), vc2.cpu().numpy()) < 1e-5


def test_mqkv_pair_layout_is_the_documented_permutation(K):
    """pe_repack_mfma_pairs == pe_repack_mfma of the rows permuted as the header states."""
    hd, n, k = 32, 64, 256
    raw = quantized_normal(dq.Q4_K, n, k, seed=5)
    blocks = np.frombuffer(raw, np.uint8).reshape(n, -1)
    perm = []
    for g in range(n // 16):
        for j in range(16):
            r = g * 16 + j
            head, rr = divmod(r, hd)
            jt, jj = divmod(rr, 16)
            perm.append(head * hd + (jj // 8) * (hd // 2) + 8 * jt + jj % 8)
    assert sorted(perm) == list(range(n))
    a = K.repack_mfma_pairs(T(blocks.reshape(-1)), dq.Q4_K, n, k, hd)
    b = K.repack_mfma(T(blocks[perm].reshape(-1)), dq.Q4_K, n, k)
    assert torch.equal(a, b)


def test_mqkv_invalid_position_writes_nan_q_and_no_cache(K):
    p = Qkv(K, (dq.Q4_K, dq.Q4_K, dq.Q6_K), 512, 4, 2, 64)
    for pos in (-1, p.cap, 64):      # negative, past the cache, past the RoPE table (cap 80)
        p.cap = 80 if pos == 64 else 40
        q, kc, vc = p.run(K, pos)
        assert torch.isnan(q).all()
        assert not kc.any() and not vc.any()


def test_mqkv_deterministic_and_graph_replay(K):
    p = Qkv(K, (dq.Q4_K, dq.Q4_K, dq.Q6_K), 3584, 28, 4, 128, seed=3)
    caches = (torch.zeros(4, 40, 128, device=DEV), torch.zeros(4, 40, 128, device=DEV))
    q0, kc, vc = p.run(K, 7, caches=caches)
    q0, k0, v0 = q0.clone(), kc.clone(), vc.clone()
    q1, _, _ = p.run(K, 7, caches=caches)
    assert torch.equal(q0, q1)
    x, nw = T(p.x), T(p.nw)
    b = [T(v) for v in p.bs]
    cs, sn, pos = T(p.cos), T(p.sin), torch.tensor([7], device=DEV)
    out = torch.empty(28, 128, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        K.qkv_rmsnorm_rope(x, nw, 1e-6, *p.ws, *b, cs, sn, pos, *caches, 28, out=out)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        K.qkv_rmsnorm_rope(x, nw, 1e-6, *p.ws, *b, cs, sn, pos, *caches, 28, out=out)
    for _ in range(3):
        out.zero_()
        caches[0].zero_()
        caches[1].zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, q0)
        assert torch.equal(caches[0], k0) and torch.equal(caches[1], v0)
