"""Parity at the full sizes of BASELINE configs 3 and 4 (run on an MI355X: pytest -m gpu).

Config 3 (the config-0 model, 8192-token prompt, decode at context 8192): causal flash
attention over 8192 positions against float64 on sampled query rows; the model's 8192-token
matrix-core prefill and eight decode steps after it against the CPU oracle. The same model
(config 0) through 24 decode steps fed random ids, against the CPU oracle.

Config 4 (Qwen2.5-7B architecture): the decode GEMVs at their full shapes against float64 on
sampled rows (gate/up 3584 -> 2 x 18944 Q4_K with SiLU, ffn_down 18944 -> 3584 Q6_K with the
residual, the 3584 -> 152064 Q8_0 LM head with its fused greedy pick, o-proj 3584 -> 3584
Q4_K; the QKV prologue at 3584 -> 28 x 128 + 2 x 4 x 128 is in test_gpu_kernels.py), and the
28-layer model through Engine: against the oracle's forward and against itself (graph replay
== eager bit for bit, device pick == argmax of the eager logits). The 7B oracle runs the
reference's forward (oracle/ref_cpu.py) on torch's own fp32 GPU ops, over weights dequantized
by pe_dequantize, which is bit-exact to the oracle's dequantizer (test_dequant_* in
test_gpu_kernels.py); its 30 GB of fp32 weights are too large for a quick CPU run.

Also Q5_0 896 -> 151936 (a config-1 shape on the looped GEMV form).
"""

import numpy as np
import pytest
import torch

from helpers import dequant_rows, random_quant, rel_err
from oracle import closed
from oracle import dequant as dq

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-3            # fp32 accumulation
TOL_FLASH = 2e-3      # fp16 operands, probabilities rounded to fp16 inside the kernel
# The matrix-core prefill multiplies fp16-rounded activations and weights (fp32 accumulation,
# fp32 residual stream) where the oracle multiplies fp32. Each operand rounds by at most 2^-11
# relative, so one product is off by at most ~1e-3 of its size; the rounding errors are
# uncorrelated along a dot product and across layers, and the measured maximum over the
# logits, every layer's sampled K/V rows and the decode steps after an 8192-token prefill is
# 3.2e-4. The bound is twice the one-product worst case.
TOL_F16_PREFILL = 2e-3


@pytest.fixture(scope="module")
def K():
    from pico_hip import kernels
    return kernels


def dev_bytes(raw: bytes) -> torch.Tensor:
    return torch.from_numpy(np.frombuffer(raw, np.uint8).copy()).to(DEV)


def qweight(K, t, raw, n, k):
    return K.pack_weight(dev_bytes(raw), t, n, k)


def sample_rows(n: int, count: int, seed: int, extra=()) -> np.ndarray:
    rows = np.random.default_rng(seed).choice(n, count, replace=False)
    return np.unique(np.concatenate([rows, [0, 1, n - 2, n - 1], list(extra)]).astype(np.int64))


def rows_of(t, raw: bytes, n: int, k: int, rows) -> np.ndarray:
    """The dequantized rows ``rows`` of an (n, k) weight in GGUF block order."""
    blk = np.frombuffer(raw, np.uint8).reshape(n, -1)[rows]
    return dequant_rows(t, blk.tobytes(), len(rows), k)


# ---- config 3: flash attention over 8192 positions ----------------------------------------

@pytest.mark.parametrize("L,pos0", [(8192, 0), (4096, 4000)])
def test_flash_prefill_full_length_sampled_rows(K, L, pos0):
    """14/2 heads, head_dim 64 (the config-0 model), against float64 attention on the same
    fp16-rounded q, k, v for 64 random query rows plus the first, the last and the rows either
    side of the 32-row query blocks and 64-position key tiles."""
    n_head, n_kv, hd = 14, 2, 64
    cap = pos0 + L + 3
    rng = np.random.default_rng(L + pos0)
    h16 = lambda a: a.astype(np.float16).astype(np.float32)
    q = h16(rng.standard_normal((L, n_head, hd)).astype(np.float32))
    k = h16(rng.standard_normal((n_kv, cap, hd)).astype(np.float32))
    v = h16(rng.standard_normal((n_kv, cap, hd)).astype(np.float32))
    out = K.flash_prefill(torch.from_numpy(q).to(DEV), torch.from_numpy(k).to(DEV),
                          torch.from_numpy(v).to(DEV), pos0=pos0).cpu().numpy()
    assert out.shape == (L, n_head * hd)
    edges = [31, 32, 63, 64, 127, 128, L // 2 - 1, L // 2, L - 33, L - 32]
    rows = sample_rows(L, 64, seed=L, extra=edges)
    k64, v64 = k.astype(np.float64), v.astype(np.float64)
    ref = np.stack([closed.attention(q[i], k64, v64, pos0 + i + 1) for i in rows])
    assert rel_err(out[rows], ref.reshape(len(rows), -1)) < TOL_FLASH


# ---- config 3: the config-0 model at context 8192 -----------------------------------------

@pytest.fixture(scope="module")
def cfg0(model_dir):
    """The config-0 model (Qwen2.5-0.5B architecture, seed 0): its arch, Engine and CPU oracle."""
    from pico_hip import synth
    from pico_hip.engine import Engine
    from oracle.ref_cpu import RefModel
    arch = synth.ARCHES["qwen2.5-0.5b"]
    path = synth.cached(arch, seed=0, cache_dir=model_dir)
    return arch, Engine(path), RefModel(path)


def test_config0_decode_teacher_forced_matches_oracle(cfg0):
    """The config-0 model at full size: a 13-token prompt, then 24 graph-replayed decode steps
    fed seeded random ids (its own greedy picks settle into a two-token cycle, which would
    exercise two embedding and LM-head rows), including the first and last vocabulary rows:
    every step's logits against the CPU oracle, and the device pick equal to the argmax."""
    arch, eng, ref = cfg0
    rng = np.random.default_rng(24)
    prompt = rng.integers(0, arch.vocab, size=13)
    feed = [0, arch.vocab - 1] + rng.integers(0, arch.vocab, size=22).tolist()
    cap = len(prompt) + len(feed)
    cache, rcache = eng._empty_cache(cap), ref.empty_cache(cap)
    graph = eng._build_decode_graph(cache)
    assert graph is not None
    lg = eng.model.forward(torch.from_numpy(prompt).to(DEV), torch.arange(13, device=DEV), cache)
    rl = ref.forward(torch.from_numpy(prompt), torch.arange(13), rcache)
    assert rel_err(lg.cpu().numpy(), rl.numpy()) < TOL
    for s, tok in enumerate(feed):
        pos = 13 + s
        got = eng._decode_step(tok, pos, cache, graph).cpu().numpy()
        assert int(eng._greedy.token) == int(np.argmax(got)), s
        rl = ref.forward(torch.tensor([tok]), torch.tensor([pos]), rcache)
        assert rel_err(got, rl.numpy()) < TOL, s


def test_config3_prefill_8192_and_decode_match_oracle(cfg0):
    """The config-0 model (seed 0) with an 8192-token random prompt: the matrix-core prefill's
    logits and the K/V rows it leaves in every layer (sampled positions) against the CPU
    oracle's fp32 prefill, then eight graph-replayed decode steps at context 8192, fed the
    oracle's greedy tokens, against the oracle's decode steps on its own cache."""
    arch, eng, ref = cfg0
    L, steps = 8192, 8
    assert eng.model.prefill_f16_min_tokens is not None and eng.model.prefill_f16_min_tokens <= L
    ids = np.random.default_rng(8192).integers(0, arch.vocab, size=L)
    cap = L + steps
    cache = eng._empty_cache(cap)
    graph = eng._build_decode_graph(cache)   # before the prefill: its warm-up steps write rows
    assert graph is not None
    lg = eng.model.forward(torch.from_numpy(ids).to(DEV), torch.arange(L, device=DEV), cache)
    lg = lg.cpu().numpy()
    rcache = ref.empty_cache(cap)
    rl = ref.forward(torch.from_numpy(ids), torch.arange(L), rcache)
    errs = {"prefill_logits": rel_err(lg, rl.numpy())}
    pos = sample_rows(L, 60, seed=3, extra=[L // 2])
    for i, ((kc, vc), (rk, rv)) in enumerate(zip(cache, rcache)):
        errs[f"k{i}"] = rel_err(kc[:, pos].cpu().numpy(), rk[:, pos].numpy())
        errs[f"v{i}"] = rel_err(vc[:, pos].cpu().numpy(), rv[:, pos].numpy())
    tok = int(rl.argmax())
    for s in range(steps):
        got = eng._decode_step(tok, L + s, cache, graph)
        pick = int(eng._greedy.token)
        got = got.cpu().numpy()
        assert np.all(np.isfinite(got))
        assert pick == int(np.argmax(got)), s           # the device-side greedy pick
        rl = ref.forward(torch.tensor([tok]), torch.tensor([L + s]), rcache)
        errs[f"decode{s}"] = rel_err(got, rl.numpy())
        tok = int(rl.argmax())
    print("config 3 relative errors:", {k: f"{v:.2e}" for k, v in errs.items()})
    bad = {k: v for k, v in errs.items() if not v < TOL_F16_PREFILL}
    assert not bad, bad


# ---- config 4: the 7B decode GEMVs at full size -------------------------------------------

def test_7b_gate_up_silu_full_shape(K):
    """3584 -> 2 x 18944 Q4_K: RMSNorm, the [gate; up] GEMV and SiLU(gate) * up in one launch."""
    t, k, ffn = dq.Q4_K, 3584, 18944
    raw = random_quant(t, 2 * ffn, k, seed=1)
    w = qweight(K, t, raw, 2 * ffn, k)
    rng = np.random.default_rng(2)
    x = rng.standard_normal(k).astype(np.float32)
    nw = rng.standard_normal(k).astype(np.float32)
    act = K.qgemv_norm_silu(torch.from_numpy(x).to(DEV), torch.from_numpy(nw).to(DEV), w, 1e-6).cpu().numpy()
    rows = sample_rows(ffn, 512, seed=3, extra=[255, 256, ffn // 2])
    h = closed.rmsnorm(x, nw, 1e-6)
    g = closed.gemv(rows_of(t, raw, 2 * ffn, k, rows), h)
    u = closed.gemv(rows_of(t, raw, 2 * ffn, k, rows + ffn), h)
    assert rel_err(act[rows], closed.silu_mul(g, u)) < TOL


def test_7b_ffn_down_residual_full_shape(K):
    """18944 -> 3584 Q6_K with the residual added (1024 sampled rows in float64)."""
    t, k, n = dq.Q6_K, 18944, 3584
    raw = random_quant(t, n, k, seed=4)
    w = qweight(K, t, raw, n, k)
    rng = np.random.default_rng(5)
    x = rng.standard_normal(k).astype(np.float32)
    r = rng.standard_normal(n).astype(np.float32)
    y = K.qgemv(torch.from_numpy(x).to(DEV), w, residual=torch.from_numpy(r).to(DEV)).cpu().numpy()
    rows = sample_rows(n, 1024, seed=6, extra=[255, 256, n // 2])
    assert rel_err(y[rows], closed.gemv(rows_of(t, raw, n, k, rows), x, residual=r[rows])) < TOL


def test_7b_oproj_residual_full_shape(K):
    """3584 -> 3584 Q4_K with the residual (the o-projection of the head_dim-128 path)."""
    t, k, n = dq.Q4_K, 3584, 3584
    raw = random_quant(t, n, k, seed=6)
    w = qweight(K, t, raw, n, k)
    rng = np.random.default_rng(7)
    x = rng.standard_normal(k).astype(np.float32)
    r = rng.standard_normal(n).astype(np.float32)
    y = K.qgemv(torch.from_numpy(x).to(DEV), w, residual=torch.from_numpy(r).to(DEV)).cpu().numpy()
    assert rel_err(y, closed.gemv(dequant_rows(t, raw, n, k), x, residual=r)) < TOL


def test_7b_lm_head_and_pick_full_shape(K):
    """3584 -> 152064 Q8_0 after the final RMSNorm, with the fused greedy pick: every logit
    against float64, and the picked row's float64 logit equal to the float64 maximum to the
    logits' tolerance (an exact tie-free check would need exact arithmetic)."""
    t, k, n = dq.Q8_0, 3584, 152064
    raw = random_quant(t, n, k, seed=8)
    w = qweight(K, t, raw, n, k)
    rng = np.random.default_rng(9)
    x = rng.standard_normal(k).astype(np.float32)
    nw = rng.standard_normal(k).astype(np.float32)
    g = K.GreedyState(n, 4, DEV)
    g.reset(11, 100, 0)
    logits = K.qgemv_norm_argmax(torch.from_numpy(x).to(DEV), torch.from_numpy(nw).to(DEV), w, 1e-6, g)
    pick = int(g.state[0])
    got = logits.cpu().numpy()
    assert pick == int(np.argmax(got)) and g.state.tolist()[1:] == [101, 1]
    h = closed.rmsnorm(x, nw, 1e-6)
    blk = np.frombuffer(raw, np.uint8).reshape(n, -1)
    ref = np.empty(n)
    for r0 in range(0, n, 16384):
        r1 = min(n, r0 + 16384)
        ref[r0:r1] = closed.gemv(dequant_rows(t, blk[r0:r1].tobytes(), r1 - r0, k), h)
    assert rel_err(got, ref) < TOL
    scale = np.max(np.abs(ref))
    assert ref[pick] >= ref.max() - TOL * scale


def test_q5_0_lm_head_shape(K):
    """896 -> 151936 Q5_0 (config 1's largest Q5_0 shape), 4096 sampled rows in float64."""
    t, k, n = dq.Q5_0, 896, 151936
    raw = random_quant(t, n, k, seed=10)
    w = qweight(K, t, raw, n, k)
    x = np.random.default_rng(11).standard_normal(k).astype(np.float32)
    y = K.qgemv(torch.from_numpy(x).to(DEV), w).cpu().numpy()
    rows = sample_rows(n, 4096, seed=12, extra=[2047, 2048, n // 2])
    assert rel_err(y[rows], closed.gemv(rows_of(t, raw, n, k, rows), x)) < TOL


# ---- config 4: the 28-layer 7B-architecture model -----------------------------------------

def test_7b_model_matches_oracle_graph_and_pick(model_dir, K):
    """The 28-layer Qwen2.5-7B-architecture model drawn and quantized on the GPU (seed 0, the
    benchmark's model): a 16-token fp32 prefill and four decode steps against the oracle's
    forward (1e-3), each graph-replayed step equal bit for bit to the same step run eagerly on
    a copy of the cache, finite logits, and the device pick equal to the eager argmax; then
    the 128-token matrix-core prefill of the benchmark against the oracle's fp32 prefill."""
    from pico_hip import synth
    from pico_hip.engine import Engine
    from oracle.ref_cpu import RefModel
    arch = synth.ARCHES["qwen2.5-7b"]
    path = synth.cached(arch, seed=0, cache_dir=model_dir, device=DEV)
    eng = Engine(path)
    c = eng.cfg
    assert (c.n_layers, c.hidden, c.n_head, c.n_kv_head, c.head_dim, c.ffn_dim, c.vocab_size) == \
        (28, 3584, 28, 4, 128, 18944, 152064)
    ref = RefModel(path, unpack_quant=False, device=DEV,
                   dequantize=lambda gt, raw, n: K.dequantize(gt, dev_bytes(raw), n))
    rng = np.random.default_rng(7)
    ids = torch.from_numpy(rng.integers(0, arch.vocab, size=16)).to(DEV)
    L, steps = len(ids), 4
    cache = eng._empty_cache(L + steps)
    graph = eng._build_decode_graph(cache)
    assert graph is not None
    rcache = ref.empty_cache(L + steps)
    saved = eng.model.prefill_f16_min_tokens
    try:
        eng.model.prefill_f16_min_tokens = None               # fp32 prefill
        lg = eng.model.forward(ids, torch.arange(L, device=DEV), cache)
        rl = ref.forward(ids, torch.arange(L, device=DEV), rcache)
        assert rel_err(lg.cpu().numpy(), rl.cpu().numpy()) < TOL
        eager_cache = [(kc.clone(), vc.clone()) for kc, vc in cache]
        tok = int(rl.argmax())
        for s in range(steps):
            pos = L + s
            got = eng._decode_step(tok, pos, cache, graph).clone()
            pick = int(eng._greedy.token)
            eager = eng.model.forward(torch.tensor([tok], device=DEV), torch.tensor([pos], device=DEV),
                                      eager_cache)
            assert torch.equal(got, eager), s
            assert bool(torch.isfinite(got).all()), s
            assert pick == int(torch.argmax(eager)), s
            rl = ref.forward(torch.tensor([tok], device=DEV), torch.tensor([pos], device=DEV), rcache)
            assert rel_err(got.cpu().numpy(), rl.cpu().numpy()) < TOL, s
            tok = int(rl.argmax())
        # the benchmark's prefill: 128 tokens on the matrix cores (fp16 operands)
        eng.model.prefill_f16_min_tokens = 64
        ids = torch.from_numpy(rng.integers(0, arch.vocab, size=128)).to(DEV)
        cache, rcache = eng._empty_cache(128), ref.empty_cache(128)
        lg = eng.model.forward(ids, torch.arange(128, device=DEV), cache)
        rl = ref.forward(ids, torch.arange(128, device=DEV), rcache)
        err = rel_err(lg.cpu().numpy(), rl.cpu().numpy())
        print(f"7B 128-token fp16 prefill logits relative error {err:.2e}")
        assert err < TOL_F16_PREFILL
        # decode where the benchmark runs it: a cache of 384 positions (its 128-token prompt +
        # 256 steps), positions 360..365 after a 360-token matrix-core prefill, graph-replayed
        # steps against the same steps run eagerly (bit for bit) and against the oracle
        # continuing on its own fp32-prefilled cache (the fp16 prefill's tolerance)
        n0, cap = 360, 384
        ids = torch.from_numpy(rng.integers(0, arch.vocab, size=n0)).to(DEV)
        cache, rcache = eng._empty_cache(cap), ref.empty_cache(cap)
        graph = eng._build_decode_graph(cache)
        lg = eng.model.forward(ids, torch.arange(n0, device=DEV), cache)
        rl = ref.forward(ids, torch.arange(n0, device=DEV), rcache)
        assert rel_err(lg.cpu().numpy(), rl.cpu().numpy()) < TOL_F16_PREFILL
        eager_cache = [(kc.clone(), vc.clone()) for kc, vc in cache]
        tok = int(rl.argmax())
        for s in range(6):
            pos = n0 + s
            got = eng._decode_step(tok, pos, cache, graph).clone()
            eager = eng.model.forward(torch.tensor([tok], device=DEV), torch.tensor([pos], device=DEV),
                                      eager_cache)
            assert torch.equal(got, eager), pos
            assert int(eng._greedy.token) == int(torch.argmax(eager)), pos
            rl = ref.forward(torch.tensor([tok], device=DEV), torch.tensor([pos], device=DEV), rcache)
            err = rel_err(got.cpu().numpy(), rl.cpu().numpy())
            assert err < TOL_F16_PREFILL, (pos, err)
            tok = int(rl.argmax())
    finally:
        eng.model.prefill_f16_min_tokens = saved
