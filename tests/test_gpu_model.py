"""End-to-end GPU parity: Engine (HIP path) vs the torch-CPU oracle of the reference forward.

* tiny 2-layer model of the 0.5B family (all four formats): prefill and decode logits within
  1e-3 relative, greedy tokens identical, graph replay == eager (the reference's
  test_integration.py:29-59 idea, here bitwise);
* config 0 (Qwen2.5-0.5B architecture, Q4_K_M-style mix, seed 0): the 64 greedy tokens of
  the committed fixture tests/golden/config0_greedy.json, produced by the oracle.
"""

import json

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from helpers import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3
# the autocast prefill against the oracle's autocast mode (both fp16 at the same points; the
# fp32 forward is ~1e-3 away at config 0)
AUTOCAST_TOL = 1e-3


@pytest.fixture(scope="module")
def tiny(tiny_model):
    from pico_hip.engine import Engine
    from oracle.ref_cpu import RefModel
    return Engine(tiny_model), RefModel(tiny_model)


def test_prefill_and_decode_logits_match_oracle(tiny):
    eng, ref = tiny
    ids = [3, 500, 17, 999, 42, 7, 256, 1023, 0, 64, 65, 300, 12]
    cap = len(ids) + 8
    cache = eng._empty_cache(cap)
    rcache = ref.empty_cache(cap)
    lg = eng.model.forward(torch.tensor(ids, device=eng.device), torch.arange(len(ids), device=eng.device), cache)
    rl = ref.forward(torch.tensor(ids), torch.arange(len(ids)), rcache)
    assert rel_err(lg.cpu().numpy(), rl.numpy()) < TOL
    for c, rc in zip(cache, rcache):  # the prefill filled the same KV
        assert rel_err(c[0][:, :len(ids)].cpu().numpy(), rc[0][:, :len(ids)].numpy()) < TOL
    tok = int(rl.argmax())
    for step in range(8):
        pos = len(ids) + step
        lg = eng.model.forward(torch.tensor([tok], device=eng.device), torch.tensor([pos], device=eng.device), cache)
        rl = ref.forward(torch.tensor([tok]), torch.tensor([pos]), rcache)
        assert rel_err(lg.cpu().numpy(), rl.numpy()) < TOL, step
        tok = int(rl.argmax())


def test_greedy_tokens_match_oracle(tiny):
    eng, ref = tiny
    ids = [1, 2, 3, 4, 5, 900, 800, 700]
    want, margins = ref.greedy(ids, 24)
    got = eng.generate_ids(ids, 24, temperature=0.0, use_graph=True)
    assert got == want, (got, want, margins)


def test_device_greedy_equals_host_loop_and_stops_at_eos(tiny):
    """Greedy picks made on the device (graph replays, chunked log reads) give the ids of the
    host loop argmax -> eos check -> decode step (evidence.py:117-123), eos included."""
    eng, _ = tiny
    ids = [11, 22, 33, 44]
    host = eng.generate_ids(ids, 20, temperature=0.0, use_graph=False)
    assert len(host) == 20
    for chunk in (16, 3, 1):
        eng.greedy_chunk = chunk
        assert eng.generate_ids(ids, 20, temperature=0.0, use_graph=True) == host, chunk
    eng.greedy_chunk = 16
    for eos in (host[0], host[5], host[19]):
        want = host[:host.index(eos)]
        assert eng.generate_ids(ids, 20, temperature=0.0, use_graph=True, eos_id=eos) == want
        assert eng.generate_ids(ids, 20, temperature=0.0, use_graph=False, eos_id=eos) == want
    assert eng.generate_ids(ids, 0, temperature=0.0, use_graph=True) == []
    assert eng.generate_ids(ids, 1, temperature=0.0, use_graph=True) == host[:1]


@pytest.mark.parametrize("step_kernel", [False, True])
def test_graph_equals_eager(tiny, step_kernel):
    """The captured greedy step replays the eager greedy step bit for bit (both decode-step
    paths: four launches per layer, or the one-launch step kernel)."""
    eng, _ = tiny
    eng.model.use_step_kernel = step_kernel
    try:
        ids = [9, 8, 7, 6, 5]
        cache = eng._empty_cache(len(ids) + 8)
        graph = eng._build_decode_graph(cache)
        assert graph is not None, "graph capture failed"
        greedy = eng._greedy
        logits = eng.model.forward(torch.tensor(ids, device=eng.device), torch.arange(len(ids), device=eng.device), cache)
        nxt = int(logits.argmax())
        for step in range(8):
            pos = len(ids) + step
            # eager first, then the graph replays the same step over the same cache slot
            eager = eng.model.forward(torch.tensor([nxt], device=eng.device),
                                      torch.tensor([pos], device=eng.device), cache, greedy).clone()
            torch.cuda.synchronize()
            g = eng._decode_step(nxt, pos, cache, graph).clone()
            torch.cuda.synchronize()
            assert torch.equal(eager, g), f"graph diverged from eager at step {step}"
            nxt = int(eager.argmax())
        assert eng.model.step_error() == 0
    finally:
        eng.model.use_step_kernel = False


def test_mid_cache_decode_split_gproj(tiny):
    """Caches of 513..4096 positions run attn_split_gproj (split attention, then the records
    merged per kv group with the group's Wo columns): decode logits within 1e-3 of the oracle,
    and each graph replay equal to the same step run eagerly, bit for bit."""
    eng, ref = tiny
    m = eng.model
    saved = m.prefill_f16_min_tokens
    m.prefill_f16_min_tokens = None  # the oracle's fp32 prefill
    try:
        ids = np.random.default_rng(5).integers(0, 1024, size=520).tolist()
        cap = len(ids) + 8
        assert m.split_gproj_capacity[0] <= cap <= m.split_gproj_capacity[1]
        cache, rcache = eng._empty_cache(cap), ref.empty_cache(cap)
        graph = eng._build_decode_graph(cache)
        assert graph is not None, "graph capture failed"
        greedy = eng._greedy
        lg = m.forward(torch.tensor(ids, device=eng.device), torch.arange(len(ids), device=eng.device), cache)
        rl = ref.forward(torch.tensor(ids), torch.arange(len(ids)), rcache)
        assert rel_err(lg.cpu().numpy(), rl.numpy()) < TOL
        tok = int(rl.argmax())
        for step in range(4):
            pos = len(ids) + step
            eager = m.forward(torch.tensor([tok], device=eng.device), torch.tensor([pos], device=eng.device),
                              cache, greedy).clone()
            rl = ref.forward(torch.tensor([tok]), torch.tensor([pos]), rcache)
            assert rel_err(eager.cpu().numpy(), rl.numpy()) < TOL, step
            torch.cuda.synchronize()
            g = eng._decode_step(tok, pos, cache, graph).clone()
            torch.cuda.synchronize()
            assert torch.equal(eager, g), f"graph diverged from eager at step {step}"
            tok = int(rl.argmax())
    finally:
        m.prefill_f16_min_tokens = saved


PATHS = {  # model flags of each path of the decode step
    "three_launch": dict(use_attn_oproj=False, use_attn_gproj=False, use_step_kernel=False),
    "attn_gproj": dict(use_attn_oproj=False, use_attn_gproj=True, use_step_kernel=False),
    "attn_oproj": dict(use_attn_oproj=True, use_ffn_fix=False, use_step_kernel=False),
    "ffn_fix": dict(use_attn_oproj=True, use_ffn_fix=True, use_step_kernel=False),
    "step_kernel": dict(use_attn_oproj=False, use_step_kernel=True),
}


def _set_path(m, path):
    old = {k: getattr(m, k) for k in PATHS[path]}
    for k, v in PATHS[path].items():
        setattr(m, k, v)
    return old


def test_fused_attention_block_equals_three_launch_path(tiny):
    """Every path of the greedy decode step -- the three-launch layers (staged QKV over the
    down-product replicas, attn_oproj_fix, the fused FFN ffn_fix), the per-head attention +
    o-projection (attn_oproj_fix with the fixed-point gate/up), attn_gproj with the partial-sum gate/up, the
    three-launch block (qkv_rmsnorm_rope, decode_attn, qgemv) and the one-launch step kernel --
    gives the same decode logits to 1e-3 and the same greedy ids."""
    from pico_hip import kernels as K
    eng, _ = tiny
    m = eng.model
    ids = [5, 6, 7, 8, 9, 10]
    outs = {}
    for path in PATHS:
        old = _set_path(m, path)
        cache = eng._empty_cache(len(ids) + 10)
        greedy = K.GreedyState(m.output.n, len(ids) + 10, eng.device)
        lg = m.forward(torch.tensor(ids, device=eng.device), torch.arange(len(ids), device=eng.device), cache)
        seq = []
        tok = int(lg.argmax())
        for step in range(10):
            lg = m.forward(torch.tensor([tok], device=eng.device),
                           torch.tensor([len(ids) + step], device=eng.device), cache, greedy)
            seq.append(lg.cpu().numpy())
            nxt = int(lg.argmax())
            assert int(greedy.state[0]) == nxt, (path, step)   # the device pick
            tok = nxt
        outs[path] = seq
        for k, v in old.items():
            setattr(m, k, v)
    assert m.step_error() == 0
    for path in PATHS:
        for a, b in zip(outs[path], outs["three_launch"]):
            assert rel_err(a, b) < TOL, path
            assert int(np.argmax(a)) == int(np.argmax(b)), path


@pytest.mark.parametrize("path", list(PATHS))
def test_config0_greedy_matches_fixture(model_dir, path):
    """Qwen2.5-0.5B-architecture synthetic model, 13-token seeded prompt, 64 greedy tokens,
    with each attention-block path of the decode step."""
    from pico_hip import synth
    from pico_hip.engine import Engine
    fx = json.loads((GOLDEN / "config0_greedy.json").read_text())
    gguf = synth.cached(synth.ARCHES["qwen2.5-0.5b"], seed=fx["seed"], cache_dir=model_dir)
    assert synth.sha256(gguf) == fx["gguf_sha256"], "synthetic model is not byte-identical"
    eng = Engine(gguf)
    _set_path(eng.model, path)
    cap = len(fx["prompt_ids"]) + fx["n_tokens"]
    assert eng.model.attn_oproj_ok(cap) == (path in ("attn_oproj", "ffn_fix"))
    assert eng.model.ffn_fix_ok(cap) == (path == "ffn_fix")
    got = eng.generate_ids(fx["prompt_ids"], fx["n_tokens"], temperature=0.0, use_graph=True)
    first_diff = next((i for i, (a, b) in enumerate(zip(got, fx["tokens"])) if a != b), None)
    assert got == fx["tokens"], f"first mismatch at step {first_diff} (margin {fx['margins'][first_diff]})"


def test_prefill_f16_close_to_fp32_path(tiny):
    """The matrix-core prefill (fp16 operands, fp32 accumulation) against the fp32 prefill on
    the same 300-token prompt: logits, the KV cache it leaves, and the decode step after it."""
    eng, _ = tiny
    m = eng.model
    ids = [(7 * i + 3) % 1024 for i in range(300)]
    saved = m.prefill_f16_min_tokens
    out = {}
    try:
        for mode, thr in (("fp32", None), ("f16", 2)):
            m.prefill_f16_min_tokens = thr
            cache = eng._empty_cache(len(ids) + 4)
            lg = m.forward(torch.tensor(ids, device=eng.device), torch.arange(len(ids), device=eng.device), cache)
            nxt = int(lg.argmax())
            lg2 = m.forward(torch.tensor([nxt], device=eng.device), torch.tensor([len(ids)], device=eng.device), cache)
            out[mode] = (lg.cpu().numpy(), [c[0][:, :len(ids)].cpu().numpy() for c in cache], lg2.cpu().numpy())
    finally:
        m.prefill_f16_min_tokens = saved
    (l32, c32, d32), (l16, c16, d16) = out["fp32"], out["f16"]
    assert rel_err(l16, l32) < 2e-2
    for a, b in zip(c16, c32):
        assert rel_err(a, b) < 2e-2
    assert rel_err(d16, d32) < 2e-2
    assert m._f16 is not None and len(m._f16) == len(m.layers)


@pytest.mark.parametrize("n_tokens", [300, 1100])
def test_prefill_hipblaslt_products_match_mfma_products(tiny, n_tokens):
    """The matrix-core prefill with its plain products (QKV + bias, o-proj and ffn_down +
    residual) on hipBLASLt against the default prefill with every product on this library's
    GEMMs (pe_gemm_h16; 1100 tokens: its long-prompt kernel): the operands are the same fp16
    values, only the fp32 summation order differs (1e-4)."""
    eng, _ = tiny
    m = eng.model
    ids = [(5 * i + 1) % 1024 for i in range(n_tokens)]
    saved = m.prefill_f16_min_tokens, m.prefill_blaslt
    out = {}
    try:
        m.prefill_f16_min_tokens = 2
        for lt in (True, False):
            m.prefill_blaslt = lt
            cache = eng._empty_cache(len(ids) + 1)
            lg = m.forward(torch.tensor(ids, device=eng.device), torch.arange(len(ids), device=eng.device), cache)
            out[lt] = (lg.cpu().numpy(), cache[-1][0][:, :len(ids)].cpu().numpy())
    finally:
        m.prefill_f16_min_tokens, m.prefill_blaslt = saved
    assert rel_err(out[True][0], out[False][0]) < 1e-4
    assert rel_err(out[True][1], out[False][1]) < 1e-4


# ---- the 7B family: head_dim 128, 7 query heads per kv head, Q4_K/Q6_K
# attention and FFN, untied Q8_0 LM head -----------------------------------------------------

def _tiny7b_arch():
    from pico_hip import synth
    return synth.tiny_arch(n_layers=2, hidden=1792, n_head=14, n_kv=2, head_dim=128, ffn=1024,
                           vocab=2048, name="qwen2.5-7b-tiny", tied=False)


@pytest.fixture(scope="module")
def tiny7b(model_dir):
    from pico_hip import synth
    from pico_hip.engine import Engine
    from oracle.ref_cpu import RefModel
    path = model_dir / "tiny7b-2l.gguf"
    if not path.exists():
        synth.build(path, _tiny7b_arch(), seed=5)
    return Engine(path), RefModel(path)


def test_7b_family_logits_match_oracle(tiny7b):
    """Prefill (fp32) and eight decode steps on the 7B-family model: logits within 1e-3 of
    the oracle, the cache the prefill leaves within 1e-3."""
    eng, ref = tiny7b
    assert eng.cfg.head_dim == 128 and eng.cfg.n_head // eng.cfg.n_kv_head == 7
    ids = [3, 500, 17, 999, 42, 7, 256, 1023, 0, 64, 65, 300, 2047]
    cap = len(ids) + 8
    cache, rcache = eng._empty_cache(cap), ref.empty_cache(cap)
    lg = eng.model.forward(torch.tensor(ids, device=eng.device), torch.arange(len(ids), device=eng.device), cache)
    rl = ref.forward(torch.tensor(ids), torch.arange(len(ids)), rcache)
    assert rel_err(lg.cpu().numpy(), rl.numpy()) < TOL
    for c, rc in zip(cache, rcache):
        assert rel_err(c[1][:, :len(ids)].cpu().numpy(), rc[1][:, :len(ids)].numpy()) < TOL
    tok = int(rl.argmax())
    for step in range(8):
        pos = len(ids) + step
        lg = eng.model.forward(torch.tensor([tok], device=eng.device), torch.tensor([pos], device=eng.device), cache)
        rl = ref.forward(torch.tensor([tok]), torch.tensor([pos]), rcache)
        assert rel_err(lg.cpu().numpy(), rl.numpy()) < TOL, step
        tok = int(rl.argmax())


def test_7b_family_greedy_matches_oracle(tiny7b):
    """32 greedy tokens through the graph-replayed step with the device-side pick."""
    eng, ref = tiny7b
    ids = [1, 2, 3, 4, 5, 900, 800, 700]
    want, margins = ref.greedy(ids, 32)
    got = eng.generate_ids(ids, 32, temperature=0.0, use_graph=True)
    assert got == want, (got, want, margins)


def test_device_built_model_matches_oracle(tmp_path):
    """A model drawn and quantized on the GPU (the 7B benchmark's build path): the file is
    read back by the oracle on the CPU, and the HIP engine's greedy tokens equal the oracle's.
    Two builds with the same seed are byte-identical."""
    from pico_hip import synth
    from pico_hip.engine import Engine
    from oracle.ref_cpu import RefModel
    arch = _tiny7b_arch()
    h1 = synth.build(tmp_path / "a.gguf", arch, seed=9, device=DEV_GPU)
    h2 = synth.build(tmp_path / "b.gguf", arch, seed=9, device=DEV_GPU)
    assert h1 == h2
    eng, ref = Engine(tmp_path / "a.gguf"), RefModel(tmp_path / "a.gguf")
    ids = [10, 20, 30, 40, 50]
    want, margins = ref.greedy(ids, 16)
    assert eng.generate_ids(ids, 16, temperature=0.0, use_graph=True) == want, margins


DEV_GPU = "cuda"


def test_7b_family_prefill_f16_close_to_fp32_path(tiny7b):
    """The matrix-core prefill at head_dim 128 (fp16 GEMMs + the fp32 prefill attention)
    against the fp32 prefill on the same 100-token prompt: logits and the decode step after."""
    eng, _ = tiny7b
    m = eng.model
    ids = [(11 * i + 5) % 2048 for i in range(100)]
    saved = m.prefill_f16_min_tokens
    out = {}
    try:
        for mode, thr in (("fp32", None), ("f16", 2)):
            m.prefill_f16_min_tokens = thr
            cache = eng._empty_cache(len(ids) + 2)
            lg = m.forward(torch.tensor(ids, device=eng.device), torch.arange(len(ids), device=eng.device), cache)
            nxt = int(lg.argmax())
            lg2 = m.forward(torch.tensor([nxt], device=eng.device), torch.tensor([len(ids)], device=eng.device), cache)
            out[mode] = (lg.cpu().numpy(), lg2.cpu().numpy())
    finally:
        m.prefill_f16_min_tokens = saved
    assert rel_err(out["f16"][0], out["fp32"][0]) < 2e-2
    assert rel_err(out["f16"][1], out["fp32"][1]) < 2e-2


# ---- the reference's CUDA prefill numerics (fp16 autocast, model.py:147-151) ----------------

def _autocast_prefill(eng, ids):
    m = eng.model
    old = m.prefill_autocast
    m.prefill_autocast = True
    try:
        cache = eng._empty_cache(len(ids) + 4)
        lg = m.forward(torch.tensor(ids, device=eng.device), torch.arange(len(ids), device=eng.device), cache)
        return lg.cpu().numpy(), cache
    finally:
        m.prefill_autocast = old


def test_autocast_prefill_matches_oracle_autocast(tiny):
    """prefill_autocast against the oracle's autocast mode: far closer than to the fp32
    forward (whose distance is the size of the fp16 roundings), and the KV cache it leaves holds
    fp16 values equal to the oracle's."""
    eng, ref = tiny
    ids = [3, 500, 17, 999, 42, 7, 256, 1023, 0, 64, 65, 300, 12]
    lg, cache = _autocast_prefill(eng, ids)
    rcache = ref.empty_cache(len(ids) + 4)
    ra = ref.forward(torch.tensor(ids), torch.arange(len(ids)), rcache, autocast=True).numpy()
    rf = ref.forward(torch.tensor(ids), torch.arange(len(ids)), ref.empty_cache(len(ids))).numpy()
    d_ac, d_fp32 = rel_err(lg, ra), rel_err(lg, rf)
    print(f"tiny autocast: vs oracle autocast {d_ac:.3e}, vs oracle fp32 {d_fp32:.3e}")
    assert d_ac < AUTOCAST_TOL
    assert d_fp32 > 3 * d_ac
    for c, rc in zip(cache, rcache):
        k = c[0][:, :len(ids)].cpu()
        assert torch.equal(k, k.half().float())                      # fp16 values
        assert rel_err(k.numpy(), rc[0][:, :len(ids)].numpy()) < AUTOCAST_TOL


def test_config0_autocast_prefill_matches_fixture(model_dir):
    """Config 0's 13-token prompt prefilled with the reference's CUDA numerics: the logits at
    the fixture's 4096 indices (the 2048 largest and 2048 random others) against the oracle's
    autocast mode, relative to the largest logit. Over 24 layers two implementations of the
    same fp16 rounding points drift apart (an fp32 sum that lands near an fp16 tie rounds to
    either neighbour, and the difference feeds every later layer): 5.0e-4 measured, against
    9.8e-4 to the fp32 forward; the tiny model above separates the two by 20x."""
    from pico_hip import synth
    from pico_hip.engine import Engine
    fx = json.loads((GOLDEN / "config0_autocast_logits.json").read_text())
    gguf = synth.cached(synth.ARCHES["qwen2.5-0.5b"], seed=0, cache_dir=model_dir)
    assert synth.sha256(gguf) == fx["gguf_sha256"], "synthetic model is not byte-identical"
    eng = Engine(gguf)
    lg, _ = _autocast_prefill(eng, fx["prompt_ids"])
    idx = np.array(fx["idx"])
    scale = fx["max_abs_autocast"]
    d_ac = float(np.abs(lg[idx] - np.array(fx["autocast"])).max() / scale)
    d_fp32 = float(np.abs(lg[idx] - np.array(fx["fp32"])).max() / scale)
    print(f"config 0 autocast: vs oracle autocast {d_ac:.3e}, vs oracle fp32 {d_fp32:.3e}")
    assert d_ac < AUTOCAST_TOL
    assert d_ac < 0.75 * d_fp32
    assert int(np.argmax(lg)) == fx["argmax_autocast"]
