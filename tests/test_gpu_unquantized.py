"""Unquantized (F16 / F32) matrices on the HIP path, against the oracle.

The reference dequantizes every tensor to fp32 (engine.py:80-98) and multiplies any matrix it
has no quantized kernel for as fp32, the LM head included (model.py:163-164). Here F16/F32
matrices are read as stored by the same GEMV / QKV / attention-projection kernels. Three tiny
models of the 0.5B family: an untied F16 LM head; F16 o-projections with an F32 ffn_down in
one layer and F32 [gate; up] in another; and a file without output.weight (tied head)."""

import numpy as np
import pytest
import torch

from helpers import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _mix_f16_head(arch, layer, tensor):
    from pico_hip import synth
    from pico_hip.dequant import GGML_F16
    return GGML_F16 if tensor == "output" else synth.q4_k_m_mix(arch, layer, tensor)


def _mix_f16_oproj(arch, layer, tensor):
    from pico_hip import synth
    from pico_hip.dequant import GGML_F16, GGML_F32
    if tensor == "attn_output":
        return GGML_F16
    if tensor == "ffn_down" and layer == 1:
        return GGML_F32
    if tensor in ("ffn_gate", "ffn_up") and layer == 0:
        return GGML_F32
    return synth.q4_k_m_mix(arch, layer, tensor)


def _build(tmp_path_factory, name, mix, tied):
    from pico_hip import synth
    arch = synth.tiny_arch(n_layers=2, hidden=256, n_head=4, n_kv=2, head_dim=64, ffn=512,
                           vocab=1024, tied=tied)
    path = tmp_path_factory.mktemp(name) / "m.gguf"
    synth.build(path, arch, seed=11, mix=mix)
    return path


@pytest.fixture(scope="module")
def f16_head(tmp_path_factory):
    return _build(tmp_path_factory, "f16head", _mix_f16_head, tied=False)


@pytest.fixture(scope="module")
def f16_oproj(tmp_path_factory):
    return _build(tmp_path_factory, "f16oproj", _mix_f16_oproj, tied=True)


def _check_against_oracle(path, steps=8):
    from pico_hip.engine import Engine
    from oracle.ref_cpu import RefModel
    eng, ref = Engine(path), RefModel(path)
    ids = [3, 500, 17, 999, 42, 7, 256, 1023, 0, 64]
    cap = len(ids) + steps
    cache, rcache = eng._empty_cache(cap), ref.empty_cache(cap)
    lg = eng.model.forward(torch.tensor(ids, device=eng.device), torch.arange(len(ids), device=eng.device), cache)
    rl = ref.forward(torch.tensor(ids), torch.arange(len(ids)), rcache)
    assert rel_err(lg.cpu().numpy(), rl.numpy()) < TOL
    tok = int(rl.argmax())
    for step in range(steps):
        pos = len(ids) + step
        lg = eng.model.forward(torch.tensor([tok], device=eng.device), torch.tensor([pos], device=eng.device), cache)
        rl = ref.forward(torch.tensor([tok]), torch.tensor([pos]), rcache)
        assert rel_err(lg.cpu().numpy(), rl.numpy()) < TOL, step
        tok = int(rl.argmax())
    want, margins = ref.greedy([1, 2, 3, 4, 5, 900], 16)
    assert eng.generate_ids([1, 2, 3, 4, 5, 900], 16, temperature=0.0, use_graph=True) == want, margins
    return eng


def test_untied_f16_lm_head_matches_oracle(f16_head):
    from pico_hip.dequant import GGML_F16
    eng = _check_against_oracle(f16_head)
    assert eng.model.output.ggml_type == GGML_F16   # the file's own head, not token_embd
    assert eng.model.output.data.numel() == 1024 * 256 * 2


def test_f16_oproj_and_f32_ffn_matrices_match_oracle(f16_oproj):
    from pico_hip.dequant import GGML_F16, GGML_F32
    eng = _check_against_oracle(f16_oproj)
    assert eng.model.layers[0].wo.ggml_type == GGML_F16
    assert eng.model.layers[1].w_down.ggml_type == GGML_F32
    assert eng.model.layers[0].w_gate_up.ggml_type == GGML_F32


def test_file_without_output_weight_ties_head_to_embedding(f16_oproj, tmp_path):
    """A GGUF with no output.weight uses token_embd as the LM head: the same logits as the
    file that stores token_embd's bytes as output.weight."""
    from pico_hip import gguf
    from pico_hip.engine import Engine
    from oracle.ref_cpu import read_gguf
    meta, tensors = read_gguf(f16_oproj)
    out = tmp_path / "no_head.gguf"
    gguf.write(out, meta, [(n, tuple(sh), gt, raw) for n, (sh, gt, raw) in tensors.items()
                           if n != "output.weight"])
    a, b = Engine(f16_oproj), Engine(out)
    assert "output.weight" not in b.quant
    ids = torch.tensor([5, 6, 7, 8], device=a.device)
    la = a.model.forward(ids, torch.arange(4, device=a.device), a._empty_cache(8))
    lb = b.model.forward(ids, torch.arange(4, device=b.device), b._empty_cache(8))
    assert torch.equal(la, lb)


def test_graph_equals_eager_with_unquantized_matrices(f16_oproj):
    from pico_hip.engine import Engine
    eng = Engine(f16_oproj)
    ids = [9, 8, 7, 6, 5]
    cache = eng._empty_cache(len(ids) + 6)
    graph = eng._build_decode_graph(cache)
    assert graph is not None
    logits = eng.model.forward(torch.tensor(ids, device=eng.device), torch.arange(len(ids), device=eng.device), cache)
    nxt = int(logits.argmax())
    for step in range(6):
        pos = len(ids) + step
        eager = eng.model.forward(torch.tensor([nxt], device=eng.device), torch.tensor([pos], device=eng.device), cache).clone()
        torch.cuda.synchronize()
        g = eng._decode_step(nxt, pos, cache, graph).clone()
        torch.cuda.synchronize()
        assert torch.equal(eager, g), step
        nxt = int(eager.argmax())


@pytest.mark.parametrize("fmt", ["F16", "F32"])
def test_unquantized_gemv_and_dequant(fmt):
    """pe_qgemv / pe_dequant_tiled on F16/F32 rows: the dequantized matrix is the stored values
    bit for bit, and the GEMV is within 1e-3 of float64."""
    from pico_hip import kernels as K
    from pico_hip.dequant import GGML_F16, GGML_F32
    t = GGML_F16 if fmt == "F16" else GGML_F32
    g = torch.Generator().manual_seed(3)
    n, k = 1000, 896
    w = torch.randn(n, k, generator=g) * 0.02
    stored = w.half() if t == GGML_F16 else w
    raw = stored.contiguous().view(torch.uint8).reshape(-1).cuda()
    qw = K.pack_weight(raw, t, n, k)
    deq = K.dequantize_weight(qw)
    assert torch.equal(deq.cpu(), stored.float())
    x = torch.randn(k, generator=g)
    y = K.qgemv(x.cuda(), qw).cpu().double()
    want = stored.double() @ x.double()
    assert rel_err(y.numpy(), want.numpy()) < TOL
