"""Host-side logic on the CPU: GGUF read/write, synthetic-model determinism and type mix,
tokenizer, sampler, engine configuration."""

import numpy as np
import pytest
import torch

from oracle import dequant as dq
from oracle import ref_cpu


def test_gguf_roundtrip(tmp_path):
    from pico_hip import gguf
    from pico_hip.quantize import quantize
    w = np.random.default_rng(0).standard_normal(64 * 512).astype(np.float32)
    tensors = [("a.weight", (512, 64), dq.Q4_K, quantize(dq.Q4_K, w)),
               ("b.bias", (33,), dq.F32, np.arange(33, dtype=np.float32).view(np.uint8)),
               ("c.weight", (64, 3), dq.Q8_0, quantize(dq.Q8_0, w[:192]))]
    meta = {"general.architecture": "qwen2", "x.u": 7, "x.f": 1.5, "x.neg": -3, "x.b": True,
            "x.s": "héllo", "x.arr": [1, 2, 3], "x.strs": ["a", "bb", ""], "x.farr": [0.5, -1.0]}
    p = tmp_path / "t.gguf"
    gguf.write(p, meta, tensors)
    g = gguf.load(p)
    assert g.version == 3 and g.alignment == 32 and g.data_start % 32 == 0
    assert g.metadata == {**meta, "x.neg": -3}
    for (name, shape, t, raw), info in zip(tensors, g.tensors):
        assert (info.name, info.shape, info.ggml_type) == (name, shape, t)
        assert info.offset % 32 == 0
        assert bytes(gguf.read_tensor_bytes(g, info)) == bytes(memoryview(raw).cast("B"))
    # the oracle's independent reader sees the same file
    meta2, tens2 = ref_cpu.read_gguf(p)
    assert meta2["x.strs"] == ["a", "bb", ""] and tens2["a.weight"][1] == dq.Q4_K
    assert tens2["c.weight"][2] == bytes(tensors[2][3])


def test_gguf_rejects_bad_magic(tmp_path):
    from pico_hip import gguf
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"GGUX" + bytes(20))
    with pytest.raises(ValueError, match="GGUF signature"):
        gguf.load(p)


def test_synth_is_deterministic_and_uses_the_mix(tmp_path):
    from pico_hip import gguf, synth
    arch = synth.tiny_arch(n_layers=2)
    a = synth.build(tmp_path / "a.gguf", arch, seed=5)
    b = synth.build(tmp_path / "b.gguf", arch, seed=5)
    c = synth.build(tmp_path / "c.gguf", arch, seed=6)
    assert a == b != c
    g = gguf.load(tmp_path / "a.gguf")
    types = {t.name: t.ggml_type for t in g.tensors}
    assert types["blk.0.attn_v.weight"] == dq.Q8_0 and types["blk.1.attn_v.weight"] == dq.Q5_0
    assert types["blk.0.ffn_down.weight"] == dq.Q6_K and types["blk.1.ffn_down.weight"] == dq.Q4_K
    assert types["blk.0.attn_q.weight"] == dq.Q5_0 and types["output.weight"] == dq.Q8_0
    assert "tokenizer.ggml.eos_token_id" not in g.metadata
    emb = g.tensor("token_embd.weight")
    out = g.tensor("output.weight")
    assert bytes(gguf.read_tensor_bytes(g, emb)) == bytes(gguf.read_tensor_bytes(g, out))  # tied


def test_7b_mix():
    from pico_hip import synth
    a = synth.ARCHES["qwen2.5-7b"]
    assert synth.q4_k_m_mix(a, 0, "attn_q") == dq.Q4_K
    assert synth.q4_k_m_mix(a, 3, "attn_v") == dq.Q6_K
    assert synth.q4_k_m_mix(a, 3, "ffn_down") == dq.Q6_K
    assert synth.q4_k_m_mix(a, -1, "token_embd") == dq.Q8_0


def test_tokenizer_bpe_roundtrip_and_specials():
    from pico_hip.tokenizer import BPETokenizer, byte_symbols
    base = [byte_symbols()[b] for b in range(256)]
    vocab = base + ["he", "ll", "hell", "hello", "Ġw", "Ġwo", "<|im_start|>", "<|im_end|>"]
    merges = ["h e", "l l", "he ll", "hell o", "Ġ w", "Ġw o"]
    tok = BPETokenizer(vocab, merges, bos_id=-1, eos_id=vocab.index("<|im_end|>"))
    ids = tok.encode("<|im_start|>hello world<|im_end|>")
    assert ids[0] == vocab.index("<|im_start|>") and ids[-1] == vocab.index("<|im_end|>")
    assert ids[1] == vocab.index("hello") and ids[2] == vocab.index("Ġwo")
    assert tok.decode(ids[1:-1]) == "hello world"
    assert tok.decode(tok.encode("naïve €5\n")) == "naïve €5\n"
    assert tok.n_vocab == len(vocab)


def test_tokenizer_from_gguf_metadata():
    from pico_hip.tokenizer import from_gguf
    from pico_hip.synth import vocab_tokens
    tok = from_gguf({"tokenizer.ggml.model": "gpt2", "tokenizer.ggml.tokens": vocab_tokens(300)})
    assert tok.eos_id == -1 and tok.bos_id == -1
    assert tok.decode(tok.encode("abc xyz")) == "abc xyz"
    with pytest.raises(ValueError):
        from_gguf({"tokenizer.ggml.model": "llama"})


def test_sampler():
    from pico_hip.sampler import sample
    logits = torch.tensor([0.1, 3.0, 3.0, -1.0])
    assert sample(logits, temperature=0.0) == 1          # first maximum on ties
    g = torch.Generator().manual_seed(0)
    draws = {sample(logits, temperature=1.0, top_k=1, generator=g) for _ in range(40)}
    assert draws == {1, 2}            # ties with the k-th value survive (sampler.py:23-24)
    draws = {sample(torch.tensor([0.1, 3.0, 2.0]), 1.0, top_k=1, generator=g) for _ in range(20)}
    assert draws == {1}
    draws = {sample(torch.tensor([5.0, 4.9, -9.0]), 1.0, top_p=0.6, generator=g) for _ in range(50)}
    assert draws <= {0, 1}


def test_engine_requires_gpu_device(tiny_model):
    from pico_hip.engine import Engine
    with pytest.raises(ValueError, match="GPU only"):
        Engine(tiny_model, device="cpu")


@pytest.mark.parametrize("t", [dq.F32, dq.F16, dq.Q8_0, dq.Q5_0, dq.Q4_K, dq.Q6_K])
def test_torch_quantizer_bytes_equal_numpy(t):
    """quantize_torch (the GPU model builder's quantizer) gives quantize()'s bytes: random
    N(0, 0.02) blocks plus all-zero, single-spike, opposite-extreme and tiny-value blocks."""
    from pico_hip.quantize import quantize, quantize_torch
    rng = np.random.default_rng(100 + t)
    x = (rng.standard_normal(256 * 48) * 0.02).astype(np.float32)
    x[:256] = 0.0
    x[300], x[301] = 0.5, -0.5
    x[512:768] = 1e-7
    x[1024] = -3.0
    got = quantize_torch(t, torch.from_numpy(x)).numpy()
    np.testing.assert_array_equal(got, quantize(t, x))


def test_synthetic_7b_mix_and_device_build(tmp_path):
    """The 7B mix (Q4_K attention q/k/o and gate/up, Q6_K attn_v and ffn_down, Q8_0 embedding
    and an untied Q8_0 output) and a reproducible device build (here on the CPU device)."""
    from pico_hip import gguf, synth
    arch = synth.tiny_arch(n_layers=1, hidden=512, n_head=4, n_kv=2, head_dim=128, ffn=512, vocab=300,
                           name="qwen2.5-7b-tiny", tied=False)
    h1 = synth.build(tmp_path / "a.gguf", arch, seed=1, device="cpu")
    assert synth.build(tmp_path / "b.gguf", arch, seed=1, device="cpu") == h1
    g = gguf.load(tmp_path / "a.gguf")
    types = {t.name: t.ggml_type for t in g.tensors}
    assert types["blk.0.attn_q.weight"] == dq.Q4_K and types["blk.0.ffn_up.weight"] == dq.Q4_K
    assert types["blk.0.attn_v.weight"] == dq.Q6_K and types["blk.0.ffn_down.weight"] == dq.Q6_K
    assert types["token_embd.weight"] == dq.Q8_0 and types["output.weight"] == dq.Q8_0
    by = {t.name: t for t in g.tensors}
    assert bytes(gguf.read_tensor_bytes(g, by["output.weight"])) != \
        bytes(gguf.read_tensor_bytes(g, by["token_embd.weight"]))


def test_truncated_gguf_raises_before_upload(tmp_path):
    """A file that ends inside a tensor's data is rejected when the tensor's bytes are read
    (the reference's f.read(n_bytes) + reshape raises too), never handed on short."""
    from pico_hip import gguf
    from pico_hip.quantize import quantize
    w = np.random.default_rng(1).standard_normal(32 * 256).astype(np.float32)
    p = tmp_path / "t.gguf"
    gguf.write(p, {"general.architecture": "qwen2"},
               [("a.weight", (256, 32), dq.Q8_0, quantize(dq.Q8_0, w))])
    data = p.read_bytes()
    cut = tmp_path / "cut.gguf"
    cut.write_bytes(data[:-100])
    g = gguf.load(cut)
    with pytest.raises(ValueError, match="spans bytes"):
        gguf.read_tensor_bytes(g, g.tensors[0])
    assert len(gguf.read_tensor_bytes(gguf.load(p), g.tensors[0])) == g.tensors[0].n_bytes


def test_short_buffers_rejected_before_any_launch():
    """dequantize / embed_gather refuse a byte buffer smaller than the elements they would
    read (checked on the host, before the device is touched)."""
    from pico_hip import kernels as K
    from pico_hip.dequant import GGML_Q8_0
    with pytest.raises(ValueError, match="fewer than"):
        K.dequantize(GGML_Q8_0, torch.zeros(33, dtype=torch.uint8), 32)
    table = K.RawTensor(torch.zeros(34 * 9, dtype=torch.uint8), GGML_Q8_0, (10, 32))
    with pytest.raises(ValueError, match="embedding table"):
        K.embed_gather(table, torch.tensor([0]))


def test_generate_rejects_more_tokens_than_the_context():
    """Prompt + new tokens beyond context_len (the RoPE table's rows) raise before anything is
    allocated or launched."""
    from pico_hip.engine import Engine
    from pico_hip.model import ModelConfig
    eng = Engine.__new__(Engine)   # no device work: the check comes first
    eng.cfg = ModelConfig(vocab_size=10, n_layers=1, hidden=32, n_head=1, n_kv_head=1,
                          head_dim=32, ffn_dim=32, rope_base=1e4, eps=1e-6, context_len=16)
    with pytest.raises(ValueError, match="context length"):
        eng.generate_ids([1] * 10, max_tokens=7)


def _golden_tok_sampler():
    import json
    from conftest import GOLDEN
    return json.loads((GOLDEN / "tokenizer_sampler.json").read_text())


def test_tokenizer_reference_toy_vocab_known_ids():
    """The reference's toy vocabulary (its tests/test_tokenizer.py): encodings worked by hand,
    round trips and vocabulary size."""
    from pico_hip.tokenizer import BPETokenizer
    fx = _golden_tok_sampler()["tokenizer"]
    tok = BPETokenizer(fx["vocab"], fx["merges"], bos_id=fx["bos_id"], eos_id=fx["eos_id"])
    assert tok.n_vocab == fx["n_vocab"]
    for case in fx["cases"]:
        assert tok.encode(case["text"]) == case["ids"], case["text"]
        assert tok.decode(case["ids"]) == case["text"]


def test_sampler_known_answers():
    """top-k keeps ties with the k-th value, top-p keeps the token that crosses p (the shifted
    mask), temperature applies first, greedy takes the first maximum: each case may only
    return its allowed ids, and returns each of them over 400 seeded draws."""
    from pico_hip.sampler import sample
    for case in _golden_tok_sampler()["sampler"]:
        logits = torch.tensor(case["logits"], dtype=torch.float32)
        g = torch.Generator().manual_seed(0)
        seen = {sample(logits.clone(), case["temperature"], case["top_k"], case["top_p"], generator=g)
                for _ in range(400)}
        assert seen <= set(case["allowed"]), case["what"]
        if case["all_seen"]:
            assert seen == set(case["allowed"]), case["what"]


def test_step_workspace_cleared_after_a_failed_launch():
    """A pe_decode_step workspace whose error word is set is zeroed whole: the launch counter,
    the error word and exchange pairs that a late workgroup of the failed launch published under
    the next launch's tag (counter + 1), which the next launch would otherwise accept."""
    from pico_hip.model import clear_step_workspace_on_error
    ws = torch.zeros(4096, dtype=torch.uint8)
    words = ws.view(torch.int32)
    pairs = ws.view(torch.int64)
    words[0] = 41                               # launch counter after the failed launch
    pairs[40:48] = (42 << 32) | 0x3F800000      # stale pairs tagged 42 (counter + 1), value 1.0
    assert clear_step_workspace_on_error(ws) == 0 and int(words[0]) == 41   # no error: untouched
    words[16] = 1                               # a wait ran out
    assert clear_step_workspace_on_error(ws) == 1
    assert int(ws.count_nonzero()) == 0
    assert clear_step_workspace_on_error(None) == 0
