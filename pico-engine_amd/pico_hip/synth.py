"""Seeded synthetic Qwen2-architecture GGUF models (random init, no checkpoint needed).

Shapes and quantization mixes follow the benchmark configurations:
  qwen2.5-0.5b: 24 layers, hidden 896, 14/2 heads, hd 64, ffn 4864, vocab 151936, theta 1e6,
                eps 1e-6, QKV bias; Q5_0 attn_q/k/o + ffn_gate/up, attn_v Q8_0 (even layers) /
                Q5_0 (odd), ffn_down Q6_K (even) / Q4_K (odd), token_embd Q8_0, and an explicit
                output.weight holding the same Q8_0 bytes (tied embeddings; the reference needs
                the tensor to exist, model.py:160-164).
  qwen2.5-7b:   28 layers, hidden 3584, 28/4 heads, hd 128, ffn 18944, vocab 152064; Q4_K
                attn_q/k/o + ffn_gate/up, Q6_K attn_v + ffn_down, Q8_0 token_embd and a separate
                (untied, as in Qwen2.5-7B) Q8_0 output.weight; built on the GPU (build(device=)).
Every tensor (norms and biases included) is N(0, 0.02) in fp32 before quantization, drawn
from numpy's PCG64 with the given seed in a fixed order, so a file is reproducible byte for
byte. The metadata holds the keys the engine reads (engine.py:26-63) and a gpt2 vocabulary of
distinct tokens (the 256 byte symbols first), with no eos id so greedy runs never stop early.
"""

from __future__ import annotations

import hashlib
import os
from dataclasses import dataclass, replace
from pathlib import Path

import numpy as np

from . import gguf
from .dequant import GGML_F32, GGML_Q4_K, GGML_Q5_0, GGML_Q6_K, GGML_Q8_0
from .quantize import quantize, quantize_torch


@dataclass(frozen=True)
class Arch:
    name: str
    n_layers: int
    hidden: int
    n_head: int
    n_kv: int
    head_dim: int
    ffn: int
    vocab: int
    rope_base: float = 1e6
    eps: float = 1e-6
    context_len: int = 32768
    tied: bool = True   # output.weight holds token_embd's bytes (else drawn on its own)


ARCHES = {
    "qwen2.5-0.5b": Arch("qwen2.5-0.5b", 24, 896, 14, 2, 64, 4864, 151936),
    "qwen2.5-7b": Arch("qwen2.5-7b", 28, 3584, 28, 4, 128, 18944, 152064, tied=False),
}


def tiny_arch(n_layers=2, hidden=256, n_head=4, n_kv=2, head_dim=64, ffn=512, vocab=1024,
              name="tiny", tied=True) -> Arch:
    """A small model of the same family for fast tests (K-quants need ffn % 256 == 0). A name
    starting with "qwen2.5-7b" selects the 7B quantization mix (then hidden % 256 == 0 too)."""
    return Arch(name, n_layers, hidden, n_head, n_kv, head_dim, ffn, vocab, context_len=4096, tied=tied)


def q4_k_m_mix(arch: Arch, layer: int, tensor: str) -> int:
    """ggml type of a weight tensor under the benchmark's Q4_K_M-style mix."""
    if arch.name.startswith("qwen2.5-7b"):
        if tensor in ("attn_v", "ffn_down"):
            return GGML_Q6_K
        if tensor in ("token_embd", "output"):
            return GGML_Q8_0
        return GGML_Q4_K
    # 0.5B mix (and tiny): 896-input tensors cannot be K-quants (K % 256 != 0)
    if tensor in ("token_embd", "output"):
        return GGML_Q8_0
    if tensor == "attn_v":
        return GGML_Q8_0 if layer % 2 == 0 else GGML_Q5_0
    if tensor == "ffn_down":
        kq_ok = arch.ffn % 256 == 0
        if not kq_ok:
            return GGML_Q8_0
        return GGML_Q6_K if layer % 2 == 0 else GGML_Q4_K
    return GGML_Q5_0


def vocab_tokens(n: int) -> list[str]:
    base = [chr(c) for c in _byte_symbols()]
    return base + [f"<t{i}>" for i in range(n - len(base))]


def _byte_symbols() -> list[int]:
    keep = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    out, extra = [], 0
    for b in range(256):
        if b in keep:
            out.append(b)
        else:
            out.append(256 + extra)
            extra += 1
    return out


def _host_source(seed: int):
    """numpy PCG64 draws, quantized on the host: the reference models (byte-reproducible
    everywhere, sha256-pinned in the test fixtures)."""
    rng = np.random.default_rng(seed)

    def weight(n_out: int, n_in: int) -> np.ndarray:
        return (rng.standard_normal(n_out * n_in, dtype=np.float32) * np.float32(0.02))

    return weight, quantize


# Draws per call of the device generator: fixed, so a tensor's values do not depend on how
# the caller chunks its work.
_DEVICE_CHUNK = 1 << 26


def _device_source(seed: int, device):
    """torch Philox draws on ``device``, quantized there (quantize_torch, the same rules as the
    host quantizer) and copied to host memory: for the large models (7B: 7.6e9 weights). The
    stream differs from numpy's, so these files differ from host-built ones of the same seed,
    but are reproducible for a given seed on the same torch/ROCm build."""
    import torch
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)

    def weight(n_out: int, n_in: int):
        n = n_out * n_in
        parts = [torch.randn(min(_DEVICE_CHUNK, n - o), generator=gen, device=device,
                             dtype=torch.float32) for o in range(0, n, _DEVICE_CHUNK)]
        return (torch.cat(parts) if len(parts) > 1 else parts[0]) * 0.02

    def quant(t: int, w) -> np.ndarray:
        step = _DEVICE_CHUNK  # a multiple of every block size (32, 256)
        chunks = [quantize_torch(t, w[o:o + step]) for o in range(0, w.numel(), step)]
        out = torch.cat(chunks).cpu().numpy() if len(chunks) > 1 else chunks[0].cpu().numpy()
        return out

    return weight, quant


def build(path: str | Path, arch: Arch, seed: int = 0, mix=q4_k_m_mix, device=None,
          progress=None) -> str:
    """Write the synthetic model to ``path``; returns its sha256. With ``device`` (a torch
    device) the weights are drawn and quantized on that device instead of by numpy.
    ``progress(msg)``, if given, is called after each layer and at the end."""
    weight, quantize = _host_source(seed) if device is None else _device_source(seed, device)
    H, hd = arch.hidden, arch.head_dim

    tensors = []
    emb_type = mix(arch, -1, "token_embd")
    emb = quantize(emb_type, weight(arch.vocab, H))
    tensors.append(("token_embd.weight", (H, arch.vocab), emb_type, emb))
    for i in range(arch.n_layers):
        p = f"blk.{i}."
        tensors.append((p + "attn_norm.weight", (H,), GGML_F32, quantize(GGML_F32, weight(1, H))))
        for nm, n_out in (("attn_q", arch.n_head * hd), ("attn_k", arch.n_kv * hd),
                          ("attn_v", arch.n_kv * hd)):
            t = mix(arch, i, nm)
            tensors.append((p + nm + ".weight", (H, n_out), t, quantize(t, weight(n_out, H))))
            tensors.append((p + nm + ".bias", (n_out,), GGML_F32, quantize(GGML_F32, weight(1, n_out))))
        t = mix(arch, i, "attn_output")
        tensors.append((p + "attn_output.weight", (arch.n_head * hd, H), t,
                        quantize(t, weight(H, arch.n_head * hd))))
        tensors.append((p + "ffn_norm.weight", (H,), GGML_F32, quantize(GGML_F32, weight(1, H))))
        for nm in ("ffn_gate", "ffn_up"):
            t = mix(arch, i, nm)
            tensors.append((p + nm + ".weight", (H, arch.ffn), t, quantize(t, weight(arch.ffn, H))))
        t = mix(arch, i, "ffn_down")
        tensors.append((p + "ffn_down.weight", (arch.ffn, H), t, quantize(t, weight(H, arch.ffn))))
        if progress:
            progress(f"synthetic {arch.name}: layer {i + 1}/{arch.n_layers} quantized")
    tensors.append(("output_norm.weight", (H,), GGML_F32, quantize(GGML_F32, weight(1, H))))
    out_type = mix(arch, -1, "output")
    out = emb if (arch.tied and out_type == emb_type) else quantize(out_type, weight(arch.vocab, H))
    tensors.append(("output.weight", (H, arch.vocab), out_type, out))

    meta = {
        "general.architecture": "qwen2",
        "general.name": f"synthetic-{arch.name}-seed{seed}",
        "qwen2.block_count": arch.n_layers,
        "qwen2.context_length": arch.context_len,
        "qwen2.embedding_length": H,
        "qwen2.feed_forward_length": arch.ffn,
        "qwen2.attention.head_count": arch.n_head,
        "qwen2.attention.head_count_kv": arch.n_kv,
        "qwen2.rope.freq_base": float(arch.rope_base),
        "qwen2.attention.layer_norm_rms_epsilon": float(arch.eps),
        "tokenizer.ggml.model": "gpt2",
        "tokenizer.ggml.tokens": vocab_tokens(arch.vocab),
    }
    tmp = str(path) + ".tmp"
    gguf.write(tmp, meta, tensors)
    os.replace(tmp, path)
    if progress:
        progress(f"synthetic {arch.name}: written to {path}")
    return sha256(path)


def sha256(path: str | Path) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 24), b""):
            h.update(chunk)
    return h.hexdigest()


def cached(arch: Arch, seed: int = 0, cache_dir: str | Path | None = None, device=None,
           progress=None) -> Path:
    """Path of the synthetic model, building it on first use (under $PICO_HIP_CACHE or /tmp);
    ``device`` as in build() (device-built files carry a "-dev" tag)."""
    cache_dir = Path(cache_dir or os.environ.get("PICO_HIP_CACHE", "/tmp/pico_hip_models"))
    cache_dir.mkdir(parents=True, exist_ok=True)
    tag = f"{arch.name}-L{arch.n_layers}-H{arch.hidden}-F{arch.ffn}-V{arch.vocab}-s{seed}"
    path = cache_dir / f"{tag}{'-dev' if device is not None else ''}.gguf"
    if not path.exists():
        build(path, arch, seed, device=device, progress=progress)
    return path


__all__ = ["Arch", "ARCHES", "tiny_arch", "q4_k_m_mix", "build", "cached", "sha256", "replace"]
