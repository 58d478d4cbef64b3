"""GGUF inference engine over the pico_hip kernels (the reference's engine.py surface).

``Engine(gguf_path, device="cuda")`` loads a dense Qwen2-style GGUF, ``generate(prompt, ...)``
runs prefill + a graph-replayed decode loop. Kept from the reference (engine.py): config from
metadata (:26-63), ``_empty_cache`` (:100-121, per layer fp32 (n_kv, capacity, hd) K/V),
``_build_decode_graph`` (:269-294: side-stream warmups, capture, eager fallback on failure),
``_decode_step`` (:296-306) and ``generate`` (:308-337).

Loading differs on purpose: instead of dequantizing every tensor to fp32 on the host and
unpacking the quantized ones to int8 + fp32 scales (engine.py:80-98, :198-267), the GGUF bytes
go to the device as they are; matrices (quantized, F16 or F32) are tiled there by
``pe_repack`` (a byte permutation, same size; F16/F32 rows stay as stored), F32 norms/biases
are used as they are, and the token embedding stays raw for the row gather. The fused
[gate; up] weight is the two tensors' blocks back to back (uploaded once, not as two tensors).
"""

from __future__ import annotations

import warnings
from pathlib import Path

import numpy as np
import torch

from . import kernels as K
from .dequant import GGML_F16, GGML_F32, MATRIX_TYPES
from .gguf import load as load_gguf, read_tensor_bytes
from .model import ModelConfig, Transformer
from .sampler import sample as sample_token
from .tokenizer import from_gguf as tokenizer_from_gguf


class Engine:
    def __init__(self, gguf_path: str | Path, device: str = "cuda", n_gpu_layers: int = 0):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("pico_hip runs on the GPU only (device must be cuda/HIP)")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.gguf = load_gguf(gguf_path)
        self.cfg = self._build_config()
        self.weights, self.quant = self._load_weights()
        self.model = Transformer(self.cfg, self.weights, self.device, self.quant)
        self.tok = tokenizer_from_gguf(self.gguf.metadata)
        self._graph = None

    def _build_config(self) -> ModelConfig:
        m = self.gguf.metadata
        arch = m["general.architecture"]
        if f"{arch}.expert_count" in m or arch == "mamba":
            raise NotImplementedError(f"{arch}: only dense decoder models are supported")
        n_kv = int(m[f"{arch}.attention.head_count_kv"])
        head_dim = None
        for t in self.gguf.tensors:
            if t.name == "blk.0.attn_k.weight":
                head_dim = t.shape[1] // n_kv
                break
        if head_dim is None:
            raise ValueError("could not derive head_dim (no blk.0.attn_k.weight)")
        return ModelConfig(
            vocab_size=len(m["tokenizer.ggml.tokens"]),
            n_layers=int(m[f"{arch}.block_count"]),
            hidden=int(m[f"{arch}.embedding_length"]),
            n_head=int(m[f"{arch}.attention.head_count"]),
            n_kv_head=n_kv,
            head_dim=head_dim,
            ffn_dim=int(m[f"{arch}.feed_forward_length"]),
            rope_base=float(m[f"{arch}.rope.freq_base"]),
            eps=float(m[f"{arch}.attention.layer_norm_rms_epsilon"]),
            context_len=int(m[f"{arch}.context_length"]),
        )

    def _upload(self, raw: np.ndarray) -> torch.Tensor:
        return torch.from_numpy(np.array(raw, dtype=np.uint8, copy=True)).to(self.device)

    def _load_weights(self):
        """Device tensors of the GGUF (engine.py:80-98): every 2-D matrix tiled for the kernels
        (quantized, F16 or F32 alike), the token embedding kept raw for the row gather, and
        1-D norms and biases as fp32. [gate; up] of a layer whose two halves share a format
        and shape are uploaded once, as one tensor, instead of as two."""
        weights: dict[str, torch.Tensor] = {}
        quant: dict[str, object] = {}
        g = self.gguf
        by_name = {t.name: t for t in g.tensors}
        fused = set()
        for i in range(self.cfg.n_layers):
            gt = by_name.get(f"blk.{i}.ffn_gate.weight")
            ut = by_name.get(f"blk.{i}.ffn_up.weight")
            if gt is not None and ut is not None and gt.ggml_type == ut.ggml_type \
                    and gt.shape == ut.shape and gt.ggml_type in MATRIX_TYPES:
                n, k = gt.shape[1], gt.shape[0]
                both = np.concatenate([read_tensor_bytes(g, gt), read_tensor_bytes(g, ut)])
                quant[f"blk.{i}.ffn_gate_up.weight"] = K.pack_weight(self._upload(both),
                                                                     gt.ggml_type, 2 * n, k)
                fused.update((gt.name, ut.name))
        for t in g.tensors:
            if t.name in fused:
                continue
            raw = read_tensor_bytes(g, t)
            shape = tuple(reversed(t.shape))     # logical (rows, cols), as engine.py:92-94
            if t.name == "token_embd.weight":
                quant["token_embd"] = K.RawTensor(self._upload(raw), t.ggml_type, shape)
                continue
            if len(shape) == 2 and t.ggml_type in MATRIX_TYPES:
                # the LM head keeps the tiled copy only: the greedy launch and the normed plain
                # GEMV both read it (the same lane groups, hence the same logits), so an MFMA
                # layout copy (447 MB for a Q6_K 7B head) would never be read
                mfma = False if t.name == "output.weight" else None
                # Wo also in the o-projection layout of the per-head attention + o-projection
                # launch (Q5_0 / Q8_0: the 0.5B family; 0.55 MB a layer at config 0)
                oproj = t.name.endswith(".attn_output.weight")
                # ffn_down also in the down-slice layout of the fused FFN launch (hidden <=
                # 2048: the 0.5B family; 3.3-4.4 MB a layer at config 0)
                slices = t.name.endswith(".ffn_down.weight")
                # q, k and v also in the RoPE-pair MFMA layout of the QKV launch on the integer
                # matrix cores (Q4_K / Q6_K with hidden % 256 == 0: the 7B family)
                pairs_hd = self.cfg.head_dim if t.name.endswith((".attn_q.weight", ".attn_k.weight",
                                                                  ".attn_v.weight")) else 0
                quant[t.name] = K.pack_weight(self._upload(raw), t.ggml_type, shape[0], shape[1],
                                              mfma=mfma, oproj=oproj, slices=slices, pairs_hd=pairs_hd)
                continue
            if len(shape) == 1 and t.ggml_type in (GGML_F32, GGML_F16):
                weights[t.name] = K.dequantize(t.ggml_type, self._upload(raw), t.n_elements)
                continue
            raise NotImplementedError(f"{t.name}: ggml type {t.ggml_type} shape {shape}")
        if "output.weight" in by_name:
            quant["output"] = quant["output.weight"]
        else:  # no output tensor: tied embeddings (the file's token_embd bytes as the LM head)
            e = quant["token_embd"]
            quant["output"] = K.pack_weight(e.data, e.ggml_type, e.shape[0], e.shape[1], mfma=False)
        torch.cuda.synchronize(self.device)
        return weights, quant

    def _empty_cache(self, capacity: int) -> list[tuple[torch.Tensor, torch.Tensor]]:
        c = self.cfg
        empty = lambda: torch.zeros(c.n_kv_head, capacity, c.head_dim, device=self.device)
        cache = [(empty(), empty()) for _ in range(c.n_layers)]
        self.model.attn_workspace(capacity)
        return cache

    # Replays issued between two host reads of the greedy log: the host checks for the stop
    # token once per chunk instead of synchronising on every token.
    greedy_chunk = 16

    @torch.inference_mode()
    def _build_decode_graph(self, cache):
        """Capture the single-token decode forward into a HIP graph (engine.py:269-294).
        The step reads its token and position from ``self._greedy.state`` and ends with the
        device-side greedy pick, which writes the next token and position back there, so
        greedy decoding replays the graph back to back. Returns the graph, or None (eager
        fallback) if capture fails."""
        capacity = cache[0][0].shape[1]
        self._greedy = K.GreedyState(self.model.output.n, capacity, self.device)
        self._static_ids = self._greedy.token
        self._static_pos = self._greedy.pos
        try:
            s = torch.cuda.Stream(self.device)
            s.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(s):
                for _ in range(3):
                    self.model.forward(self._static_ids, self._static_pos, cache, self._greedy)
            torch.cuda.current_stream(self.device).wait_stream(s)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._static_logits = self.model.forward(self._static_ids, self._static_pos,
                                                         cache, self._greedy)
            self._graph = g
            return g
        except Exception as e:  # noqa: BLE001 -- any capture failure falls back to eager
            self._graph = None
            warnings.warn(f"decode step not captured ({e}); each token runs its launches eagerly")
            return None

    @torch.inference_mode()
    def _decode_step(self, token: int, pos: int, cache, graph):
        if graph is not None:
            self._static_ids.fill_(int(token))
            self._static_pos.fill_(int(pos))
            graph.replay()
            return self._static_logits
        return self.model.forward(
            torch.tensor([token], device=self.device),
            torch.tensor([pos], device=self.device),
            cache,
        )

    @torch.inference_mode()
    def prefill_greedy(self, ids: list[int], cache) -> torch.Tensor:
        """Prefill ``ids`` and make the first greedy pick on the device (it lands in the
        greedy state as the next input, at position len(ids)). Needs _build_decode_graph
        first (it owns the greedy state). Returns the prefill logits."""
        self._greedy.reset(0, len(ids) - 1, 0)
        tokens = torch.tensor(ids, device=self.device)
        positions = torch.arange(len(ids), device=self.device)
        return self.model.forward(tokens, positions, cache, self._greedy)

    @torch.inference_mode()
    def decode_greedy(self, graph, max_tokens: int, eos: int | None) -> list[int]:
        """Greedy tokens after prefill_greedy: the same ids as the host loop
        ``nxt = argmax(logits); stop at eos; decode(nxt)`` (evidence.py:117-123) and one
        decode step per returned token, with the picks made on the device. The graph is
        replayed in chunks; the log is read once per chunk and cut at the first eos. A stop
        inside a chunk leaves some extra replays, whose cache rows lie inside the capacity
        this generation allocated and are never read."""
        done = 0
        while True:
            n = min(self.greedy_chunk, max_tokens - done)
            for _ in range(n):
                graph.replay()
            done += n
            picks = self._greedy.log[:done + 1].tolist()
            err = self.model.step_error()
            if err:
                raise RuntimeError(f"pe_decode_step failed (error word {err}): "
                                   + ("a wait ran out: the launch's workgroups were not all "
                                      "resident" if err == 1 else "token or position out of range"))
            if eos is not None and eos in picks:
                return picks[:picks.index(eos)][:max_tokens]
            if done >= max_tokens:
                return picks[:max_tokens]

    @torch.inference_mode()
    def generate_ids(self, ids: list[int], max_tokens: int = 64, temperature: float = 0.0,
                     top_k: int = 0, top_p: float = 1.0, use_graph: bool = True,
                     eos_id: int | None = None) -> list[int]:
        """Prefill ``ids`` then decode up to ``max_tokens`` tokens; returns the new ids.
        Greedy decoding with a graph picks tokens on the device; sampling and the eager path
        pick on the host (sampler.py)."""
        if not ids:
            return []
        if len(ids) + max_tokens > self.cfg.context_len:
            raise ValueError(f"{len(ids)} prompt + {max_tokens} new tokens exceed the model's "
                             f"context length {self.cfg.context_len} (the RoPE table's rows)")
        eos = self.tok.eos_id if eos_id is None else eos_id
        cache = self._empty_cache(len(ids) + max_tokens)
        graph = self._build_decode_graph(cache) if use_graph else None
        if graph is not None and temperature <= 0:
            self.prefill_greedy(ids, cache)
            return self.decode_greedy(graph, max_tokens, eos)
        tokens = torch.tensor(ids, device=self.device)
        positions = torch.arange(len(ids), device=self.device)
        logits = self.model.forward(tokens, positions, cache)
        generated: list[int] = []
        for _ in range(max_tokens):
            nxt = sample_token(logits, temperature, top_k, top_p)
            if nxt == eos:
                break
            pos = len(ids) + len(generated)
            generated.append(nxt)
            logits = self._decode_step(nxt, pos, cache, graph)
        return generated

    @torch.inference_mode()
    def generate(self, prompt: str, max_tokens: int = 64, temperature: float = 0.7,
                 top_k: int = 0, top_p: float = 0.9,
                 use_graph: bool = True) -> tuple[str, list[int]]:
        ids = self.tok.encode(prompt)
        if not ids:
            return "", []
        generated = self.generate_ids(ids, max_tokens, temperature, top_k, top_p, use_graph)
        return self.tok.decode(generated), generated
