"""torch-CPU restatement of the reference's dense Qwen2 forward (test infrastructure only).

Used as (a) the end-to-end oracle for logits and greedy tokens and (b) the reported CPU
baseline of bench.py. The reference itself cannot execute its dense path off an NVIDIA GPU
(every dense forward calls Triton kernels), so this module restates it op for op with the
reference's own CPU formulations:

* GGUF parsing                    gguf.py:79-115 (own reader below, independent of pico_hip)
* config from metadata            engine.py:26-63
* RoPE tables                     model.py:73-79
* RMSNorm                         model.py:292-295 (``_rmsnorm_cpu``)
* RoPE                            model.py:297-300 (``_rope_cpu``), applied to q and k heads
* QKV, o-projection               model.py:177, :213 (F.linear / addmm on fp32 dequantized W)
* cache write                     model.py:188-197
* decode attention                model.py:342-344 einsum softmax over valid positions, GQA
                                  head h -> kv h // group (kernels.py:99), output rounded to
                                  fp16 (kernels.py:126)
* prefill attention               model.py:201-209 (causal SDPA, fp32 off-CUDA, model.py:150)
* gate/up, down, LM head at L=1   the int8 + scale GEMV forms (model.py:266-284 ``_gemv``,
                                  kernels.py:174, :205-207, :244-249, :282, :320-322) over the
                                  reference's unpacked tensors (dequant.py:79-168)
* gate/up, down at L>1            fp32 matmul on dequantized W (model.py:223, :235)
* LM head                         q8_0 form on the last row (model.py:160-164)
* greedy                          argmax (sampler.py:26-27)
* ``autocast=True``               the prefill under CUDA fp16 autocast (model.py:147-151):
                                  fp16 roundings where the reference's GPU path rounds

Pinned by tests/test_oracle_model.py: against float64 closed forms (tests/../oracle/closed.py)
op by op, and the whole forward against an independent float64 numpy forward on a small model.
"""

from __future__ import annotations

import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

from . import dequant as dq


# ---- minimal GGUF reader (gguf.py:79-115) -------------------------------------------------

def _rd_str(f):
    (n,) = struct.unpack("<Q", f.read(8))
    return f.read(n).decode("utf-8", errors="replace")


_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q",
        11: "<q", 12: "<d"}


def _rd_val(f, vt):
    if vt in _FMT:
        return struct.unpack(_FMT[vt], f.read(struct.calcsize(_FMT[vt])))[0]
    if vt == 8:
        return _rd_str(f)
    if vt == 9:
        et, n = struct.unpack("<IQ", f.read(12))
        return [_rd_val(f, et) for _ in range(n)]
    raise ValueError(vt)


def read_gguf(path):
    """-> (metadata, {name: (ne-shape, type, raw bytes)})."""
    with open(path, "rb") as f:
        magic, version, nt, nkv = struct.unpack("<IIQQ", f.read(24))
        assert magic == 0x46554747, "not a GGUF file"
        meta = {}
        for _ in range(nkv):
            k = _rd_str(f)
            (vt,) = struct.unpack("<I", f.read(4))
            meta[k] = _rd_val(f, vt)
        align = int(meta.get("general.alignment", 32))
        infos = []
        for _ in range(nt):
            name = _rd_str(f)
            (nd,) = struct.unpack("<I", f.read(4))
            shape = struct.unpack(f"<{nd}Q", f.read(8 * nd))
            gt, off = struct.unpack("<IQ", f.read(12))
            infos.append((name, tuple(shape), gt, off))
        start = f.tell()
        start += (align - start % align) % align
        tensors = {}
        for name, shape, gt, off in infos:
            n = int(np.prod(shape))
            f.seek(start + off)
            tensors[name] = (shape, gt, f.read(dq.nbytes_for(gt, n)))
    return meta, tensors


@dataclass
class RefConfig:
    vocab: int
    n_layers: int
    hidden: int
    n_head: int
    n_kv: int
    head_dim: int
    ffn: int
    rope_base: float
    eps: float
    context_len: int


def _unpacked(gt: int, raw: bytes, n_out: int, k: int):
    """The reference's kernel form of a quantized (n_out, k) tensor: (tag, q, s1, s2)."""
    if gt == dq.Q8_0:
        q, d = dq.unpack_q8_0(raw, n_out * k)
        return ("q8", torch.from_numpy(q.reshape(n_out, k)), torch.from_numpy(d.reshape(n_out, k // 32)), None)
    if gt == dq.Q5_0:
        q, d = dq.unpack_q5_0(raw, n_out * k)
        return ("q5", torch.from_numpy(q.reshape(n_out, k)), torch.from_numpy(d.reshape(n_out, k // 32)), None)
    if gt == dq.Q6_K:
        q, dsc = dq.unpack_q6_k(raw, n_out * k)
        return ("q6", torch.from_numpy(q.reshape(n_out, k)), torch.from_numpy(dsc.reshape(n_out, k // 16)), None)
    if gt == dq.Q4_K:
        q, sc, mn = dq.unpack_q4_k(raw, n_out * k)
        return ("q4", torch.from_numpy(q.reshape(n_out, k)), torch.from_numpy(sc.reshape(n_out, k // 32)),
                torch.from_numpy(mn.reshape(n_out, k // 32)))
    raise NotImplementedError(gt)


def gemv_cpu(entry, x, bias=None, residual=None):
    """The reference's CPU quantized GEMV (model.py:266-284)."""
    tag, q, s1, s2 = entry
    x = x.float()
    N, K = q.shape
    block = 16 if tag == "q6" else 32
    nb = K // block
    q3 = q.float().reshape(N, nb, block)
    x3 = x.reshape(nb, block)
    dot = (q3 * x3).sum(-1)
    xs = x3.sum(-1)
    if tag == "q4":
        acc = (s1 * dot - s2 * xs).sum(-1)
    elif tag == "q5":
        acc = (s1 * (dot - 16.0 * xs)).sum(-1)
    else:
        acc = (s1 * dot).sum(-1)
    if bias is not None:
        acc = acc + bias
    if residual is not None:
        acc = acc + residual
    return acc


def f16(t):
    """Round to fp16 (nearest even) and back to fp32: the value an fp16 tensor holds."""
    return t.half().float()


def flash16_causal(q, k, v, group):
    """Causal GQA attention the way an fp16 flash-attention kernel computes it (SDPA under
    CUDA autocast, model.py:201-209): fp16 q, K, V; scores and softmax statistics in fp32; the
    probabilities rounded to fp16 for the P.V product (fp32 accumulation); the output divided
    by the fp32 sum and rounded to fp16. q (L, nh, hd), k / v (nkv, L, hd) -> (L, nh * hd)."""
    L, nh, hd = q.shape
    kr = k.repeat_interleave(group, dim=0)                          # (nh, L, hd)
    vr = v.repeat_interleave(group, dim=0)
    s = torch.einsum("lhd,hsd->hls", q, kr) * (hd ** -0.5)          # (nh, L, L)
    s = s.masked_fill(torch.ones(L, L, dtype=torch.bool).triu(1), float("-inf"))
    p = torch.exp(s - s.amax(-1, keepdim=True))
    o = torch.einsum("hls,hsd->hld", f16(p), vr) / p.sum(-1, keepdim=True)
    return f16(o).transpose(0, 1).reshape(L, nh * hd)


def rmsnorm_cpu(x, w, eps):
    """model.py:292-295."""
    var = (x * x).mean(-1, keepdim=True)
    return x * torch.rsqrt(var + eps) * w


def rope_cpu(x, cos, sin):
    """model.py:297-300 (rotate-half)."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1)


class RefModel:
    """The reference's dense forward on the CPU, from a GGUF file."""

    def __init__(self, path: str | Path, unpack_quant: bool = True, dequantize=None,
                 device: str | torch.device = "cpu"):
        """``dequantize(ggml_type, raw_bytes, n) -> fp32 tensor`` and ``device`` replace the
        numpy dequantizer and the CPU for models whose fp32 weights are too large for a quick
        CPU run (7B): the same forward then runs on torch's own ops on ``device``, over
        weights dequantized by the caller (use unpack_quant=False there: every matrix is then
        multiplied as fp32 dequantized weights, which the integer GEMV forms equal up to
        rounding)."""
        meta, tensors = read_gguf(path)
        self.device = torch.device(device)
        arch = meta["general.architecture"]
        n_kv = int(meta[f"{arch}.attention.head_count_kv"])
        self.cfg = c = RefConfig(
            vocab=len(meta["tokenizer.ggml.tokens"]),
            n_layers=int(meta[f"{arch}.block_count"]),
            hidden=int(meta[f"{arch}.embedding_length"]),
            n_head=int(meta[f"{arch}.attention.head_count"]),
            n_kv=n_kv,
            head_dim=tensors["blk.0.attn_k.weight"][0][1] // n_kv,
            ffn=int(meta[f"{arch}.feed_forward_length"]),
            rope_base=float(meta[f"{arch}.rope.freq_base"]),
            eps=float(meta[f"{arch}.attention.layer_norm_rms_epsilon"]),
            context_len=int(meta[f"{arch}.context_length"]),
        )
        self.meta = meta
        self.w = {}
        for name, (shape, gt, raw) in tensors.items():
            n = int(np.prod(shape))
            dense = (torch.from_numpy(dq.dequantize(gt, raw, n)) if dequantize is None
                     else dequantize(gt, raw, n))
            self.w[name] = dense.reshape(tuple(reversed(shape))).to(self.device)
        self.types = {name: gt for name, (shape, gt, raw) in tensors.items()}
        self.raw = tensors
        inv_freq = 1.0 / (c.rope_base ** (torch.arange(0, c.head_dim, 2) / c.head_dim))
        pos = torch.arange(c.context_len, dtype=torch.float32)
        ang = pos[:, None] * inv_freq[None, :]
        self.cos, self.sin = ang.cos().to(self.device), ang.sin().to(self.device)
        self.qkv_w, self.qkv_b, self.gu_w = [], [], []
        for i in range(c.n_layers):
            p = f"blk.{i}."
            self.qkv_w.append(torch.cat([self.w[p + "attn_q.weight"], self.w[p + "attn_k.weight"],
                                         self.w[p + "attn_v.weight"]], 0))
            self.qkv_b.append(torch.cat([self.w[p + "attn_q.bias"], self.w[p + "attn_k.bias"],
                                         self.w[p + "attn_v.bias"]]))
            self.gu_w.append(torch.cat([self.w[p + "ffn_gate.weight"], self.w[p + "ffn_up.weight"]], 0))
        # The reference's quantized-kernel slots (engine.py:198-267): the LM head only when
        # output.weight is Q8_0 (:216-223), gate/up only when every layer's pair is Q5_0
        # (:225-242), ffn_down per layer when Q6_K or Q4_K (:244-266); every other matrix is
        # multiplied as fp32 dequantized weights (model.py:163-164, :177, :213, :223, :235).
        self.q = {}
        if unpack_quant:
            if all(self.types[f"blk.{i}.ffn_{h}.weight"] == dq.Q5_0
                   for i in range(c.n_layers) for h in ("gate", "up")):
                for i in range(c.n_layers):
                    p = f"blk.{i}."
                    g = self._unpack(p + "ffn_gate.weight")
                    u = self._unpack(p + "ffn_up.weight")
                    self.q[p + "gu"] = (g[0], torch.cat([g[1], u[1]]), torch.cat([g[2], u[2]]), None)
            for i in range(c.n_layers):
                p = f"blk.{i}."
                if self.types[p + "ffn_down.weight"] in (dq.Q6_K, dq.Q4_K):
                    self.q[p + "down"] = self._unpack(p + "ffn_down.weight")
            if self.types.get("output.weight") == dq.Q8_0:
                self.q["output"] = self._unpack("output.weight")

    def _unpack(self, name):
        shape, gt, raw = self.raw[name]
        return _unpacked(gt, raw, shape[1], shape[0])

    def empty_cache(self, capacity: int):
        c = self.cfg
        z = lambda: torch.zeros(c.n_kv, capacity, c.head_dim, device=self.device)
        return [(z(), z()) for _ in range(c.n_layers)]

    @torch.inference_mode()
    def forward(self, ids: torch.Tensor, positions: torch.Tensor, cache,
                autocast: bool = False, return_hidden: bool = False):
        """``autocast`` restates the reference's prefill on CUDA (L > 1 runs under fp16
        autocast, model.py:147-151): F.linear, addmm and matmul take fp16 operands (fp32 weights,
        activations and biases rounded to fp16) and return fp16 (fp32 accumulation, one rounding
        of the result); SDPA runs on fp16 q, K, V (flash16_causal); the Triton RMSNorm, RoPE and
        SiLU kernels compute in fp32 and store in their input's dtype (kernels.py:22, :46-47,
        :74), so from the first o-projection on the residual stream is fp16 and the KV cache
        holds fp16 values; the Q8_0 LM head reads its input as fp32 (kernels.py:180). Decode
        (L == 1) is unaffected. ``return_hidden``: (logits, the normed last row the LM head
        multiplies)."""
        c = self.cfg
        L = ids.shape[0]
        ac = autocast and L > 1
        x = self.w["token_embd.weight"][ids]
        cos, sin = self.cos[positions], self.sin[positions]
        for i in range(c.n_layers):
            x = self._layer(i, x, positions, cos, sin, cache[i], ac)
        h = rmsnorm_cpu(x, self.w["output_norm.weight"], c.eps)
        if ac:
            h = f16(h)
        if "output" in self.q:
            logits = gemv_cpu(self.q["output"], h[-1])
        else:
            # model.py:163-164; a file without output.weight ties the head to token_embd (the
            # reference requires the tensor; this is the usual GGUF convention for tied models)
            w = self.w.get("output.weight", self.w["token_embd.weight"])
            logits = f16(h[-1] @ f16(w).T) if ac else h[-1] @ w.T
        return (logits, h[-1]) if return_hidden else logits

    def _layer(self, i, x, positions, cos, sin, cache, ac=False):
        c = self.cfg
        p = f"blk.{i}."
        L = x.shape[0]
        hd, nh, nkv = c.head_dim, c.n_head, c.n_kv
        k_buf, v_buf = cache
        h = rmsnorm_cpu(x, self.w[p + "attn_norm.weight"], c.eps)
        if ac:
            qkv = f16(F.linear(f16(h), f16(self.qkv_w[i]), f16(self.qkv_b[i])))
        else:
            qkv = F.linear(h, self.qkv_w[i], self.qkv_b[i])
        q = qkv[:, :nh * hd].view(L, nh, hd)
        k = qkv[:, nh * hd:(nh + nkv) * hd].view(L, nkv, hd)
        v = qkv[:, (nh + nkv) * hd:].view(L, nkv, hd)
        q = rope_cpu(q, cos[:, None, :], sin[:, None, :])
        k = rope_cpu(k, cos[:, None, :], sin[:, None, :])
        if ac:
            q, k = f16(q), f16(k)
        group = nh // nkv
        if ac:
            k_buf[:, :L] = k.transpose(0, 1)
            v_buf[:, :L] = v.transpose(0, 1)
            out = flash16_causal(q, k_buf[:, :L], v_buf[:, :L], group)
            x = f16(torch.addmm(f16(x), out, f16(self.w[p + "attn_output.weight"]).T))
            hn = f16(rmsnorm_cpu(x, self.w[p + "ffn_norm.weight"], c.eps))
            gate_up = f16(hn @ f16(self.gu_w[i]).T)
            g, u = gate_up[:, :c.ffn], gate_up[:, c.ffn:]
            act = f16(g * torch.sigmoid(g) * u)
            return f16(torch.addmm(x, act, f16(self.w[p + "ffn_down.weight"]).T))
        if L == 1:
            pos = int(positions[0])
            k_buf[:, pos] = k[0]
            v_buf[:, pos] = v[0]
            S = pos + 1
            kr = k_buf[:, :S].repeat_interleave(group, dim=0)        # (nh, S, hd)
            vr = v_buf[:, :S].repeat_interleave(group, dim=0)
            scores = torch.einsum("hd,hsd->hs", q[0], kr) * (hd ** -0.5)
            scores = torch.softmax(scores, dim=-1)
            out = torch.einsum("hs,hsd->hd", scores, vr)
            out = out.half().float().reshape(1, nh * hd)               # kernels.py:126
        else:
            k_buf[:, :L] = k.transpose(0, 1)
            v_buf[:, :L] = v.transpose(0, 1)
            out = F.scaled_dot_product_attention(
                q.transpose(0, 1).unsqueeze(0),
                k_buf[:, :L].unsqueeze(0).repeat_interleave(group, dim=1),
                v_buf[:, :L].unsqueeze(0).repeat_interleave(group, dim=1),
                is_causal=True).squeeze(0).transpose(0, 1).reshape(L, nh * hd)
        x = torch.addmm(x, out, self.w[p + "attn_output.weight"].T)
        if L == 1 and (p + "gu") in self.q:
            hn = rmsnorm_cpu(x[0], self.w[p + "ffn_norm.weight"], c.eps)
            gate_up = gemv_cpu(self.q[p + "gu"], hn).unsqueeze(0)
        else:
            hn = rmsnorm_cpu(x, self.w[p + "ffn_norm.weight"], c.eps)
            gate_up = hn @ self.gu_w[i].T
        g, u = gate_up[:, :c.ffn], gate_up[:, c.ffn:]
        act = g * torch.sigmoid(g) * u
        if L == 1 and (p + "down") in self.q:
            return gemv_cpu(self.q[p + "down"], act[0], residual=x[0]).unsqueeze(0)
        return torch.addmm(x, act, self.w[p + "ffn_down.weight"].T)

    def greedy(self, prompt_ids: list[int], n_tokens: int, return_logits: bool = False):
        """Prefill then greedy-decode ``n_tokens``; returns ids (and per-step top-2 margins)."""
        cache = self.empty_cache(len(prompt_ids) + n_tokens)
        logits = self.forward(torch.tensor(prompt_ids), torch.arange(len(prompt_ids)), cache)
        out, margins, all_logits = [], [], []
        for step in range(n_tokens):
            top2 = torch.topk(logits, 2).values
            margins.append(float(top2[0] - top2[1]))
            if return_logits:
                all_logits.append(logits.clone())
            nxt = int(torch.argmax(logits))
            out.append(nxt)
            pos = len(prompt_ids) + step
            if step + 1 < n_tokens:
                logits = self.forward(torch.tensor([nxt]), torch.tensor([pos]), cache)
        if return_logits:
            return out, margins, all_logits
        return out, margins
