"""Dense Qwen2 forward over the pico_hip kernels (the reference's model.py call surface).

``ModelConfig`` and ``Transformer(cfg, weights, device, quant).forward(token_ids, positions,
cache) -> logits`` keep the reference's signatures (model.py:27-57, :60-62, :128-165).
With ``use_step_kernel`` set (off by default: about 2 % faster than the four-launch step at
config 0 in a same-box A/B, 2062 vs 2025 tok/s, but it needs every workgroup resident at once
and raises if a bounded wait runs out), a greedy decode step of a model the persistent kernel
covers (head_dim 64, hidden <= 1024, ffn <= 8192, caches up to 128 positions: the 0.5B
family) is one launch, pe_decode_step. Otherwise decode (one token) runs three launches per
layer plus the LM head (the 0.5B family):

  per layer:
    qkv_fix_rmsnorm_rope (x + 2^-32 sum of the previous   model.py:175-193, :234
                        layer's FFN replicas, norm, QKV +
                        bias, RoPE, cache write; the first
                        layer: qkv_embed_rmsnorm_rope, which   model.py:152
                        decodes the token's embedding row
                        (bit-exact) as x, stores it and
                        clears the step's fixed-point
                        accumulators)
    attn_oproj_fix     (GQA attention per query head,     model.py:211-213
                        fp16-rounded, times that head's
                        columns of Wo, added in 64-bit
                        fixed point into the accumulator)
    ffn_fix            (x + 2^-32 acc, norm, gate/up,     model.py:213-234
                        SiLU*up, ffn_down split over the
                        FFN dimension, added into four
                        fixed-point replicas; the last
                        layer: qgemv_fix_norm_silu and the
                        ffn_down qgemv with its residual)
  qgemv_norm(_argmax)  (final norm + LM head [+ greedy])  model.py:159-164

Without a down-slice copy of ffn_down (ffn_fix_ok) the FFN runs as qgemv_fix_norm_silu and the
ffn_down qgemv with its residual, after qkv_rmsnorm_rope (four launches per layer).
attn_oproj_fix covers head_dim 64, caches of <= 128 positions and a Q5_0 / Q8_0 Wo (the 0.5B
family); other formats at those sizes run attn_gproj (attention per kv group times the
group's columns of Wo, one fp32 part per group) and qgemv_sum_norm_silu (x + parts).
Caches of 513..4096 positions (head_dim 64) run attn_split_gproj instead of attn_gproj: the
split-KV attention, then one launch that merges each kv group's chunk records and multiplies
them by the group's Wo columns (the parts the gate/up GEMV adds). Other shapes (head_dim 128,
other cache sizes) run decode_attn (model.py:211) and the o-projection GEMV with the residual
(model.py:213), then the normed gate/up GEMV.

Prefill (L > 1) follows the reference's L > 1 branch op for op: in fp32 for short prompts (its
off-CUDA numerics): rmsnorm, one small-M GEMM per QKV segment with bias, RoPE, cache write at
[pos0, pos0 + L), causal attention, o-projection + residual, rmsnorm, gate/up GEMM, SiLU*up,
down + residual; on the matrix cores (fp16 operands, fp32 accumulation) from
``prefill_f16_min_tokens`` tokens on. Logits from the last row. Every op is a HIP kernel;
nothing runs on the CPU.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import kernels as K
from .kernels import QWeight, RawTensor


def clear_step_workspace_on_error(ws: torch.Tensor | None) -> int:
    """The error word of a pe_decode_step workspace (bytes 64..67; 0: none); a non-zero word
    zeroes the whole workspace (launch counter at bytes 0..3, error word, exchange pairs and
    pick records)."""
    if ws is None:
        return 0
    w = int(ws[64:68].view(torch.int32).item())
    if w:
        ws.zero_()
    return w


@dataclass
class ModelConfig:
    vocab_size: int
    n_layers: int
    hidden: int          # n_embd
    n_head: int          # query heads
    n_kv_head: int       # kv heads (GQA)
    head_dim: int
    ffn_dim: int
    rope_base: float
    eps: float           # RMSNorm epsilon
    context_len: int


@dataclass
class Layer:
    attn_norm: torch.Tensor
    attn_norm_ut: torch.Tensor   # unit-transposed copies for the decode kernels
    ffn_norm_ut: torch.Tensor
    wq: QWeight
    wk: QWeight
    wv: QWeight
    bq: torch.Tensor | None
    bk: torch.Tensor | None
    bv: torch.Tensor | None
    wo: QWeight
    ffn_norm: torch.Tensor
    w_gate_up: QWeight | None   # [gate; up] when both share a format, else None
    w_gate: QWeight | None      # the halves on their own (only when not fused)
    w_up: QWeight | None
    w_down: QWeight


class Transformer:
    def __init__(self, cfg: ModelConfig, weights: dict[str, torch.Tensor], device: torch.device,
                 quant: dict | None = None):
        if torch.device(device).type != "cuda":
            raise ValueError("pico_hip runs on the GPU only")
        self.cfg = cfg
        self.device = torch.device(device)
        self.w = weights                 # name -> fp32 device tensor (norms, biases)
        self.quant = quant or {}         # name -> QWeight / RawTensor
        self.embed: RawTensor = self.quant["token_embd"]
        self.output: QWeight = self.quant["output"]
        # RoPE tables exactly as the reference builds them (model.py:73-79), on the device.
        inv_freq = 1.0 / (cfg.rope_base ** (torch.arange(0, cfg.head_dim, 2, device=self.device)
                                            / cfg.head_dim))
        pos = torch.arange(cfg.context_len, device=self.device, dtype=torch.float32)
        angles = pos[:, None] * inv_freq[None, :]
        self.cos = angles.cos().contiguous()
        self.sin = angles.sin().contiguous()
        self.layers = [self._layer_weights(i) for i in range(cfg.n_layers)]
        self.output_norm_ut = K.to_ut(self.w["output_norm.weight"])
        self._ws: dict[int, torch.Tensor] = {}
        # attention of each query head fused with its share of the o-projection, added into a
        # fixed-point accumulator that the gate/up GEMV adds to x (attn_oproj_fix), where the
        # model and cache qualify (attn_oproj_supported: a Q5_0 / Q8_0 Wo, head_dim 64, caches
        # of <= 128 positions); else attn_gproj
        self.use_attn_oproj = True
        self._acc: torch.Tensor | None = None
        # with attn_oproj_fix: the FFN of every layer but the last in one launch (ffn_fix: gate/up,
        # SiLU and ffn_down split over the FFN dimension, added into fixed-point replicas that
        # the next layer's QKV launch reads), where every such layer qualifies (ffn_fix_ok)
        self.use_ffn_fix = True
        self._acc_block: torch.Tensor | None = None
        # with ffn_fix: the token's embedding row decoded by the first layer's QKV launch, which
        # also clears the step's fixed-point accumulators (qkv_embed_rmsnorm_rope), in place of
        # an embedding-gather launch and a fill
        self.use_embed_qkv = True
        self._x0: torch.Tensor | None = None
        # attention of each kv group fused with its share of the o-projection (attn_gproj),
        # the shares added by the gate/up GEMV: four launches per layer instead of five
        self.use_attn_gproj = True
        # caches of split_gproj_capacity[0] .. [1] positions run the split attention and a merge
        # fused with the o-projection shares (attn_split_gproj: two launches where decode_attn +
        # the o-projection GEMV take two or three). Measured end to end on the 0.5B model: +5.7 %
        # at a 1000-token prompt, +2.2 % at 3000, -4.7 % at 200 (the one-launch mid-size
        # attention wins there); slower beyond ~4096 positions, where every workgroup merging
        # all of its kv group's records costs more than the merge launch
        self.split_gproj_capacity = (513, 4096)
        # prompts of at least this many tokens are prefilled on the matrix cores (fp16
        # operands, fp32 accumulation: the reference's CUDA autocast prefill, model.py:147-151);
        # shorter ones by the fp32 path (the reference's off-CUDA numerics). None: never.
        self.prefill_f16_min_tokens: int | None = 512
        # prefills (L > 1) with the reference's GPU numerics instead: every product's operands
        # and result, the norms, RoPE, attention and SiLU outputs and the residual stream held in
        # fp16 where CUDA fp16 autocast holds them (model.py:147-151; _prefill_autocast)
        self.prefill_autocast = False
        # the matrix-core prefill's plain products (QKV + bias, o-proj and ffn_down + residual)
        # on hipBLASLt instead of this library's MFMA GEMM (pe_gemm_h16); its workspace and the
        # device's hipBLASLt handle are made on first use (outside any graph capture)
        self.prefill_blaslt = False
        self._lt_ws: torch.Tensor | None = None
        # prompts from position 0 at head_dim 64: K and V also written as fp16 key blocks for the
        # flash kernel's direct-to-LDS copies; off: the flash kernel that converts the fp32 caches
        self.prefill_kv_blocks = True
        # with the key blocks, prompts past 4096 tokens split the long query sets' key ranges
        # over workgroups and merge them (within fp32 rounding); off: one workgroup per query set
        self.prefill_flash_split = True
        self._f16: list[dict[str, torch.Tensor]] | None = None
        # greedy decode steps the persistent kernel covers can run as one launch per token
        # (pe_decode_step) instead of four launches per layer; off by default: ~2 % faster, but
        # it needs all of its workgroups resident at once (one per CU)
        self.use_step_kernel = False
        self._step_ws: torch.Tensor | None = None
        self._steps: dict[tuple[int, int], K.DecodeStep] = {}

    def _layer_weights(self, i: int) -> Layer:
        p, q, w = f"blk.{i}.", self.quant, self.w
        return Layer(
            attn_norm=w[p + "attn_norm.weight"],
            attn_norm_ut=K.to_ut(w[p + "attn_norm.weight"]),
            ffn_norm_ut=K.to_ut(w[p + "ffn_norm.weight"]),
            wq=q[p + "attn_q.weight"], wk=q[p + "attn_k.weight"], wv=q[p + "attn_v.weight"],
            bq=w.get(p + "attn_q.bias"), bk=w.get(p + "attn_k.bias"), bv=w.get(p + "attn_v.bias"),
            wo=q[p + "attn_output.weight"],
            ffn_norm=w[p + "ffn_norm.weight"],
            w_gate_up=q.get(p + "ffn_gate_up.weight"),
            w_gate=q.get(p + "ffn_gate.weight"), w_up=q.get(p + "ffn_up.weight"),
            w_down=q[p + "ffn_down.weight"],
        )

    def weight_bytes_per_token(self) -> int:
        """Bytes of weights one decode token reads: every layer's packed matrices, biases and
        norms, the final norm, the LM head and one embedding row (GGUF sizes)."""
        total = self.output.nbytes + self.w["output_norm.weight"].numel() * 4
        total += self.embed.data.numel() // self.embed.shape[0]
        for L in self.layers:
            mats = [L.wq, L.wk, L.wv, L.wo, L.w_down]
            mats += [L.w_gate_up] if L.w_gate_up is not None else [L.w_gate, L.w_up]
            total += sum(m.nbytes for m in mats)
            total += sum(t.numel() * 4 for t in (L.attn_norm, L.ffn_norm, L.bq, L.bk, L.bv) if t is not None)
        return total

    def attn_workspace(self, capacity: int) -> torch.Tensor:
        """Decode-attention workspace for a cache of ``capacity`` (shared by all layers)."""
        ws = self._ws.get(capacity)
        if ws is None:
            c = self.cfg
            ws = K.decode_attn_workspace(c.n_head, c.n_kv_head, c.head_dim, capacity, self.device)
            self._ws[capacity] = ws
        return ws

    @torch.inference_mode()
    def forward(self, token_ids: torch.Tensor, positions: torch.Tensor,
                cache: list[tuple[torch.Tensor, torch.Tensor]],
                greedy: K.GreedyState | None = None) -> torch.Tensor:
        """Run ``token_ids`` (L,) at ``positions`` (L,) updating ``cache``; logits (vocab,) of
        the last position. Decode (L == 1) reads the token and position from device memory
        only, so the step can be captured once and replayed as a graph. With ``greedy`` the
        LM head also makes the greedy pick on the device and advances ``greedy.state``
        (token_ids/positions may then be its ``token``/``pos`` views)."""
        if token_ids.shape[0] == 1:
            return self._decode(token_ids, positions, cache, greedy)
        if self.prefill_autocast:
            return self._prefill_autocast(token_ids, positions, cache, greedy)
        m = self.prefill_f16_min_tokens
        if m is not None and token_ids.shape[0] >= m:
            return self._prefill_f16(token_ids, positions, cache, greedy)
        return self._prefill(token_ids, positions, cache, greedy)

    def f16_weights(self) -> list[dict[str, torch.Tensor]]:
        """Per layer fp16 (N, K) copies of the linear weights for the matrix-core prefill: qkv
        ([q; k; v] rows, with the concatenated bias), o, gu_il ([gate; up] interleaved in
        groups of 16 rows for the SiLU-fused GEMM; gu, plain, when ffn % 16 != 0) and down;
        each value the exact dequantized weight rounded to nearest even. Built once, on first
        use."""
        if self._f16 is None:
            out = []
            for L in self.layers:
                qd, kd = L.wq.n, L.wk.n
                qkv = torch.empty(qd + 2 * kd, L.wq.k, device=self.device, dtype=torch.float16)
                K.dequantize_weight_f16(L.wq, qkv[:qd])
                K.dequantize_weight_f16(L.wk, qkv[qd:qd + kd])
                K.dequantize_weight_f16(L.wv, qkv[qd + kd:])
                if L.w_gate_up is not None:
                    gu = K.dequantize_weight_f16(L.w_gate_up)
                else:
                    f = L.w_gate.n
                    gu = torch.empty(2 * f, L.w_gate.k, device=self.device, dtype=torch.float16)
                    K.dequantize_weight_f16(L.w_gate, gu[:f])
                    K.dequantize_weight_f16(L.w_up, gu[f:])
                bias = None
                if L.bq is not None:
                    bias = torch.cat([L.bq, L.bk, L.bv]).float().contiguous()
                # [gate; up] interleaved in groups of 16 rows for the SiLU-fused GEMM
                gu_il = K.interleave_gate_up_f16(gu) if (gu.shape[0] // 2) % 16 == 0 else None
                out.append(dict(qkv=qkv, qkv_bias=bias, o=K.dequantize_weight_f16(L.wo),
                                gu=gu if gu_il is None else None, gu_il=gu_il,
                                down=K.dequantize_weight_f16(L.w_down)))
            self._f16 = out
        return self._f16

    def _lm_head(self, x, norm_w, greedy, layout):
        if greedy is None:
            return K.qgemv_norm(x, norm_w, self.output, self.cfg.eps, layout=layout)
        return K.qgemv_norm_argmax(x, norm_w, self.output, self.cfg.eps, greedy, layout=layout)

    # ---- decode ---------------------------------------------------------------------------
    def decode_step_for(self, cache) -> K.DecodeStep | None:
        """The one-launch decode step bound to ``cache`` (built on first use, outside any graph
        capture), or None when pe_decode_step does not cover this model or capacity."""
        capacity = cache[0][0].shape[1]
        key = (cache[0][0].data_ptr(), capacity)
        st = self._steps.get(key)
        if st is None:
            if not K.decode_step_supported(self, capacity):
                return None
            if self._step_ws is None:
                self._step_ws = K.decode_step_workspace(self, self.device)
            if len(self._steps) > 8:   # tables of caches no longer in use
                self._steps.clear()
            st = K.DecodeStep(self, cache, self._step_ws)
            self._steps[key] = st
        return st

    def step_error(self) -> int:
        """pe_decode_step's error word (0: none; 1: a wait ran out; 2: a token or position out
        of range). A non-zero word clears the whole workspace: the launch counter, the error
        word and every exchange pair. Workgroups of a failed launch that started after its
        counter was read may have published pairs under the next launch's tag, which the next
        launch would otherwise take as ready; after the clear every pair carries tag 0 and the
        next launch's tag is 1."""
        return clear_step_workspace_on_error(self._step_ws)

    def attn_oproj_ok(self, capacity: int) -> bool:
        """Whether decode with a cache of ``capacity`` positions runs attn_oproj_fix: every
        layer's Wo has its o-projection layout, the shapes and capacity are covered, and
        [gate; up] is one tensor."""
        if not self.use_attn_oproj:
            return False
        c = self.cfg
        return all(L.w_gate_up is not None and
                   K.attn_oproj_supported(c.n_head, c.n_kv_head, c.head_dim, capacity, L.wo)
                   for L in self.layers)

    def ffn_fix_ok(self, capacity: int) -> bool:
        """Whether decode with a cache of ``capacity`` positions runs the three-launch layers
        (qkv_fix_rmsnorm_rope, attn_oproj_fix, ffn_fix): attn_oproj_ok and every layer but the
        last has an FFN that ffn_fix covers."""
        return (self.use_ffn_fix and self.attn_oproj_ok(capacity) and
                all(K.ffn_fix_supported(L.w_gate_up, L.w_down) for L in self.layers[:-1]))

    def _decode(self, token_ids, positions, cache, greedy=None):
        """One token. With a greedy state and a model pe_decode_step covers, the whole step is
        one launch that reads the token and position from the state. Otherwise four launches
        per layer; the hidden and FFN vectors stay in the unit-transposed layout between
        kernels (each producer writes it, each GEMV reads it with coalesced loads)."""
        cfg = self.cfg
        if greedy is not None and self.use_step_kernel:
            st = self.decode_step_for(cache)
            if st is not None:
                if token_ids.data_ptr() != greedy.token.data_ptr():
                    greedy.token.copy_(token_ids.reshape(-1)[:1].to(torch.int64))
                if positions.data_ptr() != greedy.pos.data_ptr():
                    greedy.pos.copy_(positions.reshape(-1)[:1].to(torch.int64))
                return st.run(greedy)
        XU, YU = K.LAYOUT_X_UT, K.LAYOUT_Y_UT
        pos = positions.reshape(-1)[:1]
        if pos.dtype != torch.int64:
            pos = pos.to(torch.int64)
        capacity = cache[0][0].shape[1]
        if self.ffn_fix_ok(capacity):
            if self._acc_block is None:
                self._acc_block = K.fix_acc_block(cfg.hidden, self.device, cfg.n_layers)
            acc = self._acc_block
            embed_first = self.use_embed_qkv and token_ids.numel() == 1 and \
                self.embed.ggml_type in K.EMBED_QKV_TYPES
            if embed_first:
                if self._x0 is None:
                    self._x0 = torch.empty(cfg.hidden, device=self.device, dtype=torch.float32)
                x = self._x0
                tok = token_ids.reshape(-1)[:1]
                if tok.dtype != torch.int64:
                    tok = tok.to(torch.int64)
            else:
                x = K.embed_gather(self.embed, token_ids, layout=YU).reshape(-1)
                acc.zero_()   # a fill kernel (graph-capturable), once per token for every layer
            last = len(self.layers) - 1
            d_acc = None   # the previous layer's down-product replicas
            for i, L in enumerate(self.layers):
                k_buf, v_buf = cache[i]
                if i == 0 and embed_first:
                    # x = the token's embedding row (stored into x), the accumulators cleared
                    q = K.qkv_embed_rmsnorm_rope(self.embed, tok, L.attn_norm_ut, cfg.eps, L.wq, L.wk, L.wv,
                                                 L.bq, L.bk, L.bv, self.cos, self.sin, pos, k_buf, v_buf,
                                                 cfg.n_head, x_out=x, clear=acc, layout=XU)
                elif d_acc is None:
                    q = K.qkv_rmsnorm_rope(x, L.attn_norm_ut, cfg.eps, L.wq, L.wk, L.wv, L.bq, L.bk,
                                           L.bv, self.cos, self.sin, pos, k_buf, v_buf, cfg.n_head,
                                           layout=XU)
                else:
                    q, x = K.qkv_fix_rmsnorm_rope(x, d_acc, L.attn_norm_ut, cfg.eps, L.wq, L.wk, L.wv,
                                                  L.bq, L.bk, L.bv, self.cos, self.sin, pos, k_buf,
                                                  v_buf, cfg.n_head, layout=XU)
                K.attn_oproj_fix(q, k_buf, v_buf, L.wo, pos, acc[i, 0], layout=YU)
                if i < last:
                    d_acc = acc[i, 1:]
                    x = K.ffn_fix(x, acc[i, 0], L.ffn_norm_ut, L.w_gate_up, L.w_down, cfg.eps, d_acc,
                                  layout=XU | YU)
                else:
                    act, x = K.qgemv_fix_norm_silu(x, acc[i, 0], L.ffn_norm_ut, L.w_gate_up, cfg.eps,
                                                   layout=XU | YU)
                    x = K.qgemv(act, L.w_down, residual=x, layout=XU | YU)
            return self._lm_head(x, self.output_norm_ut, greedy, XU)
        x = K.embed_gather(self.embed, token_ids, layout=YU).reshape(-1)
        if self.attn_oproj_ok(capacity):
            if self._acc is None:
                self._acc = K.fix_acc(cfg.hidden, self.device, cfg.n_layers)
            acc = self._acc
            acc.zero_()   # a fill kernel (graph-capturable), once per token for every layer
            for i, L in enumerate(self.layers):
                k_buf, v_buf = cache[i]
                q = K.qkv_rmsnorm_rope(x, L.attn_norm_ut, cfg.eps, L.wq, L.wk, L.wv, L.bq, L.bk, L.bv,
                                       self.cos, self.sin, pos, k_buf, v_buf, cfg.n_head, layout=XU)
                K.attn_oproj_fix(q, k_buf, v_buf, L.wo, pos, acc[i], layout=YU)
                act, x = K.qgemv_fix_norm_silu(x, acc[i], L.ffn_norm_ut, L.w_gate_up, cfg.eps,
                                               layout=XU | YU)
                x = K.qgemv(act, L.w_down, residual=x, layout=XU | YU)
            return self._lm_head(x, self.output_norm_ut, greedy, XU)
        ws = self.attn_workspace(capacity)
        for i, L in enumerate(self.layers):
            k_buf, v_buf = cache[i]
            q = K.qkv_rmsnorm_rope(x, L.attn_norm_ut, cfg.eps, L.wq, L.wk, L.wv, L.bq, L.bk, L.bv,
                                   self.cos, self.sin, pos, k_buf, v_buf, cfg.n_head, layout=XU)
            parts = None
            if self.use_attn_gproj and L.w_gate_up is not None:
                if K.attn_gproj_supported(cfg.n_head, cfg.n_kv_head, cfg.head_dim, capacity, L.wo):
                    parts = K.attn_gproj(q, k_buf, v_buf, L.wo, S=pos, S_offset=1, layout=YU)
                elif (self.split_gproj_capacity[0] <= capacity <= self.split_gproj_capacity[1] and
                      K.attn_split_gproj_supported(cfg.n_head, cfg.n_kv_head, cfg.head_dim, capacity, L.wo)):
                    parts = K.attn_split_gproj(q, k_buf, v_buf, L.wo, S=pos, S_offset=1, workspace=ws,
                                               layout=YU)
            if parts is not None:
                act, x = K.qgemv_sum_norm_silu(x, parts, L.ffn_norm_ut, L.w_gate_up, cfg.eps,
                                               layout=XU | YU)
                x = K.qgemv(act, L.w_down, residual=x, layout=XU | YU)
                continue
            attn = K.decode_attn(q, k_buf, v_buf, S=pos, S_offset=1, workspace=ws, layout=YU)
            x = K.qgemv(attn.reshape(-1), L.wo, residual=x, layout=XU | YU)
            if L.w_gate_up is not None:
                act = K.qgemv_norm_silu(x, L.ffn_norm_ut, L.w_gate_up, cfg.eps, layout=XU | YU)
                x = K.qgemv(act, L.w_down, residual=x, layout=XU | YU)
            else:
                g = K.qgemv_norm(x, L.ffn_norm_ut, L.w_gate, cfg.eps, layout=XU)
                u = K.qgemv_norm(x, L.ffn_norm_ut, L.w_up, cfg.eps, layout=XU)
                act = K.silu_mul(torch.cat([g, u]).unsqueeze(0), cfg.ffn_dim).reshape(-1)
                x = K.qgemv(act, L.w_down, residual=x, layout=YU)
        return self._lm_head(x, self.output_norm_ut, greedy, XU)

    # ---- prefill --------------------------------------------------------------------------
    def _prefill_f16(self, token_ids, positions, cache, greedy=None):
        """The prefill on the matrix cores: GEMMs with fp16 operands and flash attention
        (pe_flash_prefill; head_dim 64, else the fp32 prefill attention), fp32 residual
        stream, norms, RoPE and KV cache. Every product reads operands stored in fp16 by their
        producers (pe_rmsnorm_h16, pe_flash_prefill_h16, the SiLU GEMM), the same values
        pe_gemm_f16 would round as it reads them: QKV + bias, o-proj and ffn_down + residual
        (added in place) on pe_gemm_h16 (its direct-to-LDS kernel for long prompts), gate/up
        with its SiLU epilogue on pe_gemm_h16_silu_h. prefill_blaslt = True runs the three
        plain products on hipBLASLt (pe_gemm_lt) instead."""
        cfg = self.cfg
        Lt = token_ids.shape[0]
        hd, nh, nkv = cfg.head_dim, cfg.n_head, cfg.n_kv_head
        qd, kd = nh * hd, nkv * hd
        cos = self.cos[positions]
        sin = self.sin[positions]
        pos0 = int(positions[0].item()) if positions.numel() else 0
        w16 = self.f16_weights()
        lt = self.prefill_blaslt
        if lt and self._lt_ws is None:
            self._lt_ws = K.gemm_lt_workspace(self.device)
        ws = self._lt_ws
        x = K.embed_gather(self.embed, token_ids)                       # (L, hidden)
        x_alt = torch.empty_like(x) if lt else None                    # the residual ping-pong
        qkv = torch.empty(Lt, qd + 2 * kd, device=self.device, dtype=torch.float32)
        q_rot = torch.empty(Lt, nh, hd, device=self.device, dtype=torch.float32)
        # a prompt from position 0 at head_dim 64: the RoPE pass also writes K and V as fp16 key
        # blocks that the flash kernel copies straight into LDS (the same values)
        kv16 = K.kv16_blocks(nkv, Lt, self.device) if self.prefill_kv_blocks and hd == 64 and pos0 == 0 else None
        # past 4096 tokens the long query sets' key ranges are split over workgroups and merged
        # (a second launch), in one workspace for every layer
        fws = None
        if kv16 is not None and self.prefill_flash_split:
            need = K.flash_prefill_blocks_workspace(nh, nkv, Lt)
            fws = torch.empty(need, device=self.device, dtype=torch.uint8) if need else None
        for i, L in enumerate(self.layers):
            k_buf, v_buf = cache[i]
            W = w16[i]
            # products on operands stored in fp16 by their producers
            h16 = K.rmsnorm(x, L.attn_norm, cfg.eps, half=True)
            if lt:
                K.gemm_lt(h16, W["qkv"], bias=W["qkv_bias"], out=qkv, workspace=ws)
            else:
                K.gemm_f16(h16, W["qkv"], bias=W["qkv_bias"], out=qkv)
            # RoPE of q and k and the cache write of k and v, one pass (model.py:186-197)
            qr = K.rope_kv_write(qkv, cos, sin, nh, k_buf, v_buf, pos0=pos0, out=q_rot, kv16=kv16)
            if kv16 is not None:  # matrix-core flash attention from the key blocks, fp16 output
                attn = K.flash_prefill_blocks(qr, kv16, workspace=fws, split=self.prefill_flash_split)
            elif hd == 64:  # the same from the fp32 caches
                attn = K.flash_prefill(qr, k_buf, v_buf, pos0=pos0, half=True)
            else:         # other head sizes: the fp32 causal attention kernel
                attn = K.prefill_attn(qr, k_buf, v_buf, pos0=pos0)
            if lt and attn.dtype == torch.float16:
                x, x_alt = K.gemm_lt(attn, W["o"], residual=x, out=x_alt, workspace=ws), x
            else:
                x = K.gemm_f16(attn, W["o"], residual=x, out=x)
                if lt and x_alt.shape != x.shape:
                    x_alt = torch.empty_like(x)
            if W["gu_il"] is not None:
                # the norm stored in fp16 (the values the GEMM rounds an fp32 A to), the SiLU
                # product in fp16: the down GEMM's operand
                h16 = K.rmsnorm(x, L.ffn_norm, cfg.eps, half=True)
                act = K.gemm_f16_silu(h16, W["gu_il"], half=True)
            else:
                h = K.rmsnorm(x, L.ffn_norm, cfg.eps)
                act = K.silu_mul(K.gemm_f16(h, W["gu"]), cfg.ffn_dim)
            if lt and act.dtype == torch.float16:
                x, x_alt = K.gemm_lt(act, W["down"], residual=x, out=x_alt, workspace=ws), x
            else:
                x = K.gemm_f16(act, W["down"], residual=x, out=x)
        return self._lm_head(x[-1], self.w["output_norm.weight"], greedy, K.LAYOUT_NATURAL)

    def _prefill_autocast(self, token_ids, positions, cache, greedy=None):
        """The prompt prefill as the reference computes it on CUDA, under fp16 autocast
        (model.py:147-151, :175-235): the products take fp16 operands (pe_gemm_f16 rounds A as
        it reads it; the weights and the QKV bias rounded once) with fp32 accumulation, and each
        result is rounded to fp16 (pe_round_f16); RoPE, the SiLU product and the norms compute
        in fp32 from fp16 values and their outputs are rounded (the Triton kernels store in
        their input's dtype, kernels.py:22, :46-47, :74); attention runs on the fp16 q, K, V
        with fp16 probabilities and an fp16 output (pe_flash_prefill_h16; head_dim 64, else the
        fp32 kernel rounded after); the residual stream is fp16 from the first o-projection on
        (addmm, model.py:213) and the KV cache holds fp16 values. The LM head multiplies the
        fp16-rounded normed last row (the Q8_0 GEMV reads it as fp32, kernels.py:180)."""
        cfg = self.cfg
        Lt = token_ids.shape[0]
        hd, nh, nkv = cfg.head_dim, cfg.n_head, cfg.n_kv_head
        qd, kd = nh * hd, nkv * hd
        cos = self.cos[positions]
        sin = self.sin[positions]
        pos0 = int(positions[0].item()) if positions.numel() else 0
        w16 = self.f16_weights()
        x = K.embed_gather(self.embed, token_ids)                       # (L, hidden), fp32
        qkv = torch.empty(Lt, qd + 2 * kd, device=self.device, dtype=torch.float32)
        q_rot = torch.empty(Lt, nh, hd, device=self.device, dtype=torch.float32)
        for i, L in enumerate(self.layers):
            k_buf, v_buf = cache[i]
            W = w16[i]
            bias = W["qkv_bias"]
            if bias is not None:
                bias = K.round_f16_(bias.clone())
            h = K.rmsnorm(x, L.attn_norm, cfg.eps)                     # rounded by the GEMM's read
            K.round_f16_(K.gemm_f16(h, W["qkv"], bias=bias, out=qkv))
            qr = K.rope_kv_write(qkv, cos, sin, nh, k_buf, v_buf, pos0=pos0, out=q_rot)
            K.round_f16_(qr.view(Lt, qd))
            K.round_f16_(k_buf.view(nkv, -1)[:, pos0 * hd:(pos0 + Lt) * hd])
            if hd == 64:
                attn = K.flash_prefill(qr, k_buf, v_buf, pos0=pos0, half=True)
            else:
                attn = K.round_f16_(K.prefill_attn(qr, k_buf, v_buf, pos0=pos0).view(Lt, qd))
            if i == 0:
                x = K.round_f16_(x.clone())                             # addmm casts x to fp16
            x = K.round_f16_(K.gemm_f16(attn, W["o"], residual=x))
            h = K.round_f16_(K.rmsnorm(x, L.ffn_norm, cfg.eps))
            if W["gu"] is not None:
                gu = K.gemm_f16(h, W["gu"])
            else:  # [gate; up] interleaved in groups of 16 rows: the product's columns put back
                g4 = K.gemm_f16(h, W["gu_il"]).view(Lt, -1, 2, 16)
                gu = torch.cat([g4[:, :, 0].reshape(Lt, -1), g4[:, :, 1].reshape(Lt, -1)], dim=1)
            K.round_f16_(gu)
            act = K.round_f16_(K.silu_mul(gu, cfg.ffn_dim))
            x = K.round_f16_(K.gemm_f16(act, W["down"], residual=x))
        h = K.round_f16_(K.rmsnorm(x[-1:], self.w["output_norm.weight"], cfg.eps))
        logits = K.qgemv(h[0], self.output)
        if greedy is not None:
            # the pick of this prefill made on the host (once per prompt): the device pick of
            # the LM-head launch normalises its input itself, which would skip the fp16
            # rounding of the normed row; torch.argmax's rule (sampler.py:27)
            pos, c = (int(v) for v in greedy.state[1:3].tolist())
            pick = int(torch.argmax(logits).item())
            greedy.state.copy_(torch.tensor([pick, pos + 1, c + 1], dtype=torch.int64))
            if 0 <= c < greedy.log_cap:
                greedy.log[c] = pick
        return logits

    def _prefill(self, token_ids, positions, cache, greedy=None):
        cfg = self.cfg
        Lt = token_ids.shape[0]
        hd, nh, nkv = cfg.head_dim, cfg.n_head, cfg.n_kv_head
        qd, kd = nh * hd, nkv * hd
        cos = self.cos[positions]
        sin = self.sin[positions]
        # the cache rows of this chunk start at its first position (the reference always
        # prefills from 0, model.py:188-197: the same rows for a whole prompt)
        pos0 = int(positions[0].item()) if positions.numel() else 0
        x = K.embed_gather(self.embed, token_ids)                       # (L, hidden)
        qkv = torch.empty(Lt, qd + 2 * kd, device=self.device, dtype=torch.float32)
        for i, L in enumerate(self.layers):
            k_buf, v_buf = cache[i]
            h = K.rmsnorm(x, L.attn_norm, cfg.eps)
            K.qgemm(h, L.wq, bias=L.bq, out=qkv[:, :qd])
            K.qgemm(h, L.wk, bias=L.bk, out=qkv[:, qd:qd + kd])
            K.qgemm(h, L.wv, bias=L.bv, out=qkv[:, qd + kd:])
            qk = qkv[:, :qd + kd].view(Lt, nh + nkv, hd)
            qk = K.rope(qk, cos, sin)                                     # (L, nh+nkv, hd)
            v = qkv[:, qd + kd:].view(Lt, nkv, hd)
            K.kv_write(qk[:, nh:], v, k_buf, v_buf, pos0=pos0)
            attn = K.prefill_attn(qk[:, :nh], k_buf, v_buf, pos0=pos0)  # (L, hidden)
            x = K.qgemm(attn, L.wo, residual=x)
            h = K.rmsnorm(x, L.ffn_norm, cfg.eps)
            if L.w_gate_up is not None:
                gu = K.qgemm(h, L.w_gate_up)
            else:
                gu = torch.cat([K.qgemm(h, L.w_gate), K.qgemm(h, L.w_up)], dim=1)
            act = K.silu_mul(gu, cfg.ffn_dim)
            x = K.qgemm(act, L.w_down, residual=x)
        return self._lm_head(x[-1], self.w["output_norm.weight"], greedy, K.LAYOUT_NATURAL)
