"""HIP kernels of the decode path, with the reference's kernels.py names.

Every function launches a hand-written gfx950 kernel from libpico_hip.so through its C ABI on
torch's current stream (so it is captured by ``torch.cuda.graph``); inputs must already be on
the GPU -- there is no CPU fallback. Outputs are freshly allocated unless ``out=`` is given.

Reference names kept (src/pico_engine/kernels.py): ``rmsnorm`` (:26), ``rope`` (:50),
``silu_mul`` (:77), ``decode_attn`` (:129), ``q8_0_gemv`` (:178), ``q5_0_gemv`` (:211),
``q5_0_gemv_norm`` (:253), ``q6_k_gemv`` (:286), ``q4_k_gemv`` (:326). One signature change:
the quantized GEMVs take a ``QWeight`` (the GGUF blocks of the tensor, tiled on the device)
instead of the reference's unpacked (int8 values, fp32 scales) tensors. New fused entry points
used by model.py: ``qkv_rmsnorm_rope``, ``qgemv_norm_silu``, ``qgemv_norm``, plus the prefill
kernels ``qgemm``, ``kv_write``, ``prefill_attn`` and the load-time ``dequantize``,
``pack_weight``, ``embed_gather``.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import os

import torch

from ._lib import (LAYOUT_NATURAL, LAYOUT_X_UT, LAYOUT_Y_UT, AttnOprojArgs, FfnFixArgs, QkvArgs, StepArgs,
                   StepLayer, check, lib)
from .dequant import (BLOCK_SIZE, GGML_F16, GGML_F32, GGML_Q4_K, GGML_Q5_0, GGML_Q6_K, GGML_Q8_0, MATRIX_TYPES,
                      QUANT_TYPES, TYPE_NAMES, nbytes_for)

_VP = ctypes.c_void_p


def _ptr(t: torch.Tensor | None):
    return None if t is None else _VP(t.data_ptr())


def _stream(dev: torch.device):
    return _VP(torch.cuda.current_stream(dev).cuda_stream)


def _on_gpu(*ts: torch.Tensor | None) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(f"pico_hip kernels need GPU tensors, got a tensor on {t.device}")
        dev = t.device
    return dev


def _f32c(t: torch.Tensor) -> torch.Tensor:
    """fp32, contiguous (16-byte aligned start as a fresh allocation guarantees)."""
    t = t.float().contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def to_ut(v: torch.Tensor) -> torch.Tensor:
    """Natural -> unit-transposed layout of a 1-D vector (len % 32 == 0): element k moves to
    ((k % 32) // 4 * U + k // 32) * 4 + k % 4, U = len / 32 (see include/pico_hip.h)."""
    n = v.numel()
    return v.reshape(n // 32, 8, 4).transpose(0, 1).contiguous().reshape(n)


def from_ut(v: torch.Tensor) -> torch.Tensor:
    """Unit-transposed -> natural layout of a 1-D vector."""
    n = v.numel()
    return v.reshape(8, n // 32, 4).transpose(0, 1).contiguous().reshape(n)


@dataclass
class QWeight:
    """An (n x k) weight matrix in the tiled layout (see include/pico_hip.h): a quantized
    tensor's planes, or F16/F32 rows as stored."""

    data: torch.Tensor  # uint8 on the device, nbytes_for(ggml_type, n*k) bytes
    ggml_type: int
    n: int
    k: int
    # the same matrix in the MFMA layout (pe_repack_mfma) when the decode GEMVs run it on the
    # integer matrix cores (large Q4_K / Q6_K matrices, see mfma_eligible)
    mfma: torch.Tensor | None = None
    # the same matrix in the o-projection layout (pe_repack_oproj: Q5_0 / Q8_0 Wo) for the
    # per-head attention + o-projection launch (attn_oproj_fix)
    oproj: torch.Tensor | None = None
    # the same matrix in the down-slice layout (pe_repack_down_slices: ffn_down of hidden <=
    # 2048) for the fused FFN launch (ffn_fix)
    slices: torch.Tensor | None = None
    # the same matrix in the MFMA layout with its rows in RoPE-pair order
    # (pe_repack_mfma_pairs: Q4_K / Q6_K attn_q / attn_k / attn_v) for the QKV launch on the
    # integer matrix cores (mqkv)
    pairs: torch.Tensor | None = None

    @property
    def shape(self) -> tuple[int, int]:
        return (self.n, self.k)

    @property
    def nbytes(self) -> int:
        return self.data.numel()

    def copy(self) -> "QWeight":
        """A distinct device copy (every layout it holds)."""
        return QWeight(self.data.clone(), self.ggml_type, self.n, self.k,
                       None if self.mfma is None else self.mfma.clone(),
                       None if self.oproj is None else self.oproj.clone(),
                       None if self.slices is None else self.slices.clone(),
                       None if self.pairs is None else self.pairs.clone())

    def __repr__(self) -> str:
        return f"QWeight({TYPE_NAMES[self.ggml_type]}, n={self.n}, k={self.k})"


@dataclass
class RawTensor:
    """Raw GGUF bytes of a tensor kept untiled on the device (the embedding table)."""

    data: torch.Tensor
    ggml_type: int
    shape: tuple[int, ...]  # logical (rows, cols)


# ---- load-time ---------------------------------------------------------------------------

def dequantize(ggml_type: int, blocks: torch.Tensor, n: int, out: torch.Tensor | None = None):
    """Bit-exact fp32 dequantization of raw GGUF blocks (reference dequant.py:243-260)."""
    need = nbytes_for(ggml_type, n)
    if blocks.numel() * blocks.element_size() < need:
        raise ValueError(f"{blocks.numel() * blocks.element_size()} bytes hold fewer than {n} "
                         f"{TYPE_NAMES.get(ggml_type, ggml_type)} elements ({need} bytes)")
    dev = _on_gpu(blocks)
    if out is None:
        out = torch.empty(n, device=dev, dtype=torch.float32)
    if out.numel() < n:
        raise ValueError(f"output holds {out.numel()} of {n} elements")
    check(lib.pe_dequant(ggml_type, _ptr(blocks), _ptr(out), n, _stream(dev)), "pe_dequant")
    return out


# Decode GEMVs of Q4_K / Q6_K matrices of at least this many weights (k % 256 == 0) run on the
# integer matrix cores (pe_mgemv) from a second copy in the MFMA layout: the 7B model's
# gate/up and ffn_down, whose per-lane dot products bound the tiled GEMV on the vector ALU.
# Smaller matrices (the 7B o-projection, 12.8M weights: one item per wave, latency-bound)
# keep the tiled GEMVs only (measured: 6.3 vs 5.7 us).
MFMA_MIN_WEIGHTS = 1 << 25
# off (or PICO_MFMA_GEMV=0 in the environment): every decode GEMV on the tiled kernels
use_mfma_gemv = os.environ.get("PICO_MFMA_GEMV", "1") != "0"


def mfma_eligible(ggml_type: int, n: int, k: int) -> bool:
    return ggml_type in (GGML_Q4_K, GGML_Q6_K) and k % 256 == 0 and n * k >= MFMA_MIN_WEIGHTS


def repack_mfma(blocks: torch.Tensor, ggml_type: int, n: int, k: int) -> torch.Tensor:
    """Raw GGUF blocks of an (n x k) Q4_K / Q6_K matrix -> its MFMA layout (device uint8)."""
    dev = _on_gpu(blocks)
    size = lib.pe_mfma_bytes(ggml_type, n, k)
    if size < 0:
        raise ValueError(f"no MFMA layout for a {n}x{k} {TYPE_NAMES.get(ggml_type, ggml_type)} matrix")
    if blocks.numel() != nbytes_for(ggml_type, n * k):
        raise ValueError(f"{blocks.numel()} bytes for a {n}x{k} {TYPE_NAMES[ggml_type]} tensor")
    out = torch.empty(size, device=dev, dtype=torch.uint8)
    check(lib.pe_repack_mfma(ggml_type, _ptr(blocks), _ptr(out), n, k, _stream(dev)), "pe_repack_mfma")
    return out


# QKV of Q4_K / Q6_K matrices on the integer matrix cores (pe_mqkv_rmsnorm_rope) when every
# segment has its RoPE-pair MFMA layout (the 7B family: 10.0 -> 5.x us); off (or PICO_MQKV=0 in
# the environment): the tiled QKV launch
use_mqkv = os.environ.get("PICO_MQKV", "1") != "0"
# the activation planes of pe_mqkv_rmsnorm_rope stay in 64 KiB of LDS
MQKV_MAX_HIDDEN = 13568


def mqkv_eligible(ggml_type: int, n: int, k: int, head_dim: int) -> bool:
    """Whether an (n x k) attn_q / attn_k / attn_v matrix of heads of head_dim rows has a
    RoPE-pair MFMA layout for pe_mqkv_rmsnorm_rope."""
    return (ggml_type in (GGML_Q4_K, GGML_Q6_K) and k % 256 == 0 and k <= MQKV_MAX_HIDDEN
            and head_dim > 0 and head_dim % 16 == 0 and n % head_dim == 0)


def repack_mfma_pairs(blocks: torch.Tensor, ggml_type: int, n: int, k: int, head_dim: int) -> torch.Tensor:
    """Raw GGUF blocks of an (n x k) Q4_K / Q6_K matrix of heads of head_dim rows -> its MFMA
    layout with the rows in RoPE-pair order (every 16-row group holds 8 rotation pairs)."""
    dev = _on_gpu(blocks)
    size = lib.pe_mfma_bytes(ggml_type, n, k)
    if size < 0 or not mqkv_eligible(ggml_type, n, k, head_dim):
        raise ValueError(f"no RoPE-pair MFMA layout for a {n}x{k} {TYPE_NAMES.get(ggml_type, ggml_type)} matrix")
    if blocks.numel() != nbytes_for(ggml_type, n * k):
        raise ValueError(f"{blocks.numel()} bytes for a {n}x{k} {TYPE_NAMES[ggml_type]} tensor")
    out = torch.empty(size, device=dev, dtype=torch.uint8)
    check(lib.pe_repack_mfma_pairs(ggml_type, _ptr(blocks), _ptr(out), n, k, head_dim, _stream(dev)),
          "pe_repack_mfma_pairs")
    return out


def oproj_eligible(ggml_type: int, n: int, k: int) -> bool:
    """Whether an (n x k) matrix has an o-projection layout (pe_repack_oproj: Q5_0 / Q8_0,
    k % 64 == 0)."""
    return ggml_type in (GGML_Q5_0, GGML_Q8_0) and k % 64 == 0 and n > 0


def down_slice_eligible(ggml_type: int, n: int, k: int) -> bool:
    """Whether an (n x k) ffn_down matrix has a down-slice layout for ffn_fix (Q4_K / Q6_K /
    Q5_0 / Q8_0, n <= 2048: the 0.5B family)."""
    return n <= 2048 and n % 32 == 0 and lib.pe_down_slice_bytes(ggml_type, n, k) > 0


def repack_down_slices(blocks: torch.Tensor, ggml_type: int, n: int, k: int) -> torch.Tensor:
    """Raw GGUF blocks of an (n x k) matrix -> its down-slice layout (device uint8): per
    32-column slice, every row's 32 codes and exact fp32 scales, contiguous over the rows."""
    dev = _on_gpu(blocks)
    size = lib.pe_down_slice_bytes(ggml_type, n, k)
    if size < 0:
        raise ValueError(f"no down-slice layout for a {n}x{k} {TYPE_NAMES.get(ggml_type, ggml_type)} matrix")
    if blocks.numel() != nbytes_for(ggml_type, n * k):
        raise ValueError(f"{blocks.numel()} bytes for a {n}x{k} {TYPE_NAMES[ggml_type]} tensor")
    out = torch.empty(size, device=dev, dtype=torch.uint8)
    check(lib.pe_repack_down_slices(ggml_type, _ptr(blocks), _ptr(out), n, k, _stream(dev)),
          "pe_repack_down_slices")
    return out


def pack_weight(blocks: torch.Tensor, ggml_type: int, n: int, k: int, mfma: bool | None = None,
                oproj: bool = False, slices: bool = False, pairs_hd: int = 0) -> QWeight:
    """Raw GGUF blocks of an (n x k) tensor (device uint8) -> tiled QWeight, with the MFMA
    layout copy as well when ``mfma`` (default: when mfma_eligible), the o-projection layout
    copy when ``oproj`` and the matrix has one (oproj_eligible), the down-slice layout copy
    when ``slices`` and the matrix has one (down_slice_eligible), and the RoPE-pair MFMA layout
    for heads of ``pairs_hd`` rows when that is non-zero and the matrix has one
    (mqkv_eligible)."""
    dev = _on_gpu(blocks)
    if ggml_type not in MATRIX_TYPES:
        raise ValueError(f"no GEMV kernel for {TYPE_NAMES.get(ggml_type, ggml_type)}")
    size = nbytes_for(ggml_type, n * k)
    if blocks.numel() != size:
        raise ValueError(f"{blocks.numel()} bytes for a {n}x{k} {TYPE_NAMES[ggml_type]} tensor, expected {size}")
    data = torch.empty(size, device=dev, dtype=torch.uint8)
    check(lib.pe_repack(ggml_type, _ptr(blocks), _ptr(data), n, k, _stream(dev)), "pe_repack")
    if mfma is None:
        mfma = mfma_eligible(ggml_type, n, k)
    return QWeight(data, ggml_type, n, k, repack_mfma(blocks, ggml_type, n, k) if mfma else None,
                   repack_oproj(blocks, ggml_type, n, k) if oproj and oproj_eligible(ggml_type, n, k) else None,
                   repack_down_slices(blocks, ggml_type, n, k)
                   if slices and down_slice_eligible(ggml_type, n, k) else None,
                   repack_mfma_pairs(blocks, ggml_type, n, k, pairs_hd)
                   if pairs_hd and mqkv_eligible(ggml_type, n, k, pairs_hd) else None)


def repack_oproj(blocks: torch.Tensor, ggml_type: int, n: int, k: int) -> torch.Tensor:
    """Raw GGUF blocks of an (n x k) Q5_0 / Q8_0 matrix -> its o-projection layout (device
    uint8): per 64-column head and 16-row tile, the operand layout of attn_oproj_fix's integer
    matrix-core products."""
    dev = _on_gpu(blocks)
    size = lib.pe_oproj_layout_bytes(ggml_type, n, k)
    if size < 0:
        raise ValueError(f"no o-projection layout for a {n}x{k} {TYPE_NAMES.get(ggml_type, ggml_type)} matrix")
    if blocks.numel() != nbytes_for(ggml_type, n * k):
        raise ValueError(f"{blocks.numel()} bytes for a {n}x{k} {TYPE_NAMES[ggml_type]} tensor")
    out = torch.empty(size, device=dev, dtype=torch.uint8)
    check(lib.pe_repack_oproj(ggml_type, _ptr(blocks), _ptr(out), n, k, _stream(dev)), "pe_repack_oproj")
    return out


def _use_mfma(w: QWeight) -> bool:
    return use_mfma_gemv and w.mfma is not None


def _aligned16(t: torch.Tensor | None) -> torch.Tensor | None:
    return t if t is None or t.data_ptr() % 16 == 0 else t.clone()


def mgemv(x: torch.Tensor, w: QWeight, norm_w: torch.Tensor | None = None, eps: float = 0.0,
          residual: torch.Tensor | None = None, silu: bool = False, out: torch.Tensor | None = None,
          layout: int = LAYOUT_NATURAL) -> torch.Tensor:
    """pe_mgemv: W h (+ residual) or silu(g) * u over [g; u] = W h (``silu``), h = rmsnorm(x) *
    norm_w when ``norm_w`` is given, on the integer matrix cores from w.mfma."""
    if w.mfma is None:
        raise ValueError(f"{w} has no MFMA layout copy")
    dev = _on_gpu(x, w.mfma, norm_w, residual)
    x = _aligned16(_f32c(x.reshape(-1)))
    if x.numel() != w.k:
        raise ValueError(f"x has {x.numel()} elements, weight expects {w.k}")
    nw = None if norm_w is None else _aligned16(_f32c(norm_w.reshape(-1)))
    res = None if residual is None else residual.reshape(-1).float().contiguous()
    if silu and (w.n % 32 or res is not None):
        raise ValueError("the SiLU product needs [gate; up] rows in groups of 16 and no residual")
    n = w.n // 2 if silu else w.n
    if out is None:
        out = torch.empty(n, device=dev, dtype=torch.float32)
    check(lib.pe_mgemv(w.ggml_type, _ptr(w.mfma), n, w.k, _ptr(x), _ptr(nw), float(eps), _ptr(res),
                       _ptr(out), 1 if silu else 0, layout, _stream(dev)), "pe_mgemv")
    return out


def dequantize_weight(w: QWeight) -> torch.Tensor:
    """fp32 (n, k) from a tiled weight, through the GEMV kernels' own decode routines."""
    out = torch.empty(w.n, w.k, device=w.data.device, dtype=torch.float32)
    check(lib.pe_dequant_tiled(w.ggml_type, _ptr(w.data), _ptr(out), w.n, w.k,
                               _stream(w.data.device)), "pe_dequant_tiled")
    return out


def dequantize_weight_f16(w: QWeight, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp16 (n, k) from a tiled weight: the exact values rounded to nearest even (the prefill
    GEMM operand; autocast rounds the fp32 dequantized weights the same way). ``out`` may be a
    row slice of a larger contiguous (rows, k) fp16 tensor."""
    if out is None:
        out = torch.empty(w.n, w.k, device=w.data.device, dtype=torch.float16)
    if out.dtype != torch.float16 or tuple(out.shape) != (w.n, w.k) or not out.is_contiguous():
        raise ValueError("out must be a contiguous (n, k) float16 tensor")
    check(lib.pe_dequant_tiled_f16(w.ggml_type, _ptr(w.data), _ptr(out), w.n, w.k,
                                   _stream(w.data.device)), "pe_dequant_tiled_f16")
    return out


def gemm_f16(a: torch.Tensor, w16: torch.Tensor, bias: torch.Tensor | None = None,
             residual: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """C = A W^T (+ bias) (+ residual) on the matrix cores: A fp32 (M, K) (rows may be strided;
    rounded to fp16 as read) or fp16 (pe_gemm_h16: the same product of the same fp16 values),
    W fp16 (N, K), fp32 accumulation and result (M, N)."""
    dev = _on_gpu(a, w16, bias, residual)
    if a.dim() == 1:
        a = a.unsqueeze(0)
    if a.dtype not in (torch.float32, torch.float16):
        raise ValueError("a must be float32 or float16")
    half = a.dtype == torch.float16
    if a.stride(1) != 1 or a.stride(0) % (8 if half else 4) or a.data_ptr() % 16:
        a = a.contiguous()
    M, K = a.shape
    N = w16.shape[0]
    if w16.dtype != torch.float16 or not w16.is_contiguous() or w16.shape[1] != K:
        raise ValueError("w16 must be a contiguous (N, K) float16 tensor")
    if out is None:
        out = torch.empty(M, N, device=dev, dtype=torch.float32)
    ldr = 0
    if residual is not None:
        if residual.dtype != torch.float32 or tuple(residual.shape) != (M, N):
            raise ValueError("residual must be a float32 (M, N) tensor")
        if residual.stride(1) != 1:
            residual = residual.contiguous()
        ldr = residual.stride(0)
    fn = lib.pe_gemm_h16 if half else lib.pe_gemm_f16
    check(fn(_ptr(a), a.stride(0), _ptr(w16), _ptr(None if bias is None else _f32c(bias)),
             _ptr(residual), ldr, _ptr(out), out.stride(0), M, N, K, _stream(dev)),
          "pe_gemm_h16" if half else "pe_gemm_f16")
    return out


def interleave_gate_up_f16(gu16: torch.Tensor) -> torch.Tensor:
    """(2*ffn, K) fp16 [gate; up] rows -> the layout of gemm_f16_silu: groups of 16 gate rows
    and the 16 matching up rows alternating (ffn % 16 == 0)."""
    n, k = gu16.shape
    ffn = n // 2
    if n % 2 or ffn % 16:
        raise ValueError("gate/up rows must be 2 * ffn with ffn % 16 == 0")
    g = gu16[:ffn].reshape(ffn // 16, 16, k)
    u = gu16[ffn:].reshape(ffn // 16, 16, k)
    return torch.stack([g, u], dim=1).reshape(n, k).contiguous()


def gemm_f16_silu(a: torch.Tensor, w16_il: torch.Tensor, out: torch.Tensor | None = None,
                  half: bool = False) -> torch.Tensor:
    """silu(A Wg^T) * (A Wu^T) on the matrix cores, W = interleave_gate_up_f16([gate; up]):
    gemm_f16 then silu_mul without the (M, 2 ffn) intermediate (model.py:218-224). half: the
    result is stored in fp16 (pe_gemm_f16_silu_h), ready as gemm_f16's A operand. An fp16 A
    (rmsnorm(..., half=True)) needs half (pe_gemm_h16_silu_h) and gives the same bits as its
    fp32 original."""
    dev = _on_gpu(a, w16_il)
    if a.dim() == 1:
        a = a.unsqueeze(0)
    ah = a.dtype == torch.float16
    if a.dtype != torch.float32 and not ah:
        raise ValueError("a must be float32 or float16")
    if ah and not half:
        raise ValueError("an fp16 A needs half=True (pe_gemm_h16_silu_h)")
    if a.stride(1) != 1 or a.stride(0) % (8 if ah else 4) or a.data_ptr() % 16:
        a = a.contiguous()
    M, K = a.shape
    N = w16_il.shape[0]
    if w16_il.dtype != torch.float16 or not w16_il.is_contiguous() or w16_il.shape[1] != K or N % 32:
        raise ValueError("w16_il must be a contiguous (2*ffn, K) float16 tensor, ffn % 16 == 0")
    odt = torch.float16 if half else torch.float32
    if out is None:
        out = torch.empty(M, N // 2, device=dev, dtype=odt)
    if out.dtype != odt or out.stride(1) != 1 or tuple(out.shape) != (M, N // 2):
        raise ValueError(f"out must be a row-major ({M}, {N // 2}) {odt} tensor")
    name = "pe_gemm_h16_silu_h" if ah else "pe_gemm_f16_silu_h" if half else "pe_gemm_f16_silu"
    check(getattr(lib, name)(_ptr(a), a.stride(0), _ptr(w16_il), _ptr(out), out.stride(0), M, N // 2, K,
                             _stream(dev)), name)
    return out


def embed_gather(table: RawTensor, ids: torch.Tensor, out: torch.Tensor | None = None,
                 layout: int = LAYOUT_NATURAL):
    """Rows ``ids`` of a raw GGUF (vocab, hidden) table, dequantized (model.py:152);
    ``layout=LAYOUT_Y_UT`` writes each row unit-transposed."""
    vocab, hidden = table.shape
    need = nbytes_for(table.ggml_type, vocab * hidden)
    if table.data.numel() * table.data.element_size() < need:
        raise ValueError(f"embedding table holds {table.data.numel() * table.data.element_size()} "
                         f"bytes, a {vocab}x{hidden} {TYPE_NAMES.get(table.ggml_type)} table needs {need}")
    dev = _on_gpu(table.data, ids)
    ids = ids.to(torch.int64).contiguous()
    if out is None:
        out = torch.empty(ids.numel(), hidden, device=dev, dtype=torch.float32)
    check(lib.pe_embed_gather(table.ggml_type, _ptr(table.data), vocab, hidden, _ptr(ids),
                              ids.numel(), _ptr(out), layout, _stream(dev)), "pe_embed_gather")
    return out


# ---- reference kernels -------------------------------------------------------------------

def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, half: bool = False) -> torch.Tensor:
    """out = x / sqrt(mean(x^2) + eps) * weight over the last dim (kernels.py:26). With
    ``half`` the result is stored in fp16 (rounded to nearest even; pe_rmsnorm_h16), the
    operand of the prefill GEMMs."""
    dev = _on_gpu(x, weight)
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    x2 = x2.float()
    w = weight.float().contiguous()
    rows, n = x2.shape
    if half:
        out = torch.empty(rows, n, device=dev, dtype=torch.float16)
        check(lib.pe_rmsnorm_h16(_ptr(x2), x2.stride(0), _ptr(w), _ptr(out), n, rows, n, float(eps),
                                 _stream(dev)), "pe_rmsnorm_h16")
        return out.reshape(x.shape)
    out = torch.empty(rows, n, device=dev, dtype=torch.float32)
    check(lib.pe_rmsnorm(_ptr(x2), x2.stride(0), _ptr(w), _ptr(out), n, rows, n, float(eps),
                         _stream(dev)), "pe_rmsnorm")
    return out.reshape(x.shape).to(x.dtype)


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE; x (L, n_head, hd) (row-strided views allowed), cos/sin (L, hd/2) (kernels.py:50)."""
    dev = _on_gpu(x, cos, sin)
    L, n_head, hd = x.shape
    if x.dtype != torch.float32 or x.stride(2) != 1 or x.stride(1) != hd:
        x = x.float().contiguous()
    c, s = cos.float().contiguous(), sin.float().contiguous()
    out = torch.empty(L, n_head, hd, device=dev, dtype=torch.float32)
    check(lib.pe_rope(_ptr(x), x.stride(0), _ptr(c), _ptr(s), _ptr(out), n_head * hd, L, n_head,
                      hd, _stream(dev)), "pe_rope")
    return out


def silu_mul(gate_up: torch.Tensor, ffn: int) -> torch.Tensor:
    """silu(gate) * up from the (L, 2*ffn) [gate | up] tensor (kernels.py:77)."""
    dev = _on_gpu(gate_up)
    gu = gate_up.float()
    if gu.dim() == 1:
        gu = gu.unsqueeze(0)
    if gu.stride(-1) != 1:
        gu = gu.contiguous()
    L = gu.shape[0]
    out = torch.empty(L, ffn, device=dev, dtype=torch.float32)
    check(lib.pe_silu_mul(_ptr(gu), gu.stride(0), _ptr(out), ffn, L, ffn, _stream(dev)), "pe_silu_mul")
    return out


def round_f16_(x: torch.Tensor) -> torch.Tensor:
    """x = fp16(x) in place (round to nearest even, stored as fp32; pe_round_f16) for a float32
    tensor whose last dim is contiguous (rows of the leading dims with any row stride)."""
    _on_gpu(x)
    if x.dtype != torch.float32 or x.stride(-1) != 1:
        raise ValueError("round_f16_ needs a float32 tensor with a contiguous last dim")
    v = x if x.dim() == 2 else x.reshape(-1, x.shape[-1]) if x.is_contiguous() else None
    if v is None:
        raise ValueError("round_f16_ needs 2-D rows (or a contiguous tensor)")
    check(lib.pe_round_f16(_ptr(v), v.shape[0], v.shape[1], v.stride(0) if v.shape[0] > 1 else v.shape[1],
                           _stream(x.device)), "pe_round_f16")
    return x


def decode_attn_workspace(n_head: int, n_kv: int, hd: int, capacity: int, device) -> torch.Tensor:
    """Zero-filled workspace for decode_attn (reusable by any number of in-order calls)."""
    nbytes = lib.pe_decode_attn_workspace_bytes(n_head, n_kv, hd, capacity)
    check(0 if nbytes >= 0 else -nbytes, "pe_decode_attn_workspace_bytes")
    return torch.zeros(nbytes, device=device, dtype=torch.uint8)


def decode_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                S: torch.Tensor | int | None = None, stride: int | None = None,
                scale: float | None = None, *, S_offset: int = 0, round_fp16: bool = True,
                workspace: torch.Tensor | None = None, out: torch.Tensor | None = None,
                layout: int = LAYOUT_NATURAL):
    """Single-query GQA attention over the cache (kernels.py:129).

    q (n_head, hd); k/v (n_kv, capacity, hd); valid length S (+ ``S_offset``) read on the
    device if S is a tensor; ``stride`` (the reference's loop bound = cache capacity) defaults
    to k.shape[1]. Output rounded to fp16 and returned as fp32 like the reference.
    """
    dev = _on_gpu(q, k, v)
    q = _f32c(q)
    n_head, hd = q.shape
    n_kv, capacity, _ = k.shape
    if stride is not None:
        capacity = int(stride)
    if k.numel() < n_kv * capacity * hd or v.numel() < n_kv * capacity * hd:
        raise ValueError("stride exceeds the cache buffer")
    k, v = _f32c(k), _f32c(v)
    if scale is None:
        scale = hd ** -0.5
    if S is None:
        len_dev, dtype_code, add = None, 0, capacity + S_offset
    elif isinstance(S, int):
        len_dev, dtype_code, add = None, 0, S + S_offset
    else:
        S = S.reshape(-1)
        if S.dtype not in (torch.int32, torch.int64):
            S = S.to(torch.int64)
        S = S.contiguous()
        _on_gpu(S)
        len_dev, dtype_code, add = S, (1 if S.dtype == torch.int32 else 2), S_offset
    if workspace is None:
        workspace = decode_attn_workspace(n_head, n_kv, hd, capacity, dev)
    if out is None:
        out = torch.empty(n_head, hd, device=dev, dtype=torch.float32)
    check(lib.pe_decode_attn(_ptr(q), _ptr(k), _ptr(v), n_head, n_kv, hd, capacity, _ptr(len_dev),
                             dtype_code, add, float(scale), int(round_fp16), _ptr(out),
                             _ptr(workspace), workspace.numel(), layout, _stream(dev)), "pe_decode_attn")
    return out


def qgemv(x: torch.Tensor, w: QWeight, residual: torch.Tensor | None = None,
          bias: torch.Tensor | None = None, out: torch.Tensor | None = None,
          layout: int = LAYOUT_NATURAL) -> torch.Tensor:
    """y = W x (+ bias) (+ residual) for a tiled quantized W (M = 1); ``layout`` bits say
    which of x / (y, residual) are unit-transposed. A W with an MFMA layout copy runs on
    pe_mgemv (without a bias)."""
    if bias is None and _use_mfma(w):
        return mgemv(x, w, residual=residual, out=out, layout=layout)
    dev = _on_gpu(x, w.data, residual, bias)
    x = _f32c(x.reshape(-1))
    if x.numel() != w.k:
        raise ValueError(f"x has {x.numel()} elements, weight expects {w.k}")
    res = None if residual is None else residual.reshape(-1).float().contiguous()
    b = None if bias is None else bias.reshape(-1).float().contiguous()
    if out is None:
        out = torch.empty(w.n, device=dev, dtype=torch.float32)
    check(lib.pe_qgemv(w.ggml_type, _ptr(w.data), w.n, w.k, _ptr(x), _ptr(res), _ptr(b), _ptr(out),
                       layout, _stream(dev)), "pe_qgemv")
    return out


def _typed(w: QWeight, t: int, name: str) -> QWeight:
    if w.ggml_type != t:
        raise ValueError(f"{name} needs a {TYPE_NAMES[t]} weight, got {TYPE_NAMES[w.ggml_type]}")
    return w


def q8_0_gemv(x: torch.Tensor, w: QWeight) -> torch.Tensor:
    """Q8_0 GEMV: W x (kernels.py:178)."""
    return qgemv(x, _typed(w, GGML_Q8_0, "q8_0_gemv"))


def q5_0_gemv(x: torch.Tensor, w: QWeight) -> torch.Tensor:
    """Q5_0 GEMV: W x (kernels.py:211)."""
    return qgemv(x, _typed(w, GGML_Q5_0, "q5_0_gemv"))


def q6_k_gemv(x: torch.Tensor, w: QWeight, residual: torch.Tensor | None = None) -> torch.Tensor:
    """Q6_K GEMV: residual + W x (kernels.py:286)."""
    return qgemv(x, _typed(w, GGML_Q6_K, "q6_k_gemv"), residual=residual)


def q4_k_gemv(x: torch.Tensor, w: QWeight, residual: torch.Tensor | None = None) -> torch.Tensor:
    """Q4_K GEMV: residual + W x (kernels.py:326)."""
    return qgemv(x, _typed(w, GGML_Q4_K, "q4_k_gemv"), residual=residual)


def qgemv_norm(x: torch.Tensor, weight: torch.Tensor, w: QWeight, eps: float,
               out: torch.Tensor | None = None, layout: int = LAYOUT_NATURAL) -> torch.Tensor:
    """W (rmsnorm(x) * weight) in one launch, any quantized format (pe_mgemv for a W with an
    MFMA layout copy)."""
    if _use_mfma(w):
        return mgemv(x, w, norm_w=weight, eps=eps, out=out, layout=layout)
    dev = _on_gpu(x, weight, w.data)
    x = _f32c(x.reshape(-1))
    nw = _f32c(weight.reshape(-1))
    if out is None:
        out = torch.empty(w.n, device=dev, dtype=torch.float32)
    check(lib.pe_qgemv_rmsnorm(w.ggml_type, _ptr(w.data), w.n, w.k, _ptr(x), _ptr(nw), float(eps),
                               _ptr(out), layout, _stream(dev)), "pe_qgemv_rmsnorm")
    return out


class GreedyState:
    """Device-side greedy decode state: ``state`` = [token, pos, count] (int64) -- the next
    step's input id and position, and how many picks were made -- ``log`` of the picked ids,
    and the argmax workspace (per-workgroup partial picks)."""

    def __init__(self, n_rows: int, log_cap: int, device):
        nbytes = lib.pe_qgemv_argmax_workspace_bytes(n_rows)
        check(0 if nbytes >= 0 else -nbytes, "pe_qgemv_argmax_workspace_bytes")
        self.state = torch.zeros(3, dtype=torch.int64, device=device)
        self.log = torch.zeros(max(int(log_cap), 1), dtype=torch.int64, device=device)
        self.log_cap = int(log_cap)
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=device)

    def reset(self, token: int, pos: int, count: int = 0) -> None:
        self.state.copy_(torch.tensor([token, pos, count], dtype=torch.int64), non_blocking=False)

    @property
    def token(self) -> torch.Tensor:
        return self.state[0:1]

    @property
    def pos(self) -> torch.Tensor:
        return self.state[1:2]


def qgemv_norm_argmax(x: torch.Tensor, weight: torch.Tensor, w: QWeight, eps: float,
                      greedy: GreedyState, out: torch.Tensor | None = None,
                      layout: int = LAYOUT_NATURAL) -> torch.Tensor:
    """Logits = W (rmsnorm(x) * weight) and the greedy pick (torch.argmax of the logits) into
    ``greedy`` on the device (state[0] = pick, state[1] += 1, log[state[2]++] = pick)."""
    dev = _on_gpu(x, weight, w.data, greedy.state)
    x = _f32c(x.reshape(-1))
    nw = _f32c(weight.reshape(-1))
    if out is None:
        out = torch.empty(w.n, device=dev, dtype=torch.float32)
    check(lib.pe_qgemv_rmsnorm_argmax(w.ggml_type, _ptr(w.data), w.n, w.k, _ptr(x), _ptr(nw),
                                      float(eps), _ptr(out), _ptr(greedy.state), _ptr(greedy.log),
                                      greedy.log_cap, _ptr(greedy.workspace),
                                      greedy.workspace.numel(), layout, _stream(dev)),
          "pe_qgemv_rmsnorm_argmax")
    return out


class DecodeStep:
    """The whole decode step of a model as one launch per token (pe_decode_step): the layer
    table for one KV cache (host array + device copy) and the exchange workspace. Built once
    per cache, outside any graph capture; ``run`` launches the step on the current stream
    (capturable). Greedy only: the pick goes into a GreedyState as pe_qgemv_rmsnorm_argmax's
    does."""

    def __init__(self, model, cache, workspace: torch.Tensor):
        c = model.cfg
        dev = model.device
        self.n_layers = c.n_layers
        layers = (StepLayer * c.n_layers)()
        keep = []
        for i, L in enumerate(model.layers):
            k_buf, v_buf = cache[i]
            an = L.attn_norm.float().contiguous()
            fn = L.ffn_norm.float().contiguous()
            keep += [an, fn]
            layers[i] = StepLayer(L.wq.ggml_type, L.wk.ggml_type, L.wv.ggml_type, L.wo.ggml_type,
                                  L.w_gate_up.ggml_type, L.w_down.ggml_type,
                                  _ptr(L.wq.data), _ptr(L.wk.data), _ptr(L.wv.data), _ptr(L.wo.data),
                                  _ptr(L.w_gate_up.data), _ptr(L.w_down.data),
                                  _ptr(L.bq), _ptr(L.bk), _ptr(L.bv), _ptr(an), _ptr(fn),
                                  _ptr(k_buf), _ptr(v_buf))
        self._layers = layers
        raw = bytes(memoryview(layers).cast("B"))
        self._layers_dev = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(dev)
        self._keep = keep
        self.workspace = workspace
        self.out_norm = model.w["output_norm.weight"].float().contiguous()
        self.capacity = cache[0][0].shape[1]
        self.logits = torch.empty(model.output.n, device=dev, dtype=torch.float32)
        self.model = model
        self.n_wg = workspace_n_wg(dev)

    def run(self, greedy: "GreedyState") -> torch.Tensor:
        m, c = self.model, self.model.cfg
        a = StepArgs()
        a.layers = self._layers
        a.layers_dev = _ptr(self._layers_dev)
        a.n_layers, a.hidden, a.ffn = c.n_layers, c.hidden, c.ffn_dim
        a.n_head, a.n_kv, a.head_dim = c.n_head, c.n_kv_head, c.head_dim
        a.capacity, a.vocab, a.rope_rows = self.capacity, m.output.n, m.cos.shape[0]
        a.eps, a.scale = float(c.eps), float(c.head_dim ** -0.5)
        a.embed_type, a.embed = m.embed.ggml_type, _ptr(m.embed.data)
        a.out_type, a.w_out, a.out_norm = m.output.ggml_type, _ptr(m.output.data), _ptr(self.out_norm)
        a.cos_tab, a.sin_tab = _ptr(m.cos), _ptr(m.sin)
        a.state, a.log, a.log_cap = _ptr(greedy.state), _ptr(greedy.log), greedy.log_cap
        a.logits = _ptr(self.logits)
        a.workspace, a.workspace_bytes = _ptr(self.workspace), self.workspace.numel()
        a.n_wg = self.n_wg
        check(lib.pe_decode_step(ctypes.byref(a), _stream(self.logits.device)), "pe_decode_step")
        return self.logits

    def error(self) -> int:
        """The workspace error word: 0 after good launches, 1 if a wait ran out, 2 if a token or
        position was out of range (cleared by this call)."""
        w = int(self.workspace[64:68].view(torch.int32).item())
        if w:
            self.workspace[64:68].zero_()
        return w


def workspace_n_wg(device) -> int:
    """Workgroups of a pe_decode_step launch: one per CU of the device."""
    return int(torch.cuda.get_device_properties(device).multi_processor_count)


def decode_step_workspace(model, device) -> torch.Tensor:
    c = model.cfg
    nbytes = lib.pe_decode_step_workspace_bytes(c.n_layers, c.hidden, c.ffn_dim, c.n_head,
                                                c.n_kv_head, workspace_n_wg(device))
    check(0 if nbytes >= 0 else -nbytes, "pe_decode_step_workspace_bytes")
    return torch.zeros(nbytes, dtype=torch.uint8, device=device)


def decode_step_supported(model, capacity: int) -> bool:
    """Whether pe_decode_step covers this model and cache capacity (else the per-operation
    launches run)."""
    c = model.cfg
    if lib.pe_decode_step_supported(c.n_layers, c.hidden, c.ffn_dim, c.n_head, c.n_kv_head,
                                    c.head_dim, capacity, model.output.n) != 0:
        return False
    if model.output.ggml_type not in QUANT_TYPES:
        return False
    for L in model.layers:
        if L.w_gate_up is None:
            return False
        for w in (L.wq, L.wk, L.wv, L.wo, L.w_gate_up, L.w_down):
            if w.ggml_type not in QUANT_TYPES:
                return False
    return True


def q5_0_gemv_norm(x: torch.Tensor, weight: torch.Tensor, w: QWeight, eps: float) -> torch.Tensor:
    """Fused RMSNorm(x, weight) + Q5_0 GEMV (kernels.py:253)."""
    return qgemv_norm(x, weight, _typed(w, GGML_Q5_0, "q5_0_gemv_norm"), eps)


def qgemv_norm_silu(x: torch.Tensor, weight: torch.Tensor | None, w: QWeight, eps: float,
                    out: torch.Tensor | None = None, layout: int = LAYOUT_NATURAL) -> torch.Tensor:
    """silu(g) * u with [g; u] = W (rmsnorm(x) * weight), W = [gate; up] (2*ffn rows)
    (pe_mgemv for a W with an MFMA layout copy whose ffn is a multiple of 16)."""
    if _use_mfma(w) and w.n % 32 == 0:
        return mgemv(x, w, norm_w=weight, eps=eps, silu=True, out=out, layout=layout)
    dev = _on_gpu(x, weight, w.data)
    if w.n % 2:
        raise ValueError("gate/up weight needs an even number of rows")
    ffn = w.n // 2
    x = _f32c(x.reshape(-1))
    nw = None if weight is None else _f32c(weight.reshape(-1))
    if out is None:
        out = torch.empty(ffn, device=dev, dtype=torch.float32)
    check(lib.pe_qgemv_rmsnorm_silu(w.ggml_type, _ptr(w.data), ffn, w.k, _ptr(x), _ptr(nw),
                                    float(eps), _ptr(out), layout, _stream(dev)), "pe_qgemv_rmsnorm_silu")
    return out


def qkv_rmsnorm_rope(x: torch.Tensor, norm_w: torch.Tensor | None, eps: float,
                     wq: QWeight, wk: QWeight, wv: QWeight,
                     bq: torch.Tensor | None, bk: torch.Tensor | None, bv: torch.Tensor | None,
                     cos_tab: torch.Tensor, sin_tab: torch.Tensor, pos: torch.Tensor,
                     k_cache: torch.Tensor, v_cache: torch.Tensor, n_head: int,
                     out: torch.Tensor | None = None, layout: int = LAYOUT_NATURAL) -> torch.Tensor:
    """One decode token: q = RoPE(Wq h + bq) returned; RoPE(Wk h + bk), Wv h + bv written to
    the caches at position ``pos`` (device int64 scalar); h = rmsnorm(x) * norm_w."""
    dev = _on_gpu(x, norm_w, wq.data, wk.data, wv.data, pos, k_cache, v_cache)
    n_kv, capacity, hd = k_cache.shape
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("KV caches must be contiguous (n_kv, capacity, hd) buffers")
    if pos.dtype != torch.int64:
        raise ValueError("pos must be an int64 device tensor")
    x = _f32c(x.reshape(-1))
    if out is None:
        out = torch.empty(n_head, hd, device=dev, dtype=torch.float32)
    mq = mqkv_ok(wq, wk, wv) and norm_w is not None
    a = QkvArgs(wq.ggml_type, wk.ggml_type, wv.ggml_type,
                *((wq.pairs.data_ptr(), wk.pairs.data_ptr(), wv.pairs.data_ptr()) if mq else
                  (wq.data.data_ptr(), wk.data.data_ptr(), wv.data.data_ptr())),
                None if bq is None else bq.data_ptr(), None if bk is None else bk.data_ptr(),
                None if bv is None else bv.data_ptr(),
                x.data_ptr(), None if norm_w is None else norm_w.data_ptr(), float(eps),
                cos_tab.data_ptr(), sin_tab.data_ptr(), cos_tab.shape[0],
                pos.data_ptr(), out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                capacity, wq.k, n_head, n_kv, hd, layout)
    if mq:
        check(lib.pe_mqkv_rmsnorm_rope(ctypes.byref(a), _stream(dev)), "pe_mqkv_rmsnorm_rope")
    else:
        check(lib.pe_qkv_rmsnorm_rope(ctypes.byref(a), _stream(dev)), "pe_qkv_rmsnorm_rope")
    return out


def mqkv_ok(wq: QWeight, wk: QWeight, wv: QWeight) -> bool:
    """Whether qkv_rmsnorm_rope runs on the integer matrix cores (pe_mqkv_rmsnorm_rope): every
    segment has its RoPE-pair layout and q and k share a format (with an RMSNorm weight)."""
    return (use_mqkv and wq.pairs is not None and wk.pairs is not None and wv.pairs is not None
            and wq.ggml_type == wk.ggml_type)


def attn_gproj_supported(n_head: int, n_kv: int, hd: int, capacity: int, wo: QWeight) -> bool:
    """Whether attn_gproj covers these shapes (else decode_attn + qgemv)."""
    return lib.pe_attn_gproj_supported(n_head, n_kv, hd, capacity, wo.ggml_type, wo.n) == 0


def attn_gproj(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, wo: QWeight,
               S: torch.Tensor | int | None = None, S_offset: int = 0, scale: float | None = None,
               round_fp16: bool = True, out: torch.Tensor | None = None,
               layout: int = LAYOUT_NATURAL) -> torch.Tensor:
    """Per-kv-group shares of Wo decode_attn(q, k, v, S), shape (n_kv, wo.n): part j is Wo
    restricted to the columns of kv group j's query heads times their attention output, so
    ``residual + parts.sum(0)`` (in row order) is the o-projection with its residual. Same S
    conventions and fp16 output rounding as decode_attn; layout LAYOUT_Y_UT stores each part
    unit-transposed."""
    dev = _on_gpu(q, k, v, wo.data)
    n_head, hd = q.shape[-2], q.shape[-1]
    n_kv, capacity = k.shape[0], k.shape[1]
    q = _f32c(q.reshape(n_head, hd))
    if not (k.is_contiguous() and v.is_contiguous()):
        raise ValueError("KV caches must be contiguous (n_kv, capacity, hd) buffers")
    if scale is None:
        scale = 1.0 / float(hd) ** 0.5
    len_dev, len_dtype, len_add = None, 0, int(S_offset)
    if isinstance(S, torch.Tensor):
        len_dev = S
        len_dtype = {torch.int32: 1, torch.int64: 2}[S.dtype]
    elif S is not None:
        len_add += int(S)
    else:
        len_add += capacity
    if out is None:
        out = torch.empty(n_kv, wo.n, device=dev, dtype=torch.float32)
    check(lib.pe_attn_gproj(_ptr(q), _ptr(k), _ptr(v), n_head, n_kv, hd, capacity, _ptr(len_dev),
                            len_dtype, len_add, float(scale), int(round_fp16), wo.ggml_type,
                            _ptr(wo.data), wo.n, _ptr(out), layout, _stream(dev)), "pe_attn_gproj")
    return out


def attn_split_gproj_supported(n_head: int, n_kv: int, hd: int, capacity: int, wo: QWeight) -> bool:
    """Whether attn_split_gproj covers these shapes (head_dim 64, up to 8 query heads per kv
    head, any capacity)."""
    return lib.pe_attn_split_gproj_supported(n_head, n_kv, hd, capacity, wo.ggml_type, wo.n) == 0


def attn_split_gproj(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, wo: QWeight,
                     S: torch.Tensor | int | None = None, S_offset: int = 0,
                     workspace: torch.Tensor | None = None, scale: float | None = None,
                     round_fp16: bool = True, out: torch.Tensor | None = None,
                     layout: int = LAYOUT_NATURAL) -> torch.Tensor:
    """attn_gproj for caches of any length: the split attention's chunk records (in
    ``workspace``, decode_attn_workspace bytes), then one launch that merges them per kv group
    and multiplies by that group's columns of Wo. Same result conventions as attn_gproj."""
    dev = _on_gpu(q, k, v, wo.data)
    n_head, hd = q.shape[-2], q.shape[-1]
    n_kv, capacity = k.shape[0], k.shape[1]
    q = _f32c(q.reshape(n_head, hd))
    if not (k.is_contiguous() and v.is_contiguous()):
        raise ValueError("KV caches must be contiguous (n_kv, capacity, hd) buffers")
    if scale is None:
        scale = 1.0 / float(hd) ** 0.5
    len_dev, len_dtype, len_add = None, 0, int(S_offset)
    if isinstance(S, torch.Tensor):
        len_dev = S
        len_dtype = {torch.int32: 1, torch.int64: 2}[S.dtype]
    elif S is not None:
        len_add += int(S)
    else:
        len_add += capacity
    if workspace is None:
        workspace = decode_attn_workspace(n_head, n_kv, hd, capacity, dev)
    if out is None:
        out = torch.empty(n_kv, wo.n, device=dev, dtype=torch.float32)
    check(lib.pe_attn_split_gproj(_ptr(q), _ptr(k), _ptr(v), n_head, n_kv, hd, capacity, _ptr(len_dev),
                                  len_dtype, len_add, float(scale), int(round_fp16), wo.ggml_type,
                                  _ptr(wo.data), wo.n, _ptr(out), _ptr(workspace), workspace.numel(),
                                  layout, _stream(dev)), "pe_attn_split_gproj")
    return out


def qgemv_sum_norm_silu(x: torch.Tensor, parts: torch.Tensor, weight: torch.Tensor, w: QWeight,
                        eps: float, out: torch.Tensor | None = None,
                        x_sum: torch.Tensor | None = None,
                        layout: int = LAYOUT_NATURAL) -> tuple[torch.Tensor, torch.Tensor]:
    """(silu(g) * u, x_sum) with x_sum = x + parts.sum(0) (added in row order) and
    [g; u] = W (rmsnorm(x_sum) * weight); parts (n, k) with n <= 16. layout: LAYOUT_X_UT when
    x, parts, weight and x_sum are unit-transposed, LAYOUT_Y_UT for the result."""
    dev = _on_gpu(x, parts, weight, w.data)
    if w.n % 2:
        raise ValueError("gate/up weight needs an even number of rows")
    ffn = w.n // 2
    x = _f32c(x.reshape(-1))
    parts = _f32c(parts)
    nw = _f32c(weight.reshape(-1))
    if out is None:
        out = torch.empty(ffn, device=dev, dtype=torch.float32)
    if x_sum is None:
        x_sum = torch.empty_like(x)
    check(lib.pe_qgemv_sum_rmsnorm_silu(w.ggml_type, _ptr(w.data), ffn, w.k, _ptr(x), _ptr(parts),
                                        parts.shape[0], _ptr(nw), float(eps), _ptr(out), _ptr(x_sum),
                                        layout, _stream(dev)), "pe_qgemv_sum_rmsnorm_silu")
    return out, x_sum


def attn_oproj_supported(n_head: int, n_kv: int, hd: int, capacity: int, wo: QWeight) -> bool:
    """Whether attn_oproj_fix covers these shapes (head_dim 64, caches of <= 128 positions,
    a Q5_0 / Q8_0 Wo with its o-projection layout copy)."""
    return (wo.oproj is not None and
            lib.pe_attn_oproj_fix_supported(wo.ggml_type, wo.n, n_head, n_kv, hd, capacity) == 0)


def fix_acc(hidden: int, device, layers: int = 1) -> torch.Tensor:
    """Zeroed fixed-point accumulators for attn_oproj_fix: (layers, hidden + 2) int64 (hidden
    sums, the unrepresentable-value count, padding to 16 bytes)."""
    return torch.zeros(layers, hidden + 2, device=device, dtype=torch.int64)


def attn_oproj_fix(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, wo: QWeight,
                   pos: torch.Tensor, acc: torch.Tensor, scale: float | None = None,
                   layout: int = LAYOUT_NATURAL) -> torch.Tensor:
    """Decode attention of every query head over cache positions 0..pos (the token's own row
    already written at pos), output rounded to fp16, times the head's columns of Wo, added
    into ``acc`` (hidden + 1 int64, 2^-32 fixed point; acc[hidden] counts unrepresentable
    values) by pe_attn_oproj_fix. Wo needs its o-projection layout (QWeight.oproj). Returns
    acc. layout: LAYOUT_Y_UT stores acc in the unit-transposed layout of x."""
    dev = _on_gpu(q, k_cache, v_cache, pos, acc, wo.data)
    if wo.oproj is None:
        raise ValueError(f"{wo} has no o-projection layout copy")
    n_head, hd = q.shape[-2], q.shape[-1]
    n_kv, capacity = k_cache.shape[0], k_cache.shape[1]
    q = _f32c(q.reshape(n_head, hd))
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("KV caches must be contiguous (n_kv, capacity, hd) buffers")
    if k_cache.shape != (n_kv, capacity, hd) or v_cache.shape != k_cache.shape:
        raise ValueError(f"KV caches of shape {tuple(k_cache.shape)}, {tuple(v_cache.shape)} for head_dim {hd}")
    if wo.k != n_head * hd:
        raise ValueError(f"{wo} has {wo.k} columns for {n_head} heads of {hd}")
    if pos.dtype != torch.int64:
        raise ValueError("pos must be an int64 device tensor")
    if acc.dtype != torch.int64 or acc.numel() < wo.n + 1 or not acc.is_contiguous():
        raise ValueError(f"acc must be a contiguous int64 tensor of at least {wo.n + 1} elements")
    a = AttnOprojArgs(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), capacity, pos.data_ptr(),
                      n_head, n_kv, hd, float(hd ** -0.5 if scale is None else scale),
                      wo.ggml_type, wo.oproj.data_ptr(), wo.n, acc.data_ptr(), layout)
    check(lib.pe_attn_oproj_fix(ctypes.byref(a), _stream(dev)), "pe_attn_oproj_fix")
    return acc


def qgemv_fix_norm_silu(x: torch.Tensor, fix: torch.Tensor, weight: torch.Tensor, w: QWeight,
                        eps: float, out: torch.Tensor | None = None,
                        x_sum: torch.Tensor | None = None,
                        layout: int = LAYOUT_NATURAL) -> tuple[torch.Tensor, torch.Tensor]:
    """(silu(g) * u, x_sum) with x_sum = x + 2^-32 fix (fix: attn_oproj_fix's accumulator,
    the layout of x) and [g; u] = W (rmsnorm(x_sum) * weight) (pe_qgemv_fix_rmsnorm_silu)."""
    dev = _on_gpu(x, fix, weight, w.data)
    if w.n % 2:
        raise ValueError("gate/up weight needs an even number of rows")
    ffn = w.n // 2
    x = _f32c(x.reshape(-1))
    nw = _f32c(weight.reshape(-1))
    if fix.dtype != torch.int64 or fix.numel() < w.k + 1 or not fix.is_contiguous():
        raise ValueError(f"fix must be a contiguous int64 tensor of at least {w.k + 1} elements")
    if out is None:
        out = torch.empty(ffn, device=dev, dtype=torch.float32)
    if x_sum is None:
        x_sum = torch.empty_like(x)
    check(lib.pe_qgemv_fix_rmsnorm_silu(w.ggml_type, _ptr(w.data), ffn, w.k, _ptr(x), _ptr(fix), _ptr(nw),
                                        float(eps), _ptr(out), _ptr(x_sum), layout, _stream(dev)),
          "pe_qgemv_fix_rmsnorm_silu")
    return out, x_sum


# ---- the fused FFN launch and its consumer -------------------------------------------------

FFN_REPLICAS = 4


def fix_stride(hidden: int) -> int:
    """Elements per fixed-point accumulator copy: hidden sums, the unrepresentable-value count,
    padding to a multiple of 32 (256-byte aligned copies)."""
    return hidden + 32


def fix_acc_block(hidden: int, device, layers: int, replicas: int = FFN_REPLICAS) -> torch.Tensor:
    """Zeroed accumulators of a fused decode step: (layers, 1 + replicas, fix_stride(hidden))
    int64; [l, 0] is layer l's o-projection accumulator (attn_oproj_fix), [l, 1:] the replicas
    of its down product (ffn_fix). One fill clears them all."""
    return torch.zeros(layers, 1 + replicas, fix_stride(hidden), device=device, dtype=torch.int64)


def ffn_fix_supported(w_gu: QWeight | None, w_down: QWeight) -> bool:
    """Whether ffn_fix covers this layer: [gate; up] one Q5_0 / Q8_0 tensor, ffn_down with its
    down-slice layout copy, hidden <= 2048."""
    return (w_gu is not None and w_down.slices is not None and w_gu.n == 2 * w_down.k and
            w_gu.k == w_down.n and
            lib.pe_ffn_fix_supported(w_gu.ggml_type, w_down.ggml_type, w_down.n, w_down.k) == 0)


def ffn_fix(x: torch.Tensor, acc_in: torch.Tensor, norm_w: torch.Tensor, w_gu: QWeight,
            w_down: QWeight, eps: float, acc_out: torch.Tensor, x_sum: torch.Tensor | None = None,
            layout: int = LAYOUT_NATURAL) -> torch.Tensor:
    """The decode FFN in one launch (pe_ffn_fix): x_sum = x + 2^-32 acc_in (acc_in:
    attn_oproj_fix's accumulator), act = SiLU(W_gate h) * (W_up h) with h = rmsnorm(x_sum) *
    norm_w, and W_down act added in 2^-32 fixed point into the replicas of ``acc_out``
    ((replicas, stride) int64, zero or holding what to add to). Returns x_sum; the FFN output
    with its residual is x_sum + 2^-32 acc_out.sum(0) (qkv_fix_rmsnorm_rope reads it).
    layout: LAYOUT_X_UT for x, acc_in, norm_w and x_sum, LAYOUT_Y_UT for acc_out."""
    dev = _on_gpu(x, acc_in, norm_w, w_gu.data, acc_out)
    if w_down.slices is None:
        raise ValueError(f"{w_down} has no down-slice layout copy")
    hidden, ffn = w_down.n, w_down.k
    if w_gu.n != 2 * ffn or w_gu.k != hidden:
        raise ValueError(f"[gate; up] {w_gu} does not match ffn_down {w_down}")
    x = _f32c(x.reshape(-1))
    nw = _f32c(norm_w.reshape(-1))
    if acc_in.dtype != torch.int64 or acc_in.numel() < hidden + 1 or not acc_in.is_contiguous():
        raise ValueError(f"acc_in must be a contiguous int64 tensor of at least {hidden + 1} elements")
    if acc_out.dtype != torch.int64 or acc_out.dim() != 2 or not acc_out.is_contiguous():
        raise ValueError("acc_out must be a contiguous (replicas, stride) int64 tensor")
    if x_sum is None:
        x_sum = torch.empty_like(x)
    a = FfnFixArgs(w_gu.ggml_type, w_gu.data.data_ptr(), w_down.ggml_type, w_down.slices.data_ptr(),
                   hidden, ffn, x.data_ptr(), acc_in.data_ptr(), nw.data_ptr(), float(eps),
                   x_sum.data_ptr(), acc_out.data_ptr(), acc_out.shape[0], acc_out.shape[1], layout)
    check(lib.pe_ffn_fix(ctypes.byref(a), _stream(dev)), "pe_ffn_fix")
    return x_sum


def ffn_fix_bound(ffn: int) -> float:
    """The magnitude from which ffn_fix counts an addend as unrepresentable."""
    return float(lib.pe_ffn_fix_bound(ffn))


def qkv_fix_rmsnorm_rope(x: torch.Tensor, acc: torch.Tensor | None, norm_w: torch.Tensor, eps: float,
                         wq: QWeight, wk: QWeight, wv: QWeight,
                         bq: torch.Tensor | None, bk: torch.Tensor | None, bv: torch.Tensor | None,
                         cos_tab: torch.Tensor, sin_tab: torch.Tensor, pos: torch.Tensor,
                         k_cache: torch.Tensor, v_cache: torch.Tensor, n_head: int,
                         x_sum: torch.Tensor | None = None, out: torch.Tensor | None = None,
                         layout: int = LAYOUT_NATURAL) -> tuple[torch.Tensor, torch.Tensor | None]:
    """qkv_rmsnorm_rope over x + 2^-32 acc.sum(0) (acc: ffn_fix's (4, stride) replicas, or None
    for x alone), staged once per workgroup (pe_qkv_fix_rmsnorm_rope). Returns (q, x_sum):
    x_sum receives the summed vector when acc is given (else None: it is x)."""
    dev = _on_gpu(x, acc, norm_w, wq.data, wk.data, wv.data, pos, k_cache, v_cache)
    n_kv, capacity, hd = k_cache.shape
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("KV caches must be contiguous (n_kv, capacity, hd) buffers")
    if pos.dtype != torch.int64:
        raise ValueError("pos must be an int64 device tensor")
    x = _f32c(x.reshape(-1))
    nw = _f32c(norm_w.reshape(-1))
    replicas, stride = 0, 0
    if acc is not None:
        if acc.dtype != torch.int64 or acc.dim() != 2 or not acc.is_contiguous():
            raise ValueError("acc must be a contiguous (replicas, stride) int64 tensor")
        replicas, stride = acc.shape
        if x_sum is None:
            x_sum = torch.empty_like(x)
    else:
        x_sum = None
    if out is None:
        out = torch.empty(n_head, hd, device=dev, dtype=torch.float32)
    a = QkvArgs(wq.ggml_type, wk.ggml_type, wv.ggml_type,
                wq.data.data_ptr(), wk.data.data_ptr(), wv.data.data_ptr(),
                None if bq is None else bq.data_ptr(), None if bk is None else bk.data_ptr(),
                None if bv is None else bv.data_ptr(),
                x.data_ptr(), nw.data_ptr(), float(eps),
                cos_tab.data_ptr(), sin_tab.data_ptr(), cos_tab.shape[0],
                pos.data_ptr(), out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                capacity, wq.k, n_head, n_kv, hd, layout)
    check(lib.pe_qkv_fix_rmsnorm_rope(ctypes.byref(a), _ptr(acc), replicas, stride, _ptr(x_sum),
                                      _stream(dev)), "pe_qkv_fix_rmsnorm_rope")
    return out, x_sum


# embedding table formats the first-layer QKV launch decodes itself (pe_qkv_embed_rmsnorm_rope)
EMBED_QKV_TYPES = (GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q5_0, GGML_Q4_K, GGML_Q6_K)


def qkv_embed_rmsnorm_rope(table: RawTensor, token: torch.Tensor, norm_w: torch.Tensor, eps: float,
                           wq: QWeight, wk: QWeight, wv: QWeight,
                           bq: torch.Tensor | None, bk: torch.Tensor | None, bv: torch.Tensor | None,
                           cos_tab: torch.Tensor, sin_tab: torch.Tensor, pos: torch.Tensor,
                           k_cache: torch.Tensor, v_cache: torch.Tensor, n_head: int,
                           x_out: torch.Tensor, clear: torch.Tensor | None = None,
                           out: torch.Tensor | None = None,
                           layout: int = LAYOUT_NATURAL) -> torch.Tensor:
    """qkv_fix_rmsnorm_rope (no replicas) of the embedding row of ``token`` (a device int64
    scalar): the row is decoded into ``x_out`` (the residual stream, in ``layout``) and
    ``clear`` (a contiguous tensor of whole 16-byte words, e.g. the step's fixed-point
    accumulators) is zeroed, in the same launch (pe_qkv_embed_rmsnorm_rope). Returns q."""
    dev = _on_gpu(table.data, token, norm_w, wq.data, wk.data, wv.data, pos, k_cache, v_cache, x_out)
    vocab, hidden = table.shape
    need = nbytes_for(table.ggml_type, vocab * hidden)
    if table.data.numel() * table.data.element_size() < need:
        raise ValueError(f"embedding table holds fewer than {need} bytes")
    n_kv, capacity, hd = k_cache.shape
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("KV caches must be contiguous (n_kv, capacity, hd) buffers")
    if pos.dtype != torch.int64 or token.dtype != torch.int64:
        raise ValueError("pos and token must be int64 device tensors")
    if x_out.dtype != torch.float32 or not x_out.is_contiguous() or x_out.numel() != hidden:
        raise ValueError("x_out must be a contiguous float32 vector of the hidden size")
    nbytes = 0
    if clear is not None:
        if not clear.is_contiguous():
            raise ValueError("clear must be contiguous")
        nbytes = clear.numel() * clear.element_size()
    nw = _f32c(norm_w.reshape(-1))
    if out is None:
        out = torch.empty(n_head, hd, device=dev, dtype=torch.float32)
    a = QkvArgs(wq.ggml_type, wk.ggml_type, wv.ggml_type,
                wq.data.data_ptr(), wk.data.data_ptr(), wv.data.data_ptr(),
                None if bq is None else bq.data_ptr(), None if bk is None else bk.data_ptr(),
                None if bv is None else bv.data_ptr(),
                None, nw.data_ptr(), float(eps),
                cos_tab.data_ptr(), sin_tab.data_ptr(), cos_tab.shape[0],
                pos.data_ptr(), out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                capacity, wq.k, n_head, n_kv, hd, layout)
    check(lib.pe_qkv_embed_rmsnorm_rope(ctypes.byref(a), table.ggml_type, _ptr(table.data), vocab,
                                        _ptr(token), _ptr(x_out), _ptr(clear), nbytes, _stream(dev)),
          "pe_qkv_embed_rmsnorm_rope")
    return out


# ---- prefill (M >= 1) --------------------------------------------------------------------

def qgemm(x: torch.Tensor, w: QWeight, bias: torch.Tensor | None = None,
          residual: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """y[m] = W x[m] (+ bias) (+ residual[m]) for x (M, k); out may be a column slice view."""
    dev = _on_gpu(x, w.data, bias, residual)
    if x.dim() == 1:
        x = x.unsqueeze(0)
    if x.dtype != torch.float32 or x.stride(-1) != 1 or x.stride(0) % 4 or x.data_ptr() % 16:
        x = _f32c(x)
    M = x.shape[0]
    if out is None:
        out = torch.empty(M, w.n, device=dev, dtype=torch.float32)
    if out.stride(-1) != 1:
        raise ValueError("out rows must be contiguous")
    res_stride = 0
    if residual is not None:
        if residual.dtype != torch.float32 or residual.stride(-1) != 1:
            residual = residual.float().contiguous()
        res_stride = residual.stride(0) if residual.dim() == 2 else w.n
    check(lib.pe_qgemm(w.ggml_type, _ptr(w.data), w.n, w.k, _ptr(x), x.stride(0), M, _ptr(bias),
                       _ptr(residual), res_stride, _ptr(out), out.stride(0), _stream(dev)), "pe_qgemm")
    return out


def kv_write(k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
             pos0: int = 0) -> None:
    """cache[h][pos0 + l] = k[l, h] (and v); k, v (L, n_kv, hd) with contiguous rows of heads."""
    dev = _on_gpu(k, v, k_cache, v_cache)
    L, n_kv, hd = k.shape
    if k.stride(2) != 1 or k.stride(1) != hd or v.stride() != k.stride():
        k, v = k.contiguous(), v.contiguous()
    check(lib.pe_kv_write(_ptr(k), _ptr(v), k.stride(0), n_kv, hd, L, pos0, _ptr(k_cache),
                          _ptr(v_cache), k_cache.shape[1], _stream(dev)), "pe_kv_write")


def kv16_blocks(n_kv: int, length: int, device) -> torch.Tensor:
    """A zeroed buffer for the fp16 key blocks of ``length`` positions (head_dim 64), filled by
    rope_kv_write(kv16=...) and read by flash_prefill_blocks: (n_kv, ceil(length / 64), 16384)
    bytes; positions past ``length`` in the last block stay zero."""
    return torch.zeros(n_kv, (length + 63) // 64, 16384, device=device, dtype=torch.uint8)


def rope_kv_write(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, n_head: int,
                  k_cache: torch.Tensor, v_cache: torch.Tensor, pos0: int = 0,
                  out: torch.Tensor | None = None, kv16: torch.Tensor | None = None) -> torch.Tensor:
    """RoPE of the q and k heads of the fused QKV rows and the cache write of k and v in one
    pass: returns rope(q) (L, n_head, hd); k_cache[h][pos0 + l] = rope(k[l][h]), v likewise
    unrotated. qkv (L, (n_head + 2 n_kv) hd) with contiguous rows (row stride allowed), cos/sin
    (L, hd/2): the same values as rope + kv_write (model.py:186-197). ``kv16`` (kv16_blocks,
    head_dim 64): the same k and v also go there, rounded to fp16, as flash_prefill_blocks'
    key blocks (pe_rope_kv_write_blocks)."""
    dev = _on_gpu(qkv, cos, sin, k_cache, v_cache)
    n_kv, capacity, hd = k_cache.shape
    L = qkv.shape[0]
    if qkv.dtype != torch.float32 or qkv.stride(1) != 1 or qkv.shape[1] != (n_head + 2 * n_kv) * hd:
        raise ValueError("qkv must be float32 (L, (n_head + 2 n_kv) hd) with contiguous rows")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("KV caches must be contiguous (n_kv, capacity, hd) buffers")
    c, s = cos.float().contiguous(), sin.float().contiguous()
    if out is None:
        out = torch.empty(L, n_head, hd, device=dev, dtype=torch.float32)
    if kv16 is None:
        check(lib.pe_rope_kv_write(_ptr(qkv), qkv.stride(0), _ptr(c), _ptr(s), n_head, n_kv, hd, L, int(pos0),
                                   _ptr(out), _ptr(k_cache), _ptr(v_cache), capacity, _stream(dev)),
              "pe_rope_kv_write")
    else:
        if kv16.dtype != torch.uint8 or not kv16.is_contiguous() or kv16.dim() != 3 or kv16.shape[0] != n_kv \
                or kv16.shape[2] != 16384:
            raise ValueError("kv16 must be a contiguous uint8 (n_kv, blocks, 16384) buffer (kv16_blocks)")
        check(lib.pe_rope_kv_write_blocks(_ptr(qkv), qkv.stride(0), _ptr(c), _ptr(s), n_head, n_kv, hd, L,
                                          int(pos0), _ptr(out), _ptr(k_cache), _ptr(v_cache), capacity,
                                          _ptr(kv16), kv16.shape[1], _stream(dev)),
              "pe_rope_kv_write_blocks")
    return out


def prefill_attn(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, pos0: int = 0,
                 scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Causal GQA attention of q (L, n_head, hd) at positions pos0.. over the cache (fp32)."""
    dev = _on_gpu(q, k_cache, v_cache)
    L, n_head, hd = q.shape
    n_kv, capacity, _ = k_cache.shape
    if q.stride(2) != 1 or q.stride(1) != hd:
        q = q.contiguous()
    if scale is None:
        scale = hd ** -0.5
    if out is None:
        out = torch.empty(L, n_head * hd, device=dev, dtype=torch.float32)
    check(lib.pe_prefill_attn(_ptr(q), q.stride(0), _ptr(k_cache), _ptr(v_cache), n_head, n_kv, hd,
                              capacity, L, pos0, float(scale), _ptr(out), out.stride(0),
                              _stream(dev)), "pe_prefill_attn")
    return out


def flash_prefill(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, pos0: int = 0,
                  scale: float | None = None, out: torch.Tensor | None = None,
                  half: bool = False) -> torch.Tensor:
    """prefill_attn on the matrix cores: q, k, v rounded to fp16 as read, fp32 softmax and
    accumulation (the reference's fp16 SDPA prefill, model.py:201-209); head_dim 64. With
    ``half`` the output is stored in fp16 (pe_flash_prefill_h16), the o-projection's operand."""
    dev = _on_gpu(q, k_cache, v_cache)
    L, n_head, hd = q.shape
    n_kv, capacity, _ = k_cache.shape
    if q.stride(2) != 1 or q.stride(1) != hd or q.stride(0) % 4 or q.data_ptr() % 16:
        q = q.contiguous()
    if scale is None:
        scale = hd ** -0.5
    if out is None:
        out = torch.empty(L, n_head * hd, device=dev, dtype=torch.float16 if half else torch.float32)
    if (out.dtype == torch.float16) != half:
        raise ValueError("out dtype must be float16 with half=True, float32 otherwise")
    fn = lib.pe_flash_prefill_h16 if half else lib.pe_flash_prefill
    check(fn(_ptr(q), q.stride(0), _ptr(k_cache), _ptr(v_cache), n_head, n_kv, hd,
             capacity, L, pos0, float(scale), _ptr(out), out.stride(0), _stream(dev)),
          "pe_flash_prefill_h16" if half else "pe_flash_prefill")
    return out


def flash_prefill_blocks_workspace(n_head: int, n_kv: int, L: int) -> int:
    """Bytes of the workspace flash_prefill_blocks splits long prompts with (0: none needed)."""
    return int(lib.pe_flash_prefill_blocks_workspace(n_head, n_kv, L))


def flash_prefill_blocks(q: torch.Tensor, kv16: torch.Tensor, scale: float | None = None,
                         out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                         split: bool = True) -> torch.Tensor:
    """flash_prefill(half=True) of a prompt from position 0, reading K and V from the fp16 key
    blocks rope_kv_write(kv16=...) wrote (pe_flash_prefill_blocks); head_dim 64; q is rounded to
    fp16 after its scale * log2 e scaling (within a few fp16 ulps of flash_prefill(half=True)).
    split=False: one workgroup per 32-query set over all its keys.
    split=True: query sets that see more than 64 key blocks (L > 4096) run as several key
    ranges merged by a second launch (within fp32 rounding of the unsplit order), in
    ``workspace`` (uint8, at least flash_prefill_blocks_workspace bytes; allocated when None)."""
    dev = _on_gpu(q, kv16)
    L, n_head, hd = q.shape
    n_kv, nblk = kv16.shape[0], kv16.shape[1]
    if kv16.dtype != torch.uint8 or not kv16.is_contiguous() or kv16.dim() != 3 or kv16.shape[2] != 16384:
        raise ValueError("kv16 must be a contiguous uint8 (n_kv, blocks, 16384) buffer (kv16_blocks)")
    if q.stride(2) != 1 or q.stride(1) != hd or q.stride(0) % 4 or q.data_ptr() % 16:
        q = q.contiguous()
    if scale is None:
        scale = hd ** -0.5
    if out is None:
        out = torch.empty(L, n_head * hd, device=dev, dtype=torch.float16)
    if out.dtype != torch.float16:
        raise ValueError("out must be float16")
    ws_ptr, ws_bytes = None, 0
    if split:
        need = flash_prefill_blocks_workspace(n_head, n_kv, L)
        if need:
            if workspace is None:
                workspace = torch.empty(need, device=dev, dtype=torch.uint8)
            if workspace.dtype != torch.uint8 or not workspace.is_contiguous():
                raise ValueError("workspace must be a contiguous uint8 buffer")
            ws_ptr, ws_bytes = _ptr(workspace), workspace.numel()
    check(lib.pe_flash_prefill_blocks(_ptr(q), q.stride(0), _ptr(kv16), nblk, n_head, n_kv, hd, L, float(scale),
                                      _ptr(out), out.stride(0), ws_ptr, ws_bytes, _stream(dev)),
          "pe_flash_prefill_blocks")
    return out


GEMM_LT_WORKSPACE = 32 << 20


def gemm_lt_workspace(device) -> torch.Tensor:
    """Device workspace for gemm_lt (hipBLASLt), reusable by calls made in order on a stream.
    Also creates the device's hipBLASLt handle now (pe_gemm_lt_init), outside any capture."""
    with torch.cuda.device(torch.device(device)):
        check(lib.pe_gemm_lt_init(), "pe_gemm_lt_init")
    return torch.empty(GEMM_LT_WORKSPACE, device=device, dtype=torch.uint8)


def gemm_lt(a16: torch.Tensor, w16: torch.Tensor, bias: torch.Tensor | None = None,
            residual: torch.Tensor | None = None, out: torch.Tensor | None = None,
            workspace: torch.Tensor | None = None) -> torch.Tensor:
    """C = A W^T (+ bias) (+ residual) on hipBLASLt (pe_gemm_lt): A fp16 (M, K) (rows may be
    strided), W fp16 (N, K), fp32 accumulation and result (M, N). ``residual`` may be ``out``
    (added in place); its row stride must equal out's."""
    dev = _on_gpu(a16, w16, bias, residual)
    if a16.dim() == 1:
        a16 = a16.unsqueeze(0)
    if a16.dtype != torch.float16:
        raise ValueError("a16 must be float16")
    if a16.stride(1) != 1 or a16.stride(0) % 8 or a16.data_ptr() % 16:
        a16 = a16.contiguous()
    M, K = a16.shape
    N = w16.shape[0]
    if w16.dtype != torch.float16 or not w16.is_contiguous() or w16.shape[1] != K:
        raise ValueError("w16 must be a contiguous (N, K) float16 tensor")
    if out is None:
        out = torch.empty(M, N, device=dev, dtype=torch.float32)
    if out.dtype != torch.float32 or tuple(out.shape) != (M, N) or out.stride(1) != 1:
        raise ValueError("out must be a float32 (M, N) tensor with unit column stride")
    ldr = 0
    if residual is not None:
        if residual.dtype != torch.float32 or tuple(residual.shape) != (M, N):
            raise ValueError("residual must be a float32 (M, N) tensor")
        if residual.stride(1) != 1 or residual.stride(0) != out.stride(0):
            residual = residual.contiguous()
            if residual.stride(0) != out.stride(0):
                raise ValueError("residual must have out's row stride")
        ldr = residual.stride(0)
    if workspace is None:
        workspace = gemm_lt_workspace(dev)
    check(lib.pe_gemm_lt(_ptr(a16), a16.stride(0), _ptr(w16), M, N, K,
                         _ptr(None if bias is None else _f32c(bias)), _ptr(residual), ldr, _ptr(out),
                         out.stride(0), _ptr(workspace), workspace.numel(), _stream(dev)), "pe_gemm_lt")
    return out


__all__ = ["LAYOUT_NATURAL", "LAYOUT_X_UT", "LAYOUT_Y_UT", "to_ut", "from_ut", "QWeight", "RawTensor", "dequantize", "pack_weight", "dequantize_weight", "embed_gather",
           "rmsnorm", "rope", "silu_mul", "decode_attn", "decode_attn_workspace", "qgemv",
           "q8_0_gemv", "q5_0_gemv", "q5_0_gemv_norm", "q6_k_gemv", "q4_k_gemv", "qgemv_norm",
           "qgemv_norm_silu", "qkv_rmsnorm_rope", "qgemv_sum_norm_silu", "qgemm", "kv_write", "prefill_attn",
           "gemm_lt", "gemm_lt_workspace", "mgemv", "repack_mfma", "mfma_eligible", "MFMA_MIN_WEIGHTS",
           "repack_mfma_pairs", "mqkv_eligible", "mqkv_ok", "MQKV_MAX_HIDDEN", "qkv_embed_rmsnorm_rope", "EMBED_QKV_TYPES", "round_f16_",
           "attn_gproj", "attn_gproj_supported", "attn_oproj_fix", "attn_oproj_supported", "fix_acc",
           "repack_oproj", "oproj_eligible", "qgemv_fix_norm_silu", "qgemv_norm_argmax", "dequantize_weight_f16",
           "repack_down_slices", "down_slice_eligible", "ffn_fix", "ffn_fix_supported", "ffn_fix_bound",
           "kv16_blocks", "flash_prefill_blocks", "flash_prefill_blocks_workspace",
           "fix_acc_block", "fix_stride", "qkv_fix_rmsnorm_rope", "FFN_REPLICAS",
           "DecodeStep", "decode_step_supported", "decode_step_workspace",
           "gemm_f16", "gemm_f16_silu", "interleave_gate_up_f16", "flash_prefill",
           "BLOCK_SIZE"]
