"""GGML block types, sizes and dequantization (the reference's dequant.py surface).

``GGML_*`` ids and ``nbytes_for`` restate dequant.py:15-48 (pure arithmetic). ``dequantize``
keeps the reference signature (dequant.py:243-260: raw bytes -> float32 numpy array) but runs
the bit-exact HIP kernel ``pe_dequant`` on the GPU; ``dequantize_device`` returns the result as
a device tensor without the copy back. The reference's load-time ``unpack_*`` int8+scale forms
(dequant.py:79-168) have no counterpart: the kernels read the GGUF blocks themselves (tiled by
``pe_repack``, see kernels.QWeight).
"""

from __future__ import annotations

import numpy as np

GGML_F32 = 0
GGML_F16 = 1
GGML_Q5_0 = 6
GGML_Q8_0 = 8
GGML_Q4_K = 12
GGML_Q5_K = 13
GGML_Q6_K = 14
GGML_Q8_K = 15

TYPE_NAMES = {GGML_F32: "F32", GGML_F16: "F16", GGML_Q5_0: "Q5_0", GGML_Q8_0: "Q8_0",
              GGML_Q4_K: "Q4_K", GGML_Q6_K: "Q6_K", GGML_Q8_K: "Q8_K"}

# elements per block, bytes per block
BLOCK_SIZE = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_Q5_0: (32, 22), GGML_Q8_0: (32, 34),
              GGML_Q4_K: (256, 144), GGML_Q6_K: (256, 210), GGML_Q8_K: (256, 292)}

# the quantized formats the GEMV kernels read
QUANT_TYPES = (GGML_Q5_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K)
# every matrix format the GEMV / GEMM / QKV kernels read (F16 and F32 rows as stored)
MATRIX_TYPES = QUANT_TYPES + (GGML_F16, GGML_F32)


def nbytes_for(ggml_type: int, n: int) -> int:
    """Bytes ``n`` elements of ``ggml_type`` occupy in the data section (dequant.py:27-48)."""
    if ggml_type not in BLOCK_SIZE:
        raise NotImplementedError(f"ggml type {ggml_type} not supported")
    qk, size = BLOCK_SIZE[ggml_type]
    assert n % qk == 0, f"{TYPE_NAMES[ggml_type]} needs n%{qk}==0, got {n}"
    return (n // qk) * size


def dequantize_device(ggml_type: int, raw, n: int, device="cuda"):
    """Dequantize ``n`` elements of raw GGUF bytes on the GPU -> float32 device tensor."""
    import torch
    from . import kernels
    if isinstance(raw, torch.Tensor):
        blocks = raw.to(device=device, dtype=torch.uint8)
    else:
        blocks = torch.from_numpy(np.frombuffer(raw, dtype=np.uint8).copy()).to(device)
    return kernels.dequantize(ggml_type, blocks, n)


def dequantize(ggml_type: int, raw: bytes, n: int) -> np.ndarray:
    """Dequantize ``n`` elements of ``raw`` into a float32 numpy array (dequant.py:243-260).

    Runs on the GPU (``pe_dequant``); raises if no GPU or no built library is present.
    """
    nbytes_for(ggml_type, n)
    return dequantize_device(ggml_type, raw, n).cpu().numpy()
