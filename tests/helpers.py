"""Test helpers: seeded quantized weights and error metrics."""

from __future__ import annotations

import numpy as np

from oracle import dequant as dq

F16_FIELDS = {dq.Q8_0: [0], dq.Q5_0: [0], dq.Q4_K: [0, 2], dq.Q6_K: [208]}


def random_quant(t: int, n_rows: int, k: int, seed: int, subnormal_frac: float = 0.02) -> bytes:
    """Random GGUF blocks: random code/scale bytes (every code value occurs) with the fp16
    scale fields replaced by seeded N(0, 0.01) values, a few of them fp16-subnormal."""
    qk, size = dq.BLOCK[t]
    nblk = n_rows * k // qk
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(nblk, size), dtype=np.uint8)
    for off in F16_FIELDS[t]:
        d = (rng.standard_normal(nblk) * 0.01).astype(np.float16)
        sub = rng.random(nblk) < subnormal_frac
        d[sub] = (rng.integers(1, 1024, size=int(sub.sum())).astype(np.uint16)).view(np.float16)
        raw[:, off:off + 2] = d.view(np.uint8).reshape(-1, 2)
    return raw.reshape(-1).tobytes()


def quantized_normal(t: int, n_rows: int, k: int, seed: int, std: float = 0.02) -> bytes:
    """N(0, std) weights through the host quantizer (the synthetic-model path)."""
    from pico_hip.quantize import quantize
    rng = np.random.default_rng(seed)
    return quantize(t, (rng.standard_normal(n_rows * k) * std).astype(np.float32)).tobytes()


def dequant_rows(t: int, raw: bytes, n_rows: int, k: int) -> np.ndarray:
    return dq.dequantize(t, raw, n_rows * k).reshape(n_rows, k)


def rel_err(got, ref) -> float:
    """max |got - ref| / max |ref| (the 1e-3 relative criterion)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30))
