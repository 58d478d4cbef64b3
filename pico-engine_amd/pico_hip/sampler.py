"""Token sampling over logits (the reference's sampler.py surface, sampler.py:8-27).

Greedy (temperature <= 0) is ``argmax`` (first maximum on ties) followed by one device-to-host
read; otherwise temperature scaling, optional top-k and top-p filtering and a multinomial
draw, all as torch ops on the logits' device.
"""

from __future__ import annotations

import torch


def sample(logits: torch.Tensor, temperature: float = 1.0, top_k: int = 0, top_p: float = 1.0,
           generator: torch.Generator | None = None) -> int:
    """Draw one token id from 1-D raw ``logits``."""
    if temperature <= 0:
        return int(torch.argmax(logits).item())
    z = logits.float() / temperature
    if top_k > 0:
        kth = torch.topk(z, min(top_k, z.numel())).values[-1]
        z = torch.where(z < kth, torch.full_like(z, float("-inf")), z)
    if top_p < 1.0:
        order = torch.argsort(z, descending=True)
        probs = torch.softmax(z[order], dim=-1)
        cut = torch.cumsum(probs, dim=-1) > top_p
        cut = torch.cat([cut.new_zeros(1), cut[:-1]])  # keep the token that crosses top_p
        z = z.clone()
        z[order[cut]] = float("-inf")
    probs = torch.softmax(z, dim=-1)
    return int(torch.multinomial(probs, 1, generator=generator).item())
