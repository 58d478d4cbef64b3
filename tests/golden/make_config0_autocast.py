"""Writes config0_autocast_logits.json: the oracle's (oracle/ref_cpu.py) prefill logits of the
config-0 prompt under the reference's CUDA fp16 autocast numerics (model.py:147-151) and in
fp32, at the 2048 indices of the largest autocast logits and 2048 seeded random others.

    python tests/golden/make_config0_autocast.py   (about a minute on the CPU)
"""
import json
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "pico-engine_amd")]

from oracle.ref_cpu import RefModel  # noqa: E402
from pico_hip import synth  # noqa: E402

HERE = Path(__file__).resolve().parent
fx = json.loads((HERE / "config0_greedy.json").read_text())
gguf = synth.cached(synth.ARCHES["qwen2.5-0.5b"], seed=fx["seed"], cache_dir="/tmp/pico_hip_models")
assert synth.sha256(gguf) == fx["gguf_sha256"]
ref = RefModel(gguf)
ids = fx["prompt_ids"]
pos = torch.arange(len(ids))
ac = ref.forward(torch.tensor(ids), pos, ref.empty_cache(len(ids)), autocast=True).numpy()
f32 = ref.forward(torch.tensor(ids), pos, ref.empty_cache(len(ids))).numpy()
top = np.argsort(-ac, kind="stable")[:2048]
rest = np.setdiff1d(np.arange(ac.size), top)
sample = np.random.default_rng(0).choice(rest, 2048, replace=False)
idx = np.concatenate([top, np.sort(sample)])
out = {
    "gguf_sha256": fx["gguf_sha256"], "prompt_ids": ids,
    "idx": idx.tolist(), "autocast": ac[idx].tolist(), "fp32": f32[idx].tolist(),
    "max_abs_autocast": float(np.abs(ac).max()), "argmax_autocast": int(ac.argmax()),
    "argmax_fp32": int(f32.argmax()),
}
(HERE / "config0_autocast_logits.json").write_text(json.dumps(out))
print("wrote", len(idx), "logits; fp32 vs autocast max diff / max",
      float(np.abs(ac - f32).max() / np.abs(ac).max()))
