"""Writes tests/golden/config0_greedy.json: the oracle's greedy tokens on BASELINE config 0.

Config 0: Qwen2.5-0.5B-architecture synthetic GGUF (pico_hip.synth, seed 0, Q4_K_M-style mix),
a 13-token prompt of uniform random ids in [0, 151936) from numpy default_rng(1234), fp32
prefill, 64 greedy decode steps. The tokens come from oracle/ref_cpu.py (the torch-CPU
restatement of the reference forward, with its fp16 attention-output rounding); per-step
top-1/top-2 logit margins are recorded so a mismatch can be judged against them.

Run:  python tests/golden/make_config0_greedy.py [model_dir]   (a few minutes on 8 cores)
"""

from __future__ import annotations

import json
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "pico-engine_amd")]

import numpy as np  # noqa: E402
import torch  # noqa: E402

from oracle.ref_cpu import RefModel  # noqa: E402
from pico_hip import synth  # noqa: E402

SEED, PROMPT_SEED, N_PROMPT, N_TOKENS = 0, 1234, 13, 64


def main() -> None:
    model_dir = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/tmp/pico_hip_models")
    model_dir.mkdir(parents=True, exist_ok=True)
    arch = synth.ARCHES["qwen2.5-0.5b"]
    t0 = time.time()
    path = synth.cached(arch, seed=SEED, cache_dir=model_dir)
    sha = synth.sha256(path)
    print(f"model {path} sha256 {sha} ({time.time() - t0:.1f}s)", flush=True)
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, arch.vocab, size=N_PROMPT).tolist()
    torch.set_num_threads(8)
    ref = RefModel(path)
    t0 = time.time()
    tokens, margins = ref.greedy(prompt, N_TOKENS)
    print(f"greedy {N_TOKENS} tokens in {time.time() - t0:.1f}s; min margin {min(margins):.3e}", flush=True)
    out = {"config": "BASELINE config 0", "arch": arch.name, "seed": SEED, "prompt_seed": PROMPT_SEED,
           "gguf_sha256": sha, "prompt_ids": prompt, "n_tokens": N_TOKENS, "tokens": tokens,
           "margins": margins, "generator": "oracle/ref_cpu.py RefModel.greedy"}
    dst = Path(__file__).with_name("config0_greedy.json")
    dst.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {dst}")


if __name__ == "__main__":
    main()
