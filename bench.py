#!/usr/bin/env python
"""Batch-1 decode benchmark of BASELINE config 0 on one MI355X.

Workload: Qwen2.5-0.5B-architecture decoder, random-init N(0,0.02)
weights quantized into a Q4_K_M-style GGUF (seed 0, pico_hip.synth), a 13-token prompt of
uniform random ids (numpy default_rng(1234)), fp32 prefill, greedy decode. A "step" is one
decode token: one replay of the HIP graph holding the whole per-token forward, ending with
the greedy pick made on the device (the reference loop's argmax, evidence.py:117-123); the
host reads the picked ids once per chunk of replays.
W warm-up runs (fresh cache, graph capture, prefill, K decode steps) precede the timed run;
in the timed run the prefill happens before the bracket, then K decode steps are timed
between two device synchronizations. value = K / elapsed (tok/s).

Also reported on the same line:
  kernels       every kernel of the decode step timed alone with HIP events on the stream it
                launches on (one HIP graph of back-to-back launches rotating >= 1 GiB of
                distinct weight copies, so the 256 MB Infinity Cache cannot serve repeats,
                replayed): average launch time, launches per token, time per token,
                achieved = algorithmic bytes per launch / average launch time, against 8 TB/s;
                traffic from the rocprofv3 --pmc summary in profiles/ when present.
  roofline      the entry of `kernels` with the largest time per token (--kernel picks
                another).
  decode_roofline  weight + KV bytes per token over the measured time per token.
  cpu_baseline  the torch-CPU restatement of the reference forward (oracle/ref_cpu.py) on the
                same model and prompt, on this host's cores, over a bounded number of decode
                steps (about 10-30 s).
  config3, config4  the long-context (8192-token matrix-core prefill, decode at 8192) and the
                7B-architecture runs below, on the same line (--no-extra-configs skips them).
Usage: python bench.py [--steps 64] [--warmup 2] [--kernel gate_up|lm_head|down_q6k|...]
       python bench.py --micro   (configs 1 and 2: GEMV shapes, decode attention, QKV kernel)
       python bench.py --micro --config 4   (the decode kernels at the 7B shapes)
       python bench.py --config 3   (8192-token prefill on the matrix cores, decode at 8192)
       python bench.py --config 4   (the 7B-architecture model: 128-token prompt, 256 decode steps)
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT), str(ROOT / "pico-engine_amd")]

PEAK_HBM_GBPS = 8000.0
PROMPT_SEED, MODEL_SEED, N_PROMPT = 1234, 0, 13


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def run_decode(eng, prompt, steps, timed: bool):
    """One evidence._run_once-style run (evidence.py:96-135): fresh cache + graph, prefill
    (timed on its own), then `steps` greedy tokens (timed), stopping early only at eos. The
    greedy pick is made on the device at the end of every step, so the replays go back to
    back; the host reads the picks once per chunk of replays."""
    import torch
    cache = eng._empty_cache(len(prompt) + steps)
    graph = eng._build_decode_graph(cache)
    if graph is None:
        raise RuntimeError("HIP graph capture failed")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    eng.prefill_greedy(prompt, cache)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = eng.decode_greedy(graph, steps, eng.tok.eos_id)
    torch.cuda.synchronize()
    return time.perf_counter() - t0, prefill_s, out


def kernel_launchers(eng, which: str, attn: tuple[int, int] = (45, 80)):
    """-> (list of launch closures over distinct weight copies, algorithmic bytes per launch,
    kernel name). Copies are made until >= 1 GiB of distinct weights rotate. ``attn`` = (valid
    positions, cache capacity) of the attention kernels."""
    import torch
    from pico_hip import kernels as K
    m, cfg = eng.model, eng.cfg
    L0 = m.layers[0]
    XU, YU = K.LAYOUT_X_UT, K.LAYOUT_Y_UT
    tn = lambda w: K.TYPE_NAMES.get(w.ggml_type, w.ggml_type)
    kn = lambda w: "k_mgemv" if K.use_mfma_gemv and w.mfma is not None else "k_qgemv"
    hd, nh, nkv, h = cfg.head_dim, cfg.n_head, cfg.n_kv_head, cfg.hidden
    # the decode step's own launch configuration: activations in the unit-transposed layout
    x = torch.randn(h, device=eng.device)
    if which == "gate_up":
        # as the decode step runs it: x plus the attention block's n_kv o-projection parts,
        # RMSNorm, [gate; up] pair, SiLU; the sum is stored for the next residual
        ws = (L0.w_gate_up,)
        parts = torch.randn(nkv, h, device=eng.device) * 0.1
        name = (f"k_qgemv (Q5_0, x + {nkv} o-proj parts, rmsnorm+SiLU pair) gate/up "
                f"{h}->2x{cfg.ffn_dim}")
        fn = lambda w: K.qgemv_sum_norm_silu(x, parts, L0.ffn_norm_ut, w, cfg.eps, layout=XU | YU)
        io = 4 * (h * (3 + nkv) + cfg.ffn_dim)
    elif which == "gate_up_fix":
        # as the decode step runs it after attn_oproj_fix: x plus 2^-32 times the fixed-point
        # o-projection accumulator, RMSNorm, [gate; up] pair, SiLU; the sum is stored
        ws = (L0.w_gate_up,)
        fix = K.fix_acc(h, eng.device)[0]
        fix[:h] = (torch.randn(h, device=eng.device, dtype=torch.float64) * 0.1 * 2.0 ** 32).to(torch.int64)
        name = (f"k_qgemv (Q5_0, x + 2^-32 o-proj acc, rmsnorm+SiLU pair) gate/up "
                f"{h}->2x{cfg.ffn_dim}")
        fn = lambda w: K.qgemv_fix_norm_silu(x, fix, L0.ffn_norm_ut, w, cfg.eps, layout=XU | YU)
        io = 4 * (h * 3 + cfg.ffn_dim) + 8 * (h + 1)
    elif which == "gate_up_norm":
        # the decode step without attn_gproj (head_dim 128: the 7B): RMSNorm, [gate; up], SiLU
        ws = (L0.w_gate_up,)
        name = f"{kn(ws[0])} ({tn(ws[0])}, rmsnorm+SiLU pair) gate/up {h}->2x{cfg.ffn_dim}"
        fn = lambda w: K.qgemv_norm_silu(x, L0.ffn_norm_ut, w, cfg.eps, layout=XU | YU)
        io = 4 * (h * 2 + cfg.ffn_dim)
    elif which == "lm_head":
        ws = (m.output,)
        name = f"k_qgemv ({tn(ws[0])}, rmsnorm, device greedy pick) LM head {h}->{cfg.vocab_size}"
        g = K.GreedyState(m.output.n, 1, eng.device)
        fn = lambda w: K.qgemv_norm_argmax(x, m.output_norm_ut, w, cfg.eps, g, layout=XU)
        io = 4 * (h * 2 + cfg.vocab_size)
    elif which in ("down_q6k", "down_q4k"):
        from pico_hip.dequant import GGML_Q4_K, GGML_Q6_K
        want = GGML_Q6_K if which == "down_q6k" else GGML_Q4_K
        li = next((i for i, Lr in enumerate(m.layers) if Lr.w_down.ggml_type == want), 0)
        ws = (m.layers[li].w_down,)
        name = f"{kn(ws[0])} ({tn(ws[0])}, +residual) ffn_down {cfg.ffn_dim}->{h}"
        a = torch.randn(cfg.ffn_dim, device=eng.device)
        fn = lambda w: K.qgemv(a, w, residual=x, layout=XU | YU)
        io = 4 * (cfg.ffn_dim + 2 * h)
    elif which == "qkv":
        # RMSNorm, [Wq; Wk; Wv] + bias, RoPE, K/V row written into the cache at position 40
        ws = (L0.wq, L0.wk, L0.wv)
        cap = 64
        kc = torch.zeros(nkv, cap, hd, device=eng.device)
        vc = torch.zeros(nkv, cap, hd, device=eng.device)
        pos = torch.tensor([40], device=eng.device)
        name = (f"{'k_mqkv' if K.mqkv_ok(*ws) else 'k_qkv'} ({'/'.join(tn(w) for w in ws)}, rmsnorm, bias, RoPE, "
                f"cache write) {h}->{nh}x{hd}+2x{nkv}x{hd}")
        fn = lambda wq, wk, wv: K.qkv_rmsnorm_rope(x, L0.attn_norm_ut, cfg.eps, wq, wk, wv, L0.bq, L0.bk,
                                                   L0.bv, m.cos, m.sin, pos, kc, vc, nh, layout=XU)
        io = 4 * (2 * h + (nh + 2 * nkv) * hd + hd + nh * hd + 2 * nkv * hd)
    elif which == "qkv_fix":
        # the staged form over x + the four down-product replicas of the previous layer's
        # fused FFN (every layer but the first); stores the summed vector
        ws = (L0.wq, L0.wk, L0.wv)
        cap = 64
        kc = torch.zeros(nkv, cap, hd, device=eng.device)
        vc = torch.zeros(nkv, cap, hd, device=eng.device)
        pos = torch.tensor([40], device=eng.device)
        acc4 = torch.zeros(K.FFN_REPLICAS, K.fix_stride(h), device=eng.device, dtype=torch.int64)
        acc4[:, :h] = (torch.randn(K.FFN_REPLICAS, h, device=eng.device, dtype=torch.float64)
                       * 0.1 * 2.0 ** 32).to(torch.int64)
        name = (f"k_qkv_fix ({'/'.join(tn(w) for w in ws)}, x + 2^-32 sum of 4 replicas, rmsnorm, bias, "
                f"RoPE, cache write) {h}->{nh}x{hd}+2x{nkv}x{hd}")
        fn = lambda wq, wk, wv: K.qkv_fix_rmsnorm_rope(x, acc4, L0.attn_norm_ut, cfg.eps, wq, wk, wv, L0.bq,
                                                       L0.bk, L0.bv, m.cos, m.sin, pos, kc, vc, nh,
                                                       layout=XU)
        io = (4 * (3 * h + (nh + 2 * nkv) * hd + hd + nh * hd + 2 * nkv * hd) +
              8 * K.FFN_REPLICAS * (h + 1))
    elif which in ("ffn_fix_q6k", "ffn_fix_q4k"):
        # the fused FFN as the decode step runs it: x + 2^-32 o-projection accumulator,
        # RMSNorm, [gate; up], SiLU, and ffn_down's column slices added into the four
        # fixed-point replicas the next layer's QKV launch reads
        from pico_hip.dequant import GGML_Q4_K, GGML_Q6_K
        want = GGML_Q6_K if which == "ffn_fix_q6k" else GGML_Q4_K
        li = next((i for i, Lr in enumerate(m.layers[:-1]) if Lr.w_down.ggml_type == want), 0)
        Lr = m.layers[li]
        ws = (Lr.w_gate_up, Lr.w_down)
        fix = K.fix_acc(h, eng.device)[0]
        fix[:h] = (torch.randn(h, device=eng.device, dtype=torch.float64) * 0.1 * 2.0 ** 32).to(torch.int64)
        acc4 = torch.zeros(K.FFN_REPLICAS, K.fix_stride(h), device=eng.device, dtype=torch.int64)
        name = (f"k_ffn_fix ({tn(ws[0])} gate/up, {tn(ws[1])} ffn_down slices, x + 2^-32 o-proj acc, "
                f"rmsnorm, SiLU, 4 fixed-point replicas) {h}->2x{cfg.ffn_dim}->{h}")
        fn = lambda wgu, wd: K.ffn_fix(x, fix, Lr.ffn_norm_ut, wgu, wd, cfg.eps, acc4, layout=XU | YU)
        io = 4 * 3 * h + 8 * (h + 1) + 8 * K.FFN_REPLICAS * (h + 1)
    elif which == "attn_gproj":
        # attention over S cached positions (config 0: 45, the mean context of a 13-token
        # prompt and 64 decode steps) times each kv group's columns of Wo
        ws = (L0.wo,)
        S, cap = attn
        q = torch.randn(nh, hd, device=eng.device)
        kc = torch.randn(nkv, cap, hd, device=eng.device)
        vc = torch.randn(nkv, cap, hd, device=eng.device)
        name = f"k_attn_gproj ({tn(ws[0])} o-proj, S={S}, {nh}/{nkv} heads) {nh * hd}->{nkv}x{h}"
        fn = lambda w: K.attn_gproj(q, kc, vc, w, S=S, layout=YU)
        io = 4 * (nh * hd + 2 * nkv * S * hd + nkv * h)
    elif which == "attn_oproj":
        # attention of every query head over S cached positions (config 0: 45, the mean
        # context of a 13-token prompt and 64 decode steps) times its columns of Wo, added into
        # the fixed-point accumulator (read and written once per row, n_head atomic adds)
        ws = (L0.wo,)
        S, cap = attn
        q = torch.randn(nh, hd, device=eng.device)
        kc = torch.randn(nkv, cap, hd, device=eng.device)
        vc = torch.randn(nkv, cap, hd, device=eng.device)
        pos = torch.tensor([S - 1], device=eng.device)
        acc = K.fix_acc(h, eng.device)[0]
        name = f"k_attn_oproj ({tn(ws[0])} o-proj, S={S}, {nh}/{nkv} heads) {nh * hd}->{h}"
        fn = lambda w: K.attn_oproj_fix(q, kc, vc, w, pos, acc, layout=YU)
        io = 4 * (nh * hd + 2 * nkv * S * hd) + 16 * (h + 1)
    elif which == "attn":
        # decode attention alone (head_dim 128: the 7B), S valid positions of the cache; its
        # K/V copies rotate instead of weights
        S, cap = attn
        q = torch.randn(nh, hd, device=eng.device)
        kvb = 2 * nkv * cap * hd * 4
        kvs = [(torch.randn(nkv, cap, hd, device=eng.device), torch.randn(nkv, cap, hd, device=eng.device))
               for _ in range(max(2, -(-(1 << 30) // kvb)))]
        wsp = K.decode_attn_workspace(nh, nkv, hd, cap, eng.device)
        Sd = torch.tensor([S], device=eng.device)
        name = f"decode_attn (S={S} of {cap}, {nh}/{nkv} heads, hd {hd})"
        fns = [(lambda kv=kv: K.decode_attn(q, kv[0], kv[1], S=Sd, workspace=wsp, layout=YU)) for kv in kvs]
        return fns, 2 * nkv * S * hd * 4 + 4 * 2 * nh * hd, name
    elif which == "oproj":
        # the o-projection with the residual where attn_gproj does not apply (head_dim 128)
        ws = (L0.wo,)
        a = torch.randn(nh * hd, device=eng.device)
        name = f"{kn(ws[0])} ({tn(ws[0])}, +residual) o-proj {nh * hd}->{h}"
        fn = lambda w: K.qgemv(a, w, residual=x, layout=XU | YU)
        io = 4 * (nh * hd + 2 * h)
    else:
        raise SystemExit(f"unknown --kernel {which}")
    nbytes = sum(w.nbytes for w in ws)
    copies = max(1, -(-(1 << 30) // nbytes))
    sets = [ws] + [tuple(w.copy() for w in ws) for _ in range(copies - 1)]
    return [(lambda st=st: fn(*st)) for st in sets], nbytes + io, name


def decode_kernels(eng, capacity: int) -> list[tuple[str, int]]:
    """(kernel_launchers key, launches per decode token) for the kernels of the model's decode
    step with a cache of ``capacity`` positions: every per-layer launch and the LM head (the
    embedding row, the greedy pick and the fixed-point accumulator fill, a few us each, are
    left out)."""
    from pico_hip import kernels as K
    from pico_hip.dequant import GGML_Q4_K, GGML_Q6_K
    m, cfg = eng.model, eng.cfg
    n = cfg.n_layers
    L0 = m.layers[0]
    gproj = (m.use_attn_gproj and L0.w_gate_up is not None and
             K.attn_gproj_supported(cfg.n_head, cfg.n_kv_head, cfg.head_dim, capacity, L0.wo))
    rows = [("qkv", n)]
    if m.ffn_fix_ok(capacity):
        # three launches per layer: qkv (first layer) / qkv_fix, attn_oproj, ffn_fix (the last
        # layer: gate_up_fix and its ffn_down)
        rows = [("qkv", 1), ("qkv_fix", n - 1), ("attn_oproj", n)]
        for key, t in (("ffn_fix_q6k", GGML_Q6_K), ("ffn_fix_q4k", GGML_Q4_K)):
            c = sum(1 for Lr in m.layers[:-1] if Lr.w_down.ggml_type == t)
            if c:
                rows.append((key, c))
        rows.append(("gate_up_fix", 1))
        rows.append(("down_q6k" if m.layers[-1].w_down.ggml_type == GGML_Q6_K else "down_q4k", 1))
        rows.append(("lm_head", 1))
        return rows
    if m.attn_oproj_ok(capacity):
        rows += [("attn_oproj", n), ("gate_up_fix", n)]
    elif gproj:
        rows += [("attn_gproj", n), ("gate_up", n)]
    else:
        rows += [("attn", n), ("oproj", n), ("gate_up_norm", n)]
    for key, t in (("down_q6k", GGML_Q6_K), ("down_q4k", GGML_Q4_K)):
        c = sum(1 for Lr in m.layers if Lr.w_down.ggml_type == t)
        if c:
            rows.append((key, c))
    rows.append(("lm_head", 1))
    return rows


def kernel_table(eng, iters: int, config: int, attn: tuple[int, int] = (45, 80)) -> list[dict]:
    """Each decode kernel timed alone (time_kernel), with its time per token; ``attn`` = (valid
    positions, cache capacity) of the attention launches (config 0: the mean context of the
    64-step run, 13 + 32.5)."""
    import torch
    out = []
    for key, per_token in decode_kernels(eng, attn[1]):
        launchers, alg_bytes, kname = kernel_launchers(eng, key, attn)
        avg_us = time_kernel(launchers, iters)
        del launchers
        torch.cuda.empty_cache()
        achieved = alg_bytes / (avg_us * 1e-6) / 1e9
        log(f"{kname}: {avg_us:.2f} us/launch x {per_token}/token, {achieved:.0f} GB/s")
        out.append({"key": key, "kernel": kname, "launches_per_token": per_token,
                    "avg_launch_us": round(avg_us, 3), "us_per_token": round(avg_us * per_token, 2),
                    "algorithmic_bytes": int(alg_bytes), "achieved": round(achieved, 1),
                    "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBPS, 4),
                    "traffic": traffic_from_profiles(key, config)})
    return out


def kernel_groups(table: list[dict]) -> list[dict]:
    """The table with the entries of one kernel over several weight formats (keys differing only
    in a _q6k / _q4k suffix: the alternating ffn_down formats) merged: launches and time per
    token added, bytes per launch and launch time averaged over the launches, achieved = mean
    bytes / mean time, traffic the launch-weighted mean when every entry has one."""
    groups: dict[str, list[dict]] = {}
    for r in table:
        k = r["key"]
        base = k[:-4] if k.endswith(("_q6k", "_q4k")) else k
        groups.setdefault(base, []).append(r)
    out = []
    for base, rows in groups.items():
        if len(rows) == 1:
            out.append(rows[0])
            continue
        n = sum(r["launches_per_token"] for r in rows)
        us = sum(r["us_per_token"] for r in rows)
        alg = sum(r["algorithmic_bytes"] * r["launches_per_token"] for r in rows) / n
        avg = us / n
        traffic = (None if any(r["traffic"] is None for r in rows) else
                   int(sum(r["traffic"] * r["launches_per_token"] for r in rows) / n))
        achieved = alg / (avg * 1e-6) / 1e9
        out.append({"key": base, "kernel": " | ".join(r["kernel"] for r in rows), "launches_per_token": n,
                    "avg_launch_us": round(avg, 3), "us_per_token": round(us, 2),
                    "algorithmic_bytes": int(alg), "achieved": round(achieved, 1), "peak": PEAK_HBM_GBPS,
                    "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBPS, 4), "traffic": traffic})
    return out


def roofline_of(table: list[dict], key: str | None) -> dict:
    """The roofline object: the table entry ``key``, or the kernel with the largest time per
    token (its weight-format instantiations together, kernel_groups)."""
    row = next((r for r in table if r["key"] == key), None) if key else None
    if row is None:
        row = max(kernel_groups(table), key=lambda r: r["us_per_token"])
    return {"bound": "hbm", "kernel": row["kernel"], "achieved": row["achieved"], "peak": row["peak"],
            "unit": row["unit"], "frac": row["frac"], "traffic": row["traffic"],
            "avg_launch_us": row["avg_launch_us"], "algorithmic_bytes": row["algorithmic_bytes"],
            "launches_per_token": row["launches_per_token"], "us_per_token": row["us_per_token"],
            "selected_as": "requested by --kernel" if key and row["key"] == key else
                           "largest time per decode token of the kernels timed (weight formats of one kernel together)"}


def kernel_only(eng, args) -> None:
    """--kernel-only: time --kernel alone (launches one by one, as rocprofv3 --pmc counts
    them), then four copies of a 1 GiB buffer: the counter calibration (each reads and writes
    exactly 1 GiB)."""
    import torch
    if not args.kernel:
        raise SystemExit("--kernel-only needs --kernel")
    launchers, alg_bytes, kname = kernel_launchers(eng, args.kernel)
    avg_us = time_kernel(launchers, args.kernel_iters, graph=False)
    src = torch.ones(1 << 28, device=eng.device)
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"kernel": kname, "avg_launch_us": avg_us, "algorithmic_bytes": alg_bytes,
                      "calibration_copy_bytes": src.numel() * 4}), flush=True)


def time_kernel(launchers, iters: int, graph: bool = True) -> float:
    """Average launch duration in us, from HIP events on torch's current stream (the stream
    the kernels launch on). With ``graph`` the launches over the distinct copies are captured
    once into a HIP graph and replayed, so the figure is the kernel's own back-to-back time
    (as in the decode step's graph) rather than the host's per-launch overhead; without it
    the launches are made one by one (used for the rocprofv3 counter runs)."""
    import torch
    for f in launchers:
        f()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if not graph:
        e0.record()
        for i in range(iters):
            launchers[i % len(launchers)]()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / iters
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.inference_mode(), torch.cuda.graph(g, stream=s):   # as the engine captures
        for f in launchers:
            f()
    torch.cuda.current_stream().wait_stream(s)
    g.replay()
    torch.cuda.synchronize()
    reps = max(1, -(-iters // len(launchers)))
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) * 1000.0 / (reps * len(launchers))


def micro(device: str) -> None:
    """BASELINE configs 1 and 2 as kernel microbenchmarks, one JSON line per case: every valid
    GEMV format x shape (config 1: x ~ N(0,1), W ~ N(0,0.02) quantized), decode attention at
    L = 512, 4096, 32768 positions (config 2: fp32 K/V ~ N(0,1), 14/2 heads, hd 64) and the
    fused RMSNorm + QKV + bias + RoPE kernel. Each launch is timed in a graph of back-to-back
    launches over >= 1 GiB of distinct weight / KV copies; GB/s = algorithmic bytes / time."""
    import numpy as np
    import torch
    from pico_hip import kernels as K
    from pico_hip.quantize import quantize
    Q8_0, Q5_0, Q4_K, Q6_K = 8, 6, 12, 14
    name = {Q8_0: "Q8_0", Q5_0: "Q5_0", Q4_K: "Q4_K", Q6_K: "Q6_K"}

    def qweight(t, n, k, seed):
        rng = np.random.default_rng(seed)
        raw = quantize(t, (rng.standard_normal(n * k) * 0.02).astype(np.float32)).tobytes()
        return K.pack_weight(torch.from_numpy(np.frombuffer(raw, np.uint8).copy()).to(device), t, n, k)

    def copies(make, nbytes):
        return [make() for _ in range(max(2, min(4096, -(-(1 << 30) // nbytes))))]

    def emit(case, us, nbytes, **extra):
        gbps = nbytes / (us * 1e3)
        print(json.dumps({"micro": case, "us_per_launch": round(us, 3), "algorithmic_bytes": int(nbytes),
                          "achieved_gbps": round(gbps, 1), "frac": round(gbps / PEAK_HBM_GBPS, 4), **extra}),
              flush=True)

    shapes = [(t, k, n) for t in (Q5_0, Q8_0) for (k, n) in ((896, 1152), (896, 896), (896, 9728),
                                                             (4864, 896), (896, 151936))]
    shapes += [(Q4_K, 4864, 896), (Q6_K, 4864, 896)]
    for i, (t, k, n) in enumerate(shapes):
        w0 = qweight(t, n, k, 100 + i)
        ws = [w0] + [w0.copy() for _ in range(len(copies(lambda: 0, w0.nbytes)) - 1)]
        x = torch.randn(k, device=device)
        res = torch.randn(n, device=device)
        nbytes = w0.nbytes + 4 * (k + 2 * n)
        us = time_kernel([(lambda ww=ww: K.qgemv(x, ww, residual=res)) for ww in ws], 400)
        emit("config1_gemv", us, nbytes, format=name[t], shape=f"{k}->{n}", residual=True)
        del ws
    nh, nkv, hd = 14, 2, 64
    q = torch.randn(nh, hd, device=device)
    for L in (512, 4096, 32768):
        kvb = 2 * nkv * L * hd * 4
        kvs = copies(lambda: (torch.randn(nkv, L, hd, device=device), torch.randn(nkv, L, hd, device=device)), kvb)
        wsp = K.decode_attn_workspace(nh, nkv, hd, L, device)
        S = torch.tensor([L], device=device)
        us = time_kernel([(lambda kv=kv: K.decode_attn(q, kv[0], kv[1], S=S, workspace=wsp)) for kv in kvs], 200)
        emit("config2_decode_attn", us, kvb + 4 * 2 * nh * hd, positions=L, heads=f"{nh}/{nkv}", head_dim=hd)
        del kvs
    h = 896
    wq, wk, wv = qweight(Q5_0, nh * hd, h, 1), qweight(Q5_0, nkv * hd, h, 2), qweight(Q8_0, nkv * hd, h, 3)
    qkv_bytes = wq.nbytes + wk.nbytes + wv.nbytes
    trip = [(wq, wk, wv)] + [tuple(w.copy() for w in (wq, wk, wv))
                             for _ in range(len(copies(lambda: 0, qkv_bytes)) - 1)]
    x = K.to_ut(torch.randn(h, device=device))
    nw = K.to_ut(torch.ones(h, device=device))
    bq, bk, bv = (torch.randn(m * hd, device=device) for m in (nh, nkv, nkv))
    cos = torch.randn(4096, hd // 2, device=device)
    sin = torch.randn(4096, hd // 2, device=device)
    pos = torch.tensor([60], device=device)
    kc = torch.zeros(nkv, 77, hd, device=device)
    vc = torch.zeros_like(kc)
    us = time_kernel([(lambda tr=tr: K.qkv_rmsnorm_rope(x, nw, 1e-6, *tr, bq, bk, bv, cos, sin, pos, kc, vc, nh,
                                                        layout=K.LAYOUT_X_UT)) for tr in trip], 400)
    emit("config2_qkv_rmsnorm_rope", us, qkv_bytes + 4 * (3 * h + 2 * (nh + 2 * nkv) * hd),
         shape="896->14x64 + 2x2x64, Q5_0/Q5_0/Q8_0")


def micro7b(device: str) -> None:
    """The decode kernels at the 7B shapes, one JSON line each: o-proj
    Q4_K 3584->3584 + residual, RMSNorm + [gate; up] Q4_K 3584->2x18944 + SiLU, ffn_down Q6_K
    18944->3584 + residual, the fused RMSNorm + QKV (Q4_K/Q4_K/Q6_K) + RoPE, and decode attention
    (28/4 heads, hd 128) at 384 and 4096 positions. Weights N(0,0.02) drawn and quantized on the
    GPU; timing as in --micro (graphs over >= 1 GiB of distinct copies)."""
    import torch
    from pico_hip import kernels as K
    from pico_hip.quantize import quantize_torch
    Q8_0, Q4_K, Q6_K = 8, 12, 14
    gen = torch.Generator(device=device)
    gen.manual_seed(7)

    def qweight(t, n, k):
        w = torch.randn(n * k, generator=gen, device=device) * 0.02
        return K.pack_weight(quantize_torch(t, w), t, n, k)

    def ncopies(nbytes):
        return max(2, min(4096, -(-(1 << 30) // nbytes)))

    def emit(case, us, nbytes, **extra):
        gbps = nbytes / (us * 1e3)
        print(json.dumps({"micro": case, "us_per_launch": round(us, 3), "algorithmic_bytes": int(nbytes),
                          "achieved_gbps": round(gbps, 1), "frac": round(gbps / PEAK_HBM_GBPS, 4), **extra}),
              flush=True)

    h, f, nh, nkv, hd = 3584, 18944, 28, 4, 128
    XU, YU = K.LAYOUT_X_UT, K.LAYOUT_Y_UT
    x = torch.randn(h, device=device)
    nw = K.to_ut(torch.ones(h, device=device))
    res = torch.randn(h, device=device)
    act = torch.randn(f, device=device)
    cases = [
        ("o_proj Q4_K 3584->3584 +res", Q4_K, h, h, lambda ww: K.qgemv(x, ww, residual=res, layout=XU | YU),
         4 * 3 * h),
        ("gate_up Q4_K rmsnorm 3584->2x18944 silu", Q4_K, 2 * f, h,
         lambda ww: K.qgemv_norm_silu(x, nw, ww, 1e-6, layout=XU | YU), 4 * (2 * h + f)),
        ("ffn_down Q6_K 18944->3584 +res", Q6_K, h, f, lambda ww: K.qgemv(act, ww, residual=res, layout=XU | YU),
         4 * (f + 2 * h)),
    ]
    for name, t, n, k, fn, io in cases:
        w0 = qweight(t, n, k)
        ws = [w0] + [w0.copy() for _ in range(ncopies(w0.nbytes) - 1)]
        us = time_kernel([(lambda ww=ww: fn(ww)) for ww in ws], 200)
        emit("config4_gemv", us, w0.nbytes + io, kernel=name)
        del ws, w0
        torch.cuda.empty_cache()
    wq, wk, wv = qweight(Q4_K, nh * hd, h), qweight(Q4_K, nkv * hd, h), qweight(Q6_K, nkv * hd, h)
    qkv_bytes = wq.nbytes + wk.nbytes + wv.nbytes
    trip = [(wq, wk, wv)] + [tuple(w.copy() for w in (wq, wk, wv)) for _ in range(ncopies(qkv_bytes) - 1)]
    bq, bk, bv = (torch.randn(m * hd, device=device) for m in (nh, nkv, nkv))
    cos = torch.randn(4096, hd // 2, device=device)
    sin = torch.randn(4096, hd // 2, device=device)
    pos = torch.tensor([200], device=device)
    kc = torch.zeros(nkv, 384, hd, device=device)
    vc = torch.zeros_like(kc)
    xu = K.to_ut(x)
    us = time_kernel([(lambda tr=tr: K.qkv_rmsnorm_rope(xu, nw, 1e-6, *tr, bq, bk, bv, cos, sin, pos, kc, vc, nh,
                                                        layout=XU)) for tr in trip], 200)
    emit("config4_qkv_rmsnorm_rope", us, qkv_bytes + 4 * (3 * h + 2 * (nh + 2 * nkv) * hd),
         kernel="3584->28x128 + 2x4x128, Q4_K/Q4_K/Q6_K")
    del trip
    q = torch.randn(nh, hd, device=device)
    for L in (384, 4096):
        kvb = 2 * nkv * L * hd * 4
        kvs = [(torch.randn(nkv, L, hd, device=device), torch.randn(nkv, L, hd, device=device))
               for _ in range(ncopies(kvb))]
        wsp = K.decode_attn_workspace(nh, nkv, hd, L, device)
        S = torch.tensor([L], device=device)
        us = time_kernel([(lambda kv=kv: K.decode_attn(q, kv[0], kv[1], S=S, workspace=wsp, layout=YU))
                          for kv in kvs], 200)
        emit("config4_decode_attn", us, kvb + 4 * 2 * nh * hd, positions=L, heads=f"{nh}/{nkv}", head_dim=hd)
        del kvs


def config3(eng, arch, path) -> dict:
    """the config-0 model with an 8192-token random-id prompt prefilled on the
    matrix cores (fp16 operands, fp32 accumulation), then 256 greedy decode steps of the
    graph-captured step at context ~8192. Returns the JSON object: prefill tok/s, its
    algorithmic TFLOP/s against the 2.5 PFLOP/s dense fp16 MFMA peak, decode tok/s."""
    import numpy as np
    import torch
    L, steps = 8192, 256
    prompt = np.random.default_rng(PROMPT_SEED + 3).integers(0, arch.vocab, size=L).tolist()
    cache = eng._empty_cache(L + steps + 8)
    graph = eng._build_decode_graph(cache)
    times = []
    for _ in range(3):  # the first also builds the fp16 weight copies
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        eng.prefill_greedy(prompt, cache)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    pf = statistics.median(times[1:])
    t0 = time.perf_counter()
    toks = eng.decode_greedy(graph, steps, None)
    torch.cuda.synchronize()
    dec = time.perf_counter() - t0
    c = eng.cfg
    hd, nh, nkv, h, f = c.head_dim, c.n_head, c.n_kv_head, c.hidden, c.ffn_dim
    gemm_flop = 2.0 * L * c.n_layers * (h * (nh + 2 * nkv) * hd + nh * hd * h + 2 * f * h + h * f)
    attn_flop = 4.0 * hd * nh * (L * (L + 1) / 2) * c.n_layers   # causal: QK^T and P.V
    tflops = (gemm_flop + attn_flop) / pf / 1e12
    log(f"config 3: prefill {pf * 1e3:.2f} ms ({tflops:.0f} TFLOP/s), decode at 8192 {steps / dec:.1f} tok/s")
    return {"metric": "config 3: 8192-token prefill on MFMA + decode at context 8192",
            "prefill_tok_s": round(L / pf, 1), "prefill_ms": round(pf * 1e3, 2),
            "prefill_ms_samples": [round(t * 1e3, 2) for t in times[1:]],
            "prefill_flop": gemm_flop + attn_flop, "prefill_tflops": round(tflops, 1),
            "prefill_mfma_frac": round(tflops / 2500.0, 4), "mfma_peak_tflops": 2500.0,
            "decode_tok_s": round(steps / dec, 1),
            "decode_steps": steps, "context": L, "dtype": "fp16 operands, fp32 accumulate (prefill); fp32 (decode)",
            "data": "synthetic config-0 model (seed 0), uniform random prompt ids", "tokens_head": toks[:8],
            "gguf_sha256": synth_sha(path)}


def config4(args) -> dict | None:
    """Qwen2.5-7B-architecture decoder, random-init N(0,0.02) quantized
    Q4_K_M-style (Q4_K attn q/k/o + gate/up, Q6_K attn_v + ffn_down, Q8_0 token_embd and an
    untied Q8_0 LM head), built on the GPU (pico_hip.synth, device draws; seed 0). Batch 1,
    128-token random prompt (fp16 matrix-core prefill), 256 greedy decode steps of the
    HIP-graph step. Returns the JSON object: decode tok/s (median of the timed runs), weight +
    KV bytes per token and their fraction of 8 TB/s, and every decode kernel timed alone over
    >= 1 GiB of copies (the roofline object is the one with the largest time per token)."""
    import numpy as np
    import torch
    from pico_hip import synth
    from pico_hip.engine import Engine
    arch = synth.ARCHES["qwen2.5-7b"]
    t0 = time.time()
    path = synth.cached(arch, seed=MODEL_SEED, cache_dir=args.model_dir, device="cuda:0", progress=log)
    log(f"7B model {path} ready in {time.time() - t0:.1f}s")
    t0 = time.time()
    eng = Engine(path, device="cuda:0")
    log(f"engine loaded in {time.time() - t0:.1f}s")
    if args.kernel_only:
        kernel_only(eng, args)
        return None
    n_prompt, steps = 128, 256
    # the 128-token prompt is prefilled on the matrix cores (fp16 operands, fp32 accumulation:
    # the reference's CUDA autocast prefill, model.py:147-151); the fp32 small-M path re-reads
    # and re-decodes 4.75 GB of packed weights per 8-token tile
    eng.model.prefill_f16_min_tokens = 64
    prompt = np.random.default_rng(PROMPT_SEED + 4).integers(0, arch.vocab, size=n_prompt).tolist()
    run_decode(eng, prompt, steps, timed=False)
    samples, toks, pf = [], None, []
    for _ in range(3):
        el, p_s, out = run_decode(eng, prompt, steps, timed=True)
        samples.append(len(out) / el)
        pf.append(p_s)
        toks = out
        log(f"7B decode {samples[-1]:.1f} tok/s")
    value = statistics.median(samples)
    c = eng.cfg
    weight_bytes = eng.model.weight_bytes_per_token()
    kv_pos = 2 * c.n_kv_head * c.head_dim * 4 * c.n_layers
    mean_S = n_prompt + (steps + 1) / 2.0
    bytes_per_token = weight_bytes + kv_pos * (mean_S + 1)
    dec_gbps = bytes_per_token * value / 1e9
    # the attention row of the kernel table: the mean context of the timed run
    table = kernel_table(eng, 200, 4, attn=(int(mean_S), n_prompt + steps))
    line = {
        "metric": "config 4: batch-1 decode tok/s (7B Q4_K_M arch)", "value": round(value, 2),
        "unit": "tok/s", "n_gpus": 1, "steps": steps, "ms_per_step": round(1000.0 / value, 4),
        "higher_is_better": True,
        "dtype": "fp32 (Q4_K_M-style packed weights, fp32 activations/KV)",
        "data": "synthetic: random-init N(0,0.02) weights drawn and quantized on the GPU (seed 0), "
                "128 uniform random prompt ids (fp16 MFMA prefill)",
        "config": {"workload": "BASELINE config 4: Qwen2.5-7B-arch Q4_K_M-style GGUF, batch 1, 128-token "
                               "prompt, 256 greedy decode steps, HIP-graph step",
                   "gguf_sha256": synth.sha256(path)},
        "decode_samples_tok_s": [round(v, 2) for v in samples],
        "prefill_tok_s": round(n_prompt / statistics.median(pf), 1),
        "decode_roofline": {"bytes_per_token": int(bytes_per_token), "weight_bytes_per_token": int(weight_bytes),
                            "achieved": round(dec_gbps, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                            "frac": round(dec_gbps / PEAK_HBM_GBPS, 4)},
        "roofline": roofline_of(table, None),
        "kernels": table,
        "tokens_head": toks[:8]}
    del eng
    torch.cuda.empty_cache()
    return line


def synth_sha(path):
    from pico_hip import synth
    return synth.sha256(path)


def traffic_from_profiles(kernel: str, config: int = 0):
    """HBM bytes per launch of ``kernel`` from the committed counter summary
    (profiles/traffic_decode_kernels.json: reads by request size + WRITE_SIZE), or None."""
    p = ROOT / "profiles" / "traffic_decode_kernels.json"
    try:
        return json.loads(p.read_text())[f"config{config}_{kernel}"]["bytes_per_launch"]
    except (ValueError, OSError, KeyError):
        return None


def cpu_baseline(path, prompt, budget_s: float):
    import torch
    from oracle.ref_cpu import RefModel
    cores = len(os.sched_getaffinity(0))
    cores = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))
    torch.set_num_threads(cores)
    ref = RefModel(path)
    steps_max = 64
    cache = ref.empty_cache(len(prompt) + steps_max)
    logits = ref.forward(torch.tensor(prompt), torch.arange(len(prompt)), cache)
    done, t0 = 0, time.perf_counter()
    while done < steps_max:
        tok = int(logits.argmax())
        logits = ref.forward(torch.tensor([tok]), torch.tensor([len(prompt) + done]), cache)
        done += 1
        if time.perf_counter() - t0 > budget_s and done >= 2:
            break
    el = time.perf_counter() - t0
    return {"value": round(done / el, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"config 0 on the host CPU: fp32 prefill of the 13-token prompt, then {done} "
                      f"greedy decode steps timed ({el:.1f} s) with oracle/ref_cpu.py (the reference's "
                      "torch-CPU forward formulations), torch threads = cores"}


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64, help="timed decode tokens")
    ap.add_argument("--warmup", type=int, default=2, help="untimed full runs before the timed one")
    ap.add_argument("--reps", type=int, default=9, help="extra timed runs for median/p10/p90")
    ap.add_argument("--kernel", default=None,
                    help="kernel for the roofline object (default: the largest time per token), or the "
                         "kernel --kernel-only times: gate_up, gate_up_norm, lm_head, down_q6k, down_q4k, "
                         "qkv, attn_oproj, gate_up_fix, attn_gproj, attn, oproj")
    ap.add_argument("--no-extra-configs", action="store_true",
                    help="leave the config 3 and config 4 objects off the config-0 line")
    ap.add_argument("--kernel-iters", type=int, default=400)
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU-baseline decode")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--config", type=int, default=0, choices=(0, 3, 4),
                    help="3: long-context prefill on the matrix cores + decode at 8192 instead; "
                         "4: the 7B-architecture model")
    ap.add_argument("--micro", action="store_true",
                    help="BASELINE configs 1 and 2 kernel microbenchmarks (one JSON line each) instead")
    ap.add_argument("--kernel-only", action="store_true",
                    help="only time --kernel and a 1 GiB copy (for rocprofv3 --pmc traffic runs)")
    ap.add_argument("--model-dir", default=os.environ.get("PICO_HIP_CACHE", "/tmp/pico_hip_models"))
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build runs the batch-1 decode on "
              "exactly one GPU (the multi-GPU sharding plan is design-only).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    from pico_hip import synth
    from pico_hip.engine import Engine

    if args.micro:
        micro7b("cuda:0") if args.config == 4 else micro("cuda:0")
        return

    if args.config == 4:
        line = config4(args)
        if line is not None:
            print(json.dumps(line), flush=True)
        return

    arch = synth.ARCHES["qwen2.5-0.5b"]
    t0 = time.time()
    path = synth.cached(arch, seed=MODEL_SEED, cache_dir=args.model_dir)
    log(f"model {path} ready in {time.time() - t0:.1f}s")
    eng = Engine(path, device="cuda:0")
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, arch.vocab, size=N_PROMPT).tolist()
    log(f"engine loaded; {torch.cuda.get_device_name(0)}")
    if args.config == 3:
        print(json.dumps(config3(eng, arch, path)), flush=True)
        return

    if args.kernel_only:
        kernel_only(eng, args)
        return

    for _ in range(args.warmup):
        run_decode(eng, prompt, args.steps, timed=False)
    # 1 + reps timed runs of exactly `steps` decode tokens each (evidence.py:138-163: the
    # receipt's median / p10 / p90 over repetitions); value = their median
    samples, tokens, prefill = [], None, []
    for _ in range(1 + args.reps):
        e, p_s, t = run_decode(eng, prompt, args.steps, timed=True)
        samples.append(len(t) / e)
        prefill.append(p_s)
        tokens = t
    value = statistics.median(samples)
    log(f"decode {value:.1f} tok/s (median of {len(samples)}; first {samples[0]:.1f})")

    # decode roofline: weight bytes per token + KV bytes (read S positions, write one)
    c = eng.cfg
    weight_bytes = eng.model.weight_bytes_per_token()
    kv_pos = 2 * c.n_kv_head * c.head_dim * 4 * c.n_layers
    mean_S = N_PROMPT + (args.steps + 1) / 2.0
    bytes_per_token = weight_bytes + kv_pos * (mean_S + 1)
    dec_gbps = bytes_per_token * value / 1e9

    # every decode kernel alone; the roofline object is the one with the largest time per token.
    # The monotonic clock in the log separates the decode runs from these loops in a profile.
    torch.cuda.synchronize()
    log(f"kernel table begins at monotonic {time.monotonic_ns()} ns")
    table = kernel_table(eng, args.kernel_iters, 0,
                         attn=(int(mean_S), N_PROMPT + args.steps))
    roof = roofline_of(table, args.kernel)
    if args.kernel and not any(r["key"] == args.kernel for r in table):
        launchers, alg_bytes, kname = kernel_launchers(eng, args.kernel)
        avg_us = time_kernel(launchers, args.kernel_iters)
        achieved = alg_bytes / (avg_us * 1e-6) / 1e9
        roof = {"bound": "hbm", "kernel": kname, "achieved": round(achieved, 1), "peak": PEAK_HBM_GBPS,
                "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBPS, 4),
                "traffic": traffic_from_profiles(args.kernel), "avg_launch_us": round(avg_us, 3),
                "algorithmic_bytes": int(alg_bytes), "selected_as": "requested by --kernel"}
    log(f"roofline kernel: {roof['kernel']} ({roof['frac'] * 100:.1f} % of {PEAK_HBM_GBPS:.0f} GB/s)")

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(path, prompt, args.cpu_budget)
        log(f"cpu baseline {cpu['value']} tok/s on {cpu['cores']} cores")

    line = {
        "metric": "batch-1 decode tok/s (0.5B Q4_K_M arch)",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1000.0 / value, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 (Q4_K_M-style packed weights, fp32 activations/KV)",
        "data": "synthetic: random-init N(0,0.02) weights quantized to GGUF (seed 0), 13 uniform random prompt ids",
        "config": {"workload": "BASELINE config 0: Qwen2.5-0.5B-arch Q4_K_M-style GGUF, batch 1, "
                               "13-token prompt, greedy decode, HIP-graph step",
                   "prompt_tokens": N_PROMPT, "decode_tokens": args.steps, "gguf_sha256": synth.sha256(path)},
        "decode_samples_tok_s": {"median": round(value, 2),
                                 "p10": round(float(np.percentile(samples, 10)), 2),
                                 "p90": round(float(np.percentile(samples, 90)), 2), "n": len(samples),
                                 "all": [round(v, 2) for v in samples]},
        "prefill_tok_s": round(N_PROMPT / statistics.median(prefill), 1),
        "decode_roofline": {"bytes_per_token": int(bytes_per_token), "achieved": round(dec_gbps, 1),
                            "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": round(dec_gbps / PEAK_HBM_GBPS, 4)},
        "roofline": roof,
        "kernels": table,
        "cpu_baseline": cpu,
        "tokens_head": tokens[:8],
    }
    if not args.no_extra_configs:
        # configs 3 and 4 on the same line (about a minute together)
        line["config3"] = config3(eng, arch, path)
        del eng
        torch.cuda.empty_cache()
        line["config4"] = config4(args)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
