"""Benchmark of the speculative-decoding verification path on one MI355X.

Workload: batched chain verification, B=64
sequences, K=8 draft tokens, V=128256, temperature 0.7.  Target logits
[64,9,V] fp32 ~ 2*N(0,1); draft logits [64,8,V] = target + 0.5*N(0,1); drafts
drawn from softmax(draft/T); seeded U(0,1) uniforms [64,9].  One step = one
call of the fused kernel path (softmax of target and draft + per-sequence
acceptance + exact resample / bonus draw) over one batch resident in HBM;
NSETS batches rotate so that the 256 MB last-level cache cannot serve them.

value = verified tokens per second = sum over sequences of (accepted drafts
+ 1 resampled-or-bonus token) / wall time, per-sequence rules of
csrc/src/scheduler/speculative.cpp:50-103.

Prints one JSON line (rank 0).  --gpus above 1 is refused: this build runs on
one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "verified tok/s (B=64,K=8,V=128k) + tree-attn/sampling HBM GB/s as % of peak"
HBM_PEAK_GBS = 8000.0
B, K, V, T = 64, 8, 128256, 0.7
SIGMA, NOISE = 2.0, 0.5
NSETS = 4
# algorithmic bytes of one step: target [B,K+1,V] + draft [B,K,V] logits, read once
ALG_BYTES = B * (2 * K + 1) * V * 4


def make_inputs(dev, seed):
    import torch

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    tl = torch.randn(B, K + 1, V, device=dev, generator=g) * SIGMA
    dl = tl[:, :K] + NOISE * torch.randn(B, K, V, device=dev, generator=g)
    probs = torch.softmax(dl / T, dim=-1).reshape(B * K, V)
    tok = torch.multinomial(probs, 1, generator=g).reshape(B, K).to(torch.int32)
    U = torch.rand(B, K + 1, device=dev, generator=g)
    return tl.contiguous(), dl.contiguous(), tok, U


def cpu_baseline(tl, dl, tok, U, budget_s=12.0):
    """The oracle (plain C restatement of speculative.cpp, OpenMP over rows)
    on the host cores: softmax of both logit tensors, then per-row
    verification; repeated on the same batch until ~budget_s elapse."""
    import numpy as np
    from oracle import oracle as O

    threads = int(os.environ.get("OMP_NUM_THREADS", 0)) or len(os.sched_getaffinity(0))
    os.environ["OMP_NUM_THREADS"] = str(threads)
    t, d = tl.cpu().numpy(), dl.cpu().numpy()
    tk, u = tok.cpu().numpy(), U.cpu().numpy()
    passes, emitted, t0 = 0, 0, time.perf_counter()
    while True:
        tp = O.softmax_rows(t, T)
        dp = O.softmax_rows(d, T)
        out = O.chain_verify(tp, dp, tk, u)
        emitted += int(out["num_emitted"].sum())
        passes += 1
        el = time.perf_counter() - t0
        if el >= budget_s or passes >= 50:
            break
    return {"value": emitted / el, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{passes} full passes over one B=64,K=8,V=128256 batch "
                      f"(oracle softmax + per-row verify, {el:.1f} s)"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (no multi-GPU path); "
              "run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    from cudaforge_amd import _lib
    from cudaforge_amd.verify import chain_verify, chain_workspace_bytes

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    _lib.load()
    sets = [make_inputs(dev, 1000 + s) for s in range(NSETS)]
    ws = torch.empty(chain_workspace_bytes(B, K, V, "logits", "cpp"), dtype=torch.uint8,
                     device=dev)

    def step(i):
        tl, dl, tok, U = sets[i % NSETS]
        return chain_verify(tl, dl, tok, U, input_kind="logits", temperature=T, mode="cpp",
                            workspace=ws)

    emitted = []
    for s in range(NSETS):
        emitted.append(int(step(s).num_emitted.sum().item()))
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # timed region: no per-kernel events (they add a few µs per launch)
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(args.steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_total = e0.elapsed_time(e1)
    ms_per_step = ms_total / args.steps
    tokens = sum(emitted[i % NSETS] for i in range(args.steps))
    value = tokens / (ms_total / 1e3)

    # per-kernel durations: the same steps again, each launch bracketed by
    # HIP events on the stream it runs on
    _lib.profile_reset()
    _lib.profile_enable(True)
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    _lib.profile_enable(False)

    kern = {}
    for name in ("chain_stats", "chain_decide", "chain_plan", "chain_mw_sums", "chain_mw_records",
                 "chain_mw_walk", "chain_finish"):
        n, ms = _lib.profile_query(name)
        kern[name] = ms / args.steps  # per step (records and walk run twice)
    _lib.profile_reset()
    stats_ms = kern["chain_stats"]  # one launch per step
    achieved = ALG_BYTES / (stats_ms * 1e-3) / 1e9

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded torch.randn logits, multinomial drafts, U(0,1))",
        "config": {"workload": "chain acceptance sampling B=64,K=8,V=128256,T=0.7 "
                               "(BASELINE configs[1]); per-sequence rules",
                   "B": B, "K": K, "V": V, "temperature": T, "input": "fp32 logits",
                   "mean_accept_len": round(sum(emitted) / (NSETS * B) - 1, 3)},
        "roofline": {"bound": "hbm", "kernel": "chain_stats",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None},
        "kernels_ms_per_step": {k: round(v, 5) for k, v in kern.items()},
        "step_hbm_gbs": round(ALG_BYTES / (ms_per_step * 1e-3) / 1e9, 1),
        "wall_s": round(wall, 4),
    }
    if not args.no_cpu_baseline:
        tl, dl, tok, U = sets[0]
        line["cpu_baseline"] = cpu_baseline(tl, dl, tok, U)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
