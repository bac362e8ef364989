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
MFMA_BF16_PEAK = 2.5e15  # dense bf16 FLOP/s
B, K, V, T = 64, 8, 128256, 0.7
SIGMA, NOISE = 2.0, 0.5
NSETS = 4
# algorithmic bytes of one step: target [B,K+1,V] + draft [B,K,V] logits, read once
ALG_BYTES = B * (2 * K + 1) * V * 4   # every logit of both windows
# Under the per-sequence rules with logits, the library reads the rows of
# positions 0 .. HEAD-1 of every sequence first, and the other rows (the
# remaining positions and the target's row K) only for sequences that
# accepted all HEAD of them (kHeadPositions in csrc/chain_verify.hip).
HEAD_POSITIONS = 3


def stats_rows(accept_len) -> int:
    """Rows the two statistics passes read in one step, given the step's
    accepted-draft counts: each of them read once."""
    pending = int((accept_len >= HEAD_POSITIONS).sum())
    return B * 2 * HEAD_POSITIONS + pending * (2 * (K - HEAD_POSITIONS) + 1)
# per-dispatch HBM traffic measured with rocprofv3 --pmc for this build
TRAFFIC_TABLE = os.path.join(ROOT, "profiles", "hbm_traffic_per_dispatch.md")


def traffic_from_profile(kernel: str):
    """HBM bytes (read + written) per dispatch of `kernel` from the counter
    table in profiles/hbm_traffic_per_dispatch.md (the table whose header has
    columns "HBM bytes read" and "HBM bytes written"); None when there is no
    such row."""
    try:
        with open(TRAFFIC_TABLE) as f:
            lines = [ln.strip() for ln in f]
    except OSError:
        return None

    def cells(ln):
        return [c.strip() for c in ln.strip("|").split("|")]

    for i, ln in enumerate(lines):
        if not ln.startswith("|"):
            continue
        head = cells(ln)
        if "HBM bytes read" not in head or "HBM bytes written" not in head:
            continue
        ir, iw = head.index("HBM bytes read"), head.index("HBM bytes written")
        for row in lines[i + 2:]:
            if not row.startswith("|"):
                break
            c = cells(row)
            if c[0].strip("`") == kernel:
                return int(c[ir].replace(",", "")) + int(c[iw].replace(",", ""))
    return None


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


def _cpu_model() -> str:
    """/proc/cpuinfo's model name with its family / model / stepping numbers
    (virtual machines often report only "AMD EPYC" as the name)."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if not ln.strip():
                    break                      # first processor only
                k, _, v = ln.partition(":")
                info[k.strip()] = v.strip()
    except OSError:
        return "unknown"
    name = info.get("model name", "unknown")
    ids = [f"{k} {info[k]}" for k in ("cpu family", "model", "stepping") if k in info]
    return f"{name} ({', '.join(ids)})" if ids else name


def _timed(fn, budget_s):
    """Call fn() (returns tokens emitted) until budget_s elapse; (passes,
    tokens, seconds)."""
    passes, emitted, t0 = 0, 0, time.perf_counter()
    while True:
        emitted += fn()
        passes += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            return passes, emitted, el


def cpu_baseline(tl, dl, tok, budget_s=6.0):
    """The chain-acceptance workload on the host cores, from the same logits:
    torch-CPU softmax of the target and draft windows (what the reference's
    python engine runs, speculative.py:118, :145), then the reference's own
    SpeculativeEngine::verify_candidates (csrc/src/scheduler/speculative.cpp,
    compiled from source into oracle/_ref) once per sequence on one engine,
    as its pybind binding serves it.  Timed with every host thread and with
    one; the build's C port of the same rules (OpenMP over rows) beside it.
    Without oracle/_ref the port is the reported figure."""
    import numpy as np
    import torch
    from oracle import oracle as O

    threads = len(os.sched_getaffinity(0))
    t_c, d_c = tl.cpu(), dl.cpu()
    tk = tok.cpu().numpy()
    ref = O.ref_lib()

    def softmax():
        return (torch.softmax(t_c / T, dim=-1).numpy(), torch.softmax(d_c / T, dim=-1).numpy())

    def ref_pass():
        tp, dp = softmax()
        out = O.ref_verify(1234, tk, dp, tp, -1)
        return int(out["num_accepted"].sum()) + B  # accepted drafts + one final token each

    def port_pass():
        tp = O.softmax_rows(t_c.numpy(), T)
        dp = O.softmax_rows(d_c.numpy(), T)
        u = np.random.default_rng(0).random((B, K + 1)).astype(np.float32)
        return int(O.chain_verify(tp, dp, tk, u)["num_emitted"].sum())

    sample = "passes over one B=64,K=8,V=128256 logit batch (softmax of both windows + verify)"
    res = {"cpu_model": _cpu_model(), "threads_available": threads}
    old = torch.get_num_threads()
    try:
        for label, fn in (("reference", ref_pass), ("port", port_pass)):
            if label == "reference" and ref is None:
                continue
            for nt in (threads, 1):
                torch.set_num_threads(nt)
                O.set_threads(nt)
                passes, emitted, el = _timed(fn, budget_s if nt > 1 else budget_s / 2)
                res[f"{label}_{nt}t"] = {"value": round(emitted / el, 1), "unit": "tok/s",
                                         "cores": nt, "sample": f"{passes} {sample}, {el:.1f} s"}
    finally:
        torch.set_num_threads(old)
        O.set_threads(threads)
    head = res.get(f"reference_{threads}t") or res[f"port_{threads}t"]
    out = dict(head)
    out["kind"] = "reference" if f"reference_{threads}t" in res else "port"
    out.update({k: v for k, v in res.items() if k not in (f"{out['kind']}_{threads}t",)})
    if out["kind"] == "reference":
        out["sample"] += ("; reference verify_candidates single-threaded per call, softmax on "
                          f"{threads} threads")
    return out


def chain_step_c1_leg(dev, steps=20, warmup=3, cpu_budget_s=6.0):
    """the drop-in SpeculativeEngine.step() (python
    mode, the reference's default) with random-init fp32 runners -- target
    4 layers / d 512 / 8 heads of 64, draft 1 layer / d 256 / 4 heads,
    V = 32000 -- at B = 1, K = 4, a 128-token seeded prompt, T = 1.0; every
    step verifies from the same prompt.  Beside it the same step on the host
    (oracle/speculative_cpu.py: torch-CPU runners with the same weights and
    the C oracle's rejection sampling)."""
    import torch
    from cudaforge_amd.runners import draft_runner, target_runner
    from cudaforge_amd.speculative import SpeculativeEngine
    from oracle.speculative_cpu import chain_step

    Kc, Vc, P = 4, 32000, 128
    tgt_c, drf_c = target_runner(seed=1), draft_runner(seed=2)
    tgt, drf = tgt_c.to(dev), drf_c.to(dev)
    g = torch.Generator().manual_seed(42)
    prompt = torch.randint(0, Vc, (1, P), generator=g)
    eng = SpeculativeEngine(drf, tgt, num_speculative_tokens=Kc, temperature=1.0,
                            generator=torch.Generator(device=dev).manual_seed(43))
    ids = prompt.to(dev)
    for _ in range(warmup):
        eng.step(ids)
    torch.cuda.synchronize()
    eng.total_draft_tokens = eng.total_accepted_tokens = 0
    t0 = time.perf_counter()
    dlat = tlat = 0.0
    for _ in range(steps):
        r = eng.step(ids)
        dlat += r.draft_latency_ms
        tlat += r.target_latency_ms
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    out = {"config": "chain step B=1,K=4,V=32000,prompt 128,T=1.0; random-init fp32 target "
                     "4L/d512/8x64, draft 1L/d256/4x64 (BASELINE configs[0]); drop-in "
                     "SpeculativeEngine.step(), python mode",
           "gpu": {"ms_per_step": round(dt / steps * 1e3, 3),
                   "steps_s": round(steps / dt, 1),
                   "accepted_tok_s": round(eng.total_accepted_tokens / dt, 1),
                   "acceptance_rate": round(eng.get_aggregate_acceptance_rate(), 3),
                   "draft_ms": round(dlat / steps, 3), "target_ms": round(tlat / steps, 3)}}
    threads = len(os.sched_getaffinity(0))
    old = torch.get_num_threads()
    try:
        for nt in (threads, 1):
            torch.set_num_threads(nt)
            gc = torch.Generator().manual_seed(44)
            chain_step(drf_c, tgt_c, prompt, Kc, generator=gc)  # warm-up
            emitted, n, t0 = 0, 0, time.perf_counter()
            while True:
                emitted += chain_step(drf_c, tgt_c, prompt, Kc, generator=gc)[1]
                n += 1
                el = time.perf_counter() - t0
                if el >= (cpu_budget_s if nt > 1 else cpu_budget_s / 2):
                    break
            out[f"cpu_{nt}t"] = {"ms_per_step": round(el / n * 1e3, 2),
                                 "steps_s": round(n / el, 2),
                                 "accepted_tok_s": round(emitted / el, 1), "cores": nt,
                                 "kind": "port", "sample": f"{n} steps, {el:.1f} s"}
    finally:
        torch.set_num_threads(old)
    out["cpu_model"] = _cpu_model()
    return out


def _time_launches(fn, reps, names):
    """Run fn() reps times with per-kernel HIP events; returns avg ms per call
    per kernel name (launches inside one call are summed)."""
    import torch
    from cudaforge_amd import _lib

    torch.cuda.synchronize()
    _lib.profile_reset()
    _lib.profile_enable(True)
    for _ in range(reps):
        fn()
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    out = {n: _lib.profile_query(n)[1] / reps for n in names}
    _lib.profile_reset()
    return out


def _warm_up(fn, seconds=0.3, min_calls=40):
    """Call fn() in rounds of 20 until at least min_calls calls and `seconds`
    of wall time have passed: a leg's first calls run up to 20% slower than
    its later ones (tree attention: 97 against 81 us per call after 40
    warm-up calls in a fresh process)."""
    import torch

    torch.cuda.synchronize()
    t_end = time.perf_counter() + seconds
    n = 0
    while n < min_calls or time.perf_counter() < t_end:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        n += 20


def tree_attention_leg(dev, reps=20):
    """B=16, 63-node binary tree, 32 q / 8 KV heads,
    head_dim 128, context 4096, page 16, random page table, bf16 N(0,1)."""
    import torch
    from cudaforge_amd import tree as Tr
    from cudaforge_amd.verify import tree_attention, tree_attention_workspace_bytes

    Bt, N, Hq, Hkv, D, bs, C = 16, 63, 32, 8, 128, 16, 4096
    nps = (C + N + bs - 1) // bs
    nblk = Bt * nps + 8
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    kp = torch.randn(nblk, 1, Hkv, bs, D, device=dev, generator=g).bfloat16()
    vp = torch.randn(nblk, 1, Hkv, bs, D, device=dev, generator=g).bfloat16()
    bt = torch.randperm(nblk, device=dev, generator=g)[: Bt * nps].int().reshape(Bt, nps)
    q = torch.randn(Bt, N, Hq, D, device=dev, generator=g).bfloat16()
    ctx = torch.full((Bt,), C, dtype=torch.int32, device=dev)
    masks = Tr.ancestor_masks(Tr.binary_tree_parents(N))
    mt = Tr.mask_tensor(masks, dev)
    anc = int(sum(bin(int(x)).count("1") for x in masks))
    flops = 4 * Bt * Hq * D * (N * C + anc)
    nbytes = (Bt * Hkv * (C + N) * D * 2 * 2      # K and V rows read once
              + 2 * q.numel() * 2 + bt.numel() * 4)  # q in, out, page table
    out = torch.empty_like(q)
    ws = torch.empty(tree_attention_workspace_bytes(Bt, N, Hq, Hkv, D, C + N), dtype=torch.uint8,
                     device=dev)

    def run():
        tree_attention(q, kp, vp, bt, ctx, mt, max_keys=C + N, out=out, workspace=ws)

    _warm_up(run)
    ms = _time_launches(run, reps, ("tree_attn", "tree_attn_merge"))
    t = (ms["tree_attn"] + ms["tree_attn_merge"]) * 1e-3
    # the whole call on its stream, back to back (adds the dispatch gap
    # between the two kernels and between calls)
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(reps):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    t_call = e0.elapsed_time(e1) / reps * 1e-3
    return {"config": "B=16,N=63 binary tree,Hq=32,Hkv=8,d=128,ctx=4096,page=16 (BASELINE configs[2])",
            "us": round(t * 1e6, 2), "kernels_us": {k: round(v * 1e3, 2) for k, v in ms.items()},
            "call_us": round(t_call * 1e6, 2),
            "flop": flops, "tflops": round(flops / t / 1e12, 1),
            "mfma_frac": round(flops / t / MFMA_BF16_PEAK, 4),
            "bytes": nbytes, "gbs": round(nbytes / t / 1e9, 1),
            "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}


def tree_accept_commit_leg(dev, reps=10):
    """B=32, 63-node binary tree, V=128256, fp32
    target/draft logits per node (as configs[1]), node tokens drawn from the
    parent's draft softmax, T=0.7, seeded uniforms; then the KV commit of the
    accepted paths (32 layers x 8 KV heads x 128, bf16, page 16, ctx 1024)."""
    import torch
    from cudaforge_amd import tree as Tr
    from cudaforge_amd.verify import kv_commit, tree_verify

    Bt, N, Vt, L, Hkv, D, bs, C = 32, 63, 128256, 32, 8, 128, 16, 1024
    parents = Tr.binary_tree_parents(N)
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    tl = torch.randn(Bt, N, Vt, device=dev, generator=g) * SIGMA
    dl = tl + NOISE * torch.randn(Bt, N, Vt, device=dev, generator=g)
    par = torch.from_numpy(parents).to(dev)
    probs = torch.softmax(dl[:, par[1:].long()] / T, dim=-1).reshape(-1, Vt)
    tok = torch.zeros(Bt, N, dtype=torch.int32, device=dev)
    tok[:, 1:] = torch.multinomial(probs, 1, generator=g).reshape(Bt, N - 1).int()
    del probs
    U = torch.rand(Bt, N + 1, device=dev, generator=g)
    nps = (C + N + bs - 1) // bs
    nblk = Bt * nps
    kp = torch.randn(nblk, L, Hkv, bs, D, device=dev, generator=g).bfloat16()
    vp = torch.randn(nblk, L, Hkv, bs, D, device=dev, generator=g).bfloat16()
    bt = torch.randperm(nblk, device=dev, generator=g).int().reshape(Bt, nps)
    ctx = torch.full((Bt,), C, dtype=torch.int32, device=dev)

    res = {}

    def run():
        res["tv"] = tree_verify(tl, dl, par, tok, U, input_kind="logits", temperature=T,
                                mode="cpp")
        res["kc"] = kv_commit(kp, vp, bt, ctx, res["tv"].path, res["tv"].path_len)

    for _ in range(2):
        run()
    torch.cuda.synchronize()
    res["tv"].check_status()  # a failed walk's paths are not valid (RuntimeError)
    plen = res["tv"].path_len.cpu().numpy()
    path = res["tv"].path.cpu().numpy()
    emitted = int(res["tv"].num_emitted.sum())
    visited_nodes = int(plen.sum())  # target rows of path nodes; draft rows of non-leaf ones
    alg_accept = (visited_nodes * 2) * Vt * 4
    moved = int(sum(sum(1 for j in range(int(plen[b])) if path[b, j] != j) for b in range(Bt)))
    alg_commit = moved * 2 * (L * Hkv * D * 2 * 2)  # read + write of K and V rows
    ms = _time_launches(run, reps, ("tree_verify", "kv_commit"))
    res["tv"].check_status()
    t_acc, t_com = ms["tree_verify"] * 1e-3, ms["kv_commit"] * 1e-3
    return {"config": "B=32,63-node binary tree,V=128256,T=0.7; commit 32L x 8H x 128 bf16 "
                      "(BASELINE configs[3])",
            "accept_us": round(t_acc * 1e6, 1), "commit_us": round(t_com * 1e6, 2),
            "mean_path_len": round(float(plen.mean()), 3),
            "accepted_tok_s": round(emitted / (t_acc + t_com), 1),
            "accept_alg_bytes": alg_accept,
            "accept_gbs": round(alg_accept / t_acc / 1e9, 1),
            "commit_moved_tokens": moved, "commit_alg_bytes": alg_commit,
            "commit_gbs": round(alg_commit / t_com / 1e9, 1) if moved else None}


def w4a16_gemm_leg(dev, reps=20):
    """The 8B target's four W4A16 projections at the verify step's M = B * 63
    = 504 rows (QKV 4096 -> 6144, O 4096 -> 4096, gate/up 4096 -> 28672,
    down 14336 -> 4096; group 128, zero point 7.5): cfa_w4a16_gemm_zp beside
    dequantise-to-[N, K] + hipBLASLt (the path it replaces), HIP-event time
    per call on the launch stream."""
    import torch
    from cudaforge_amd.w4a16 import w4a16_dequant, w4a16_gemm_zp

    M = 504
    shapes = {"qkv": (4096, 6144), "o": (4096, 4096), "gate_up": (4096, 28672),
              "down": (14336, 4096)}
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    ws = torch.empty(80 << 20, dtype=torch.uint8, device=dev)
    out = {}
    for name, (K, N) in shapes.items():
        a = torch.randn(M, K, device=dev, generator=g).bfloat16()
        q = torch.randint(-2 ** 31, 2 ** 31 - 1, (K // 8, N), dtype=torch.int32, device=dev,
                          generator=g)
        sc = ((torch.rand(K // 128, N, device=dev, generator=g) * 0.5 + 0.5) / K ** 0.5).half()
        z = torch.full_like(sc, 7.5)
        c = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        wt = torch.empty(N, K, dtype=torch.bfloat16, device=dev)

        def fused():
            w4a16_gemm_zp(a, q, sc, z, out=c, workspace=ws)

        def base():
            w4a16_dequant(q, sc, z, dtype=torch.bfloat16, out=wt, transposed=True)
            torch.matmul(a, wt.t(), out=c)

        legs = [("fused_us", fused), ("dequant_hipblaslt_us", base)]
        if name == "gate_up":
            # the target's FFN input: silu(gate) * up, by the SiLU-gated
            # epilogue or by the plain product followed by cfa_silu_mul
            from cudaforge_amd.spec_step import silu_mul
            act = torch.empty(M, N // 2, dtype=torch.bfloat16, device=dev)

            def fused_silu():
                w4a16_gemm_zp(a, q, sc, z, out=act, workspace=ws, silu=True)

            def fused_then_silu_mul():
                w4a16_gemm_zp(a, q, sc, z, out=c, workspace=ws)
                silu_mul(c)

            legs += [("fused_silu_epilogue_us", fused_silu),
                     ("fused_then_silu_mul_us", fused_then_silu_mul)]
        row = {}
        for label, fn in legs:
            _warm_up(fn, seconds=0.2, min_calls=20)
            stream = torch.cuda.current_stream(dev)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record(stream)
            for _ in range(reps):
                fn()
            e1.record(stream)
            torch.cuda.synchronize()
            row[label] = round(e0.elapsed_time(e1) / reps * 1e3, 1)
        flops = 2.0 * M * N * K
        row["fused_tflops"] = round(flops / (row["fused_us"] * 1e-6) / 1e12, 1)
        row["fused_mfma_frac"] = round(flops / (row["fused_us"] * 1e-6) / MFMA_BF16_PEAK, 4)
        out[name] = row
        del a, q, sc, z, c, wt
    out["config"] = "M=504 (B=8 x 63 nodes), bf16 activations, INT4 group 128, zero point 7.5"
    return out


def verify_step_8b_leg(dev, steps=6, warmup=2):
    """one speculative verify step at Llama-3-8B shape --
    random-init W4A16 (group 128) target (32L, d4096, GQA 32/8, FFN 14336,
    V128256), random-init 1B-shape bf16 draft proposing a 63-node binary tree
    (children drawn from the draft softmax), B=8, context 2048 (synthetic
    N(0,1) K/V), T=1.0; tree attention, sampling, verification and commit
    on this library's kernels; the draft levels replay from HIP graphs.
    Random-init models agree on nothing, so the accepted path is the root
    alone and verified tok/s = B / step time."""
    import torch
    from cudaforge_amd.spec_step import (DRAFT_1B, TARGET_8B, DraftModel, TargetModel,
                                         TreeSpeculator)

    Bs, ctx = 8, 2048
    tm = TargetModel(TARGET_8B, dev, seed=0)
    dm = DraftModel(DRAFT_1B, dev, Bs, max_slots=ctx + 64 + 8 * (steps + warmup + 2))
    sp = TreeSpeculator(tm, dm, Bs, ctx, depth=5, temperature=1.0, mode="cpp",
                        max_steps=steps + warmup + 2, use_graphs=True)
    for _ in range(warmup):
        sp.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    emitted = 0
    for _ in range(steps):
        emitted += sum(sp.step().path_len)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    phases = {}
    for _ in range(2):
        sp.step(phases)
    out = {"config": "Llama-3-8B-shape W4A16 g128 target, 1B-shape bf16 draft, 63-node binary "
                     "tree, B=8, ctx 2048, T=1.0 (BASELINE configs[4]); random init",
           "ms_per_step": round(dt / steps * 1e3, 2),
           "verified_tok_s": round(emitted / dt, 1),
           "mean_path_len": round(emitted / (steps * Bs), 3),
           "phases_ms": {k: round(v / 2, 3) for k, v in phases.items()}}
    del sp, tm, dm
    torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-tree", action="store_true",
                    help="skip the extra legs (tree attention, tree accept/commit, 8B verify step)")
    ap.add_argument("--legs",
                    default="chain_step_c1,tree_attention,tree_accept_commit,w4a16_gemm,"
                            "verify_step_8b",
                    help="comma-separated extra legs to run")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device copy (reference for HBM byte counters)")
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
    if args.calibrate_copy:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": src.numel() * 4, "copies": 3}), flush=True)
        return 0
    _lib.load()
    sets = [make_inputs(dev, 1000 + s) for s in range(NSETS)]
    ws = torch.empty(chain_workspace_bytes(B, K, V, "logits", "cpp"), dtype=torch.uint8,
                     device=dev)

    def step(i):
        tl, dl, tok, U = sets[i % NSETS]
        return chain_verify(tl, dl, tok, U, input_kind="logits", temperature=T, mode="cpp",
                            workspace=ws)

    emitted, rows = [], []
    for s in range(NSETS):
        o = step(s)
        emitted.append(int(o.num_emitted.sum().item()))
        rows.append(stats_rows(o.accept_len.cpu().numpy()))
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
    for name in ("chain_stats_head", "chain_stats_tail", "chain_decide", "chain_plan",
                 "chain_mw_first", "chain_mw_tail", "chain_finish"):
        n, ms = _lib.profile_query(name)
        kern[name] = ms / args.steps  # per step
    _lib.profile_reset()
    # the statistics passes: the logits of their rows, each read once
    stats_bytes = sum(rows[i % NSETS] for i in range(args.steps)) / args.steps * V * 4
    stats_ms = kern["chain_stats_head"] + kern["chain_stats_tail"]
    achieved = stats_bytes / (stats_ms * 1e-3) / 1e9
    # the whole step on the workload's algorithmic bytes (every logit once)
    step_gbs = ALG_BYTES / (ms_per_step * 1e-3) / 1e9
    head_t = traffic_from_profile("cfa::chain::stats_kernel<256, 4> (head)")
    tail_t = traffic_from_profile("cfa::chain::stats_tail_kernel<256>")

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
        "roofline": {"bound": "hbm", "kernel": "chain_stats (head + tail passes)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": (head_t + tail_t) if head_t and tail_t else None,
                     "algorithmic_bytes": int(stats_bytes),
                     "logits_read_frac": round(stats_bytes / ALG_BYTES, 4),
                     "step_achieved": round(step_gbs, 1),
                     "step_frac": round(step_gbs / HBM_PEAK_GBS, 4)},
        "kernels_ms_per_step": {k: round(v, 5) for k, v in kern.items()},
        "step_hbm_gbs": round(step_gbs, 1),
        "wall_s": round(wall, 4),
    }
    legs = [] if args.no_tree else [x for x in args.legs.split(",") if x]
    known = {"chain_step_c1": chain_step_c1_leg, "tree_attention": tree_attention_leg,
             "w4a16_gemm": w4a16_gemm_leg,
             "tree_accept_commit": tree_accept_commit_leg, "verify_step_8b": verify_step_8b_leg}
    if legs:
        del sets
        torch.cuda.empty_cache()
    for name in legs:
        if name not in known:
            print(f"bench.py: unknown leg {name!r} (known: {sorted(known)})", file=sys.stderr)
            return 2
        line[name] = known[name](dev)
        torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        tl, dl, tok, U = make_inputs(dev, 1000)
        line["cpu_baseline"] = cpu_baseline(tl, dl, tok)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
