"""Write golden vectors of the reference's python speculative engine.

Runs in the build container only, where /root/reference is mounted:

    python tests/golden/make_python_golden.py

It loads ``cudaforge/speculative.py`` from the reference tree by file path
(the package's ``__init__`` imports the CUDA extension, which is not built
here) and drives its ``SpeculativeEngine.step`` on the CPU with
``TableRunner`` runners (tests/golden/recipes.py).

``torch.multinomial`` cannot be fed uniforms, so for the duration of each
step three torch functions are replaced by recording stand-ins:

  rand_like(p_draft)    returns the next fed acceptance column (speculative.py:161)
                        and records p_draft, the draft probability at the token
  minimum(ones, ratio)  records the acceptance ratio the engine computed (:162-164)
  multinomial(w, 1)     records the weights w and returns fed_inverse_cdf(w, u)
                        (:119 draft draws, :182 resample, :84 bonus), with u the
                        next draft-draw column for the K draft forwards and the
                        next final-draw column afterwards

The engine's ``_sample_next_token`` is wrapped on the instance to tag the bonus
draws and record their temperature and top_p.  Empty inputs go to the real
``torch.multinomial``, so its behaviour on them is the reference's.

Outputs (committed; the tests read them, never the reference):
  python_engine.json  per case: shape, recipe, SHA-256 of the logit tables,
                      per step the result fields, lifetime totals, the
                      acceptance-test count, the kinds of the final draws
                      and any exception (type and message)
  python_engine.npz   per case and step: the fed uniforms, the drafted
                      tokens, p_draft and the ratios of every acceptance
                      test, accepted_tokens, the final draws' ids, weights
                      (small cases) and distances to the nearest CDF boundary
"""
from __future__ import annotations

import contextlib
import hashlib
import importlib.util
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from tests.golden.recipes import TableRunner, fed_inverse_cdf, python_step_case  # noqa: E402

REFERENCE = os.environ.get("CFA_REFERENCE", "/root/reference")
PROMPT_LEN = 3

# name, seed, B, K, V, steps, temperature, top_p, sigma, noise
RANDOM = [
    ("b1_k4_v32000", 11, 1, 4, 32000, 3, 1.0, 0.9, 2.0, 0.5),  # BASELINE configs[0] V, K, T
    ("b1_k8_p05", 12, 1, 8, 1000, 4, 0.7, 0.5, 2.0, 0.1),
    ("b1_k1_p10", 13, 1, 1, 1000, 6, 1.0, 1.0, 2.0, 0.5),
    ("b4_k4_p09", 14, 4, 4, 512, 4, 0.7, 0.9, 2.0, 0.2),
    ("b4_k8_p05", 15, 4, 8, 512, 3, 1.0, 0.5, 2.0, 0.1),
    ("b4_k1_p10", 16, 4, 1, 512, 4, 1.0, 1.0, 2.0, 0.5),
    ("b64_k8_p09", 17, 64, 8, 128, 3, 0.7, 0.9, 2.0, 0.01),
    ("b64_k4_p05", 18, 64, 4, 128, 3, 1.0, 0.5, 2.0, 0.02),
    ("b64_k1_p10", 19, 64, 1, 128, 3, 1.0, 1.0, 2.0, 0.5),
    ("b64_k8_c2", 20, 64, 8, 128, 2, 0.7, 0.9, 2.0, 0.5),
]
# engines whose step raises or sees an empty batch: name, B, K, V
DEGENERATE = [("k0_b1", 1, 0, 64), ("k0_b4", 4, 0, 64), ("b0_k4", 0, 4, 64)]
STORE_WEIGHTS_MAX = 65536  # final-draw weights are stored when B * V is at most this


def load_reference():
    path = os.path.join(REFERENCE, "cudaforge", "speculative.py")
    spec = importlib.util.spec_from_file_location("cudaforge_reference_speculative", path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod  # dataclasses resolve the module by name
    spec.loader.exec_module(mod)
    return mod


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


class FedDraws:
    """The recording stand-ins of one step (see the module docstring)."""

    def __init__(self, K: int, draft_u, acc_u, fin_u):
        self.K = K
        self.draft_u, self.acc_u, self.fin_u = draft_u, acc_u, fin_u
        self.p_draft, self.ratio = [], []
        self.finals = []  # (kind, weights, ids, margin)
        self.n_multinomial = 0
        self.in_bonus = False
        self.bonus_args = []

    @contextlib.contextmanager
    def installed(self, engine):
        real_rand_like, real_multinomial, real_minimum = (torch.rand_like, torch.multinomial,
                                                          torch.minimum)
        real_sample = engine._sample_next_token

        def rand_like(x, *a, **k):
            i = len(self.p_draft)
            self.p_draft.append(x.detach().clone().reshape(-1).numpy())
            col = torch.from_numpy(np.ascontiguousarray(self.acc_u[:, i]))
            return col.reshape(x.shape).to(x.dtype)

        def minimum(a, b, *args, **k):
            out = real_minimum(a, b, *args, **k)
            self.ratio.append(out.detach().clone().reshape(-1).numpy())
            return out

        def multinomial(w, num_samples, *a, **k):
            assert num_samples == 1 and not a and not k, "the engine draws one sample per row"
            if w.numel() == 0:
                return real_multinomial(w, num_samples)
            j = self.n_multinomial
            self.n_multinomial += 1
            wn = w.detach().to(torch.float32).numpy().copy()
            if j < self.K:  # the draft forwards (speculative.py:113-123)
                ids, _ = fed_inverse_cdf(wn, self.draft_u[:, j])
            else:
                f = len(self.finals)
                ids, margin = fed_inverse_cdf(wn, self.fin_u[:, f])
                self.finals.append(("bonus" if self.in_bonus else "resample", wn, ids, margin))
            return torch.from_numpy(ids).reshape(-1, 1)

        def sample_next_token(logits, temperature=1.0, top_p=0.9):
            self.in_bonus = True
            self.bonus_args.append([float(temperature), float(top_p)])
            try:
                return real_sample(logits, temperature=temperature, top_p=top_p)
            finally:
                self.in_bonus = False

        torch.rand_like, torch.multinomial, torch.minimum = rand_like, multinomial, minimum
        engine._sample_next_token = sample_next_token
        try:
            yield self
        finally:
            torch.rand_like, torch.multinomial, torch.minimum = (real_rand_like,
                                                                 real_multinomial, real_minimum)
            del engine._sample_next_token


def run_case(ref, name, dl, tl, ud, ua, uf, temperature, top_p, arrays):
    """Run len(dl) successive steps of one reference engine; record everything."""
    S, B, K, V = dl.shape
    draft, target = TableRunner(dl, draft=True), TableRunner(tl, draft=False)
    eng = ref.SpeculativeEngine(draft, target, num_speculative_tokens=K,
                                temperature=temperature, top_p=top_p)
    ids = torch.from_numpy(np.arange(B * PROMPT_LEN, dtype=np.int64).reshape(B, PROMPT_LEN) % V)
    steps = []
    for s in range(S):
        fed = FedDraws(K, ud[s], ua[s], uf[s])
        rec = {}
        try:
            with fed.installed(eng):
                res = eng.step(ids)
        except Exception as e:  # recorded, as the reference surfaces it
            rec["exception"] = [type(e).__name__, str(e)]
            res = None
        p = f"{name}__{s}__"
        arrays[p + "draft_u"] = ud[s]
        arrays[p + "acc_u"] = ua[s]
        arrays[p + "fin_u"] = uf[s]
        rec["n_tests"] = len(fed.p_draft)
        if fed.p_draft:
            arrays[p + "p_draft"] = np.stack(fed.p_draft).astype(np.float32)
            arrays[p + "ratio"] = np.stack(fed.ratio).astype(np.float32)
        rec["final_kinds"] = [f[0] for f in fed.finals]
        rec["bonus_args"] = fed.bonus_args
        if fed.finals:
            arrays[p + "final_ids"] = np.stack([f[2] for f in fed.finals])
            arrays[p + "final_margin"] = np.stack([f[3] for f in fed.finals])
            arrays[p + "final_wsum"] = np.stack([f[1].astype(np.float64).sum(-1)
                                                 for f in fed.finals])
            if B * V <= STORE_WEIGHTS_MAX:
                arrays[p + "final_weights"] = np.stack([f[1] for f in fed.finals])
        rec["draft_calls"] = draft.calls
        rec["target_calls"] = target.calls
        if res is not None:
            # the drafted tokens, as the target forward received them (:138)
            arrays[p + "draft_tokens"] = target.inputs[-1][:, PROMPT_LEN:].numpy()
            arrays[p + "accepted_tokens"] = res.accepted_tokens.numpy()
            rec.update(num_accepted=res.num_accepted,
                       draft_tokens_generated=res.draft_tokens_generated,
                       acceptance_rate=res.acceptance_rate,
                       accepted_shape=list(res.accepted_tokens.shape))
        rec.update(total_draft_tokens=eng.total_draft_tokens,
                   total_accepted_tokens=eng.total_accepted_tokens,
                   aggregate_rate=eng.get_aggregate_acceptance_rate())
        steps.append(rec)
    return steps


def probe_ratios(ref, dl, tl, ud, temperature, top_p):
    """Acceptance ratios [K, B] of one step, every test run (u = 0 accepts any
    ratio above 0)."""
    S, B, K, V = dl.shape
    fed = FedDraws(K, ud[0], np.zeros((B, K), np.float32), np.zeros((B, 2), np.float32))
    eng = ref.SpeculativeEngine(TableRunner(dl[:1], True), TableRunner(tl[:1], False),
                                num_speculative_tokens=K, temperature=temperature, top_p=top_p)
    with fed.installed(eng):
        eng.step(torch.zeros(B, PROMPT_LEN, dtype=torch.long))
    assert len(fed.ratio) == K
    return np.stack(fed.ratio)


def main() -> None:
    ref = load_reference()
    torch.manual_seed(0)
    meta, arrays = {}, {}

    for name, seed, B, K, V, S, T, top_p, sigma, noise in RANDOM:
        dl, tl, ud, ua, uf = python_step_case(seed, B, K, V, S, sigma=sigma, noise=noise)
        meta[name] = dict(kind="random", seed=seed, B=B, K=K, V=V, steps=S, temperature=T,
                          top_p=top_p, sigma=sigma, noise=noise,
                          sha256=digest(dl, tl),
                          step=run_case(ref, name, dl, tl, ud, ua, uf, T, top_p, arrays))

    # Known answer: the target probability of the drafted token is exactly 0
    # and the acceptance uniform is 0.  The python rule u < ratio (:166) rejects.
    B, K, V = 2, 2, 64
    dl = np.zeros((1, B, K, V), np.float32)
    dl[0, :, 0, 5] = 30.0
    dl[0, :, 1, 9] = 30.0
    tl = python_step_case(21, B, K, V, 1)[1]
    tl[0, 0, 0, 5] = -300.0  # exp underflows: probability exactly 0 in fp32
    ud = np.full((1, B, K), 0.5, np.float32)
    ua = np.zeros((1, B, K), np.float32)
    uf = np.full((1, B, 2), 0.25, np.float32)
    arrays["kat_zero_target__draft_logits"], arrays["kat_zero_target__target_logits"] = dl, tl
    meta["kat_zero_target"] = dict(kind="kat", B=B, K=K, V=V, steps=1, temperature=1.0,
                                   top_p=0.9, sha256=digest(dl, tl),
                                   step=run_case(ref, "kat_zero_target", dl, tl, ud, ua, uf,
                                                 1.0, 0.9, arrays))

    # Known answer: the draft row equals the target row, so the residual
    # max(0, t - d) is zero and the resample falls back to the target row
    # (:177-180).  The drafted token 0 has probability ~1e-6, so its ratio
    # p / (p + 1e-8) is ~0.99 and u just below 1 rejects it by a wide margin.
    B, K, V = 2, 2, 64
    tl = python_step_case(24, B, K, V, 1)[1]
    tl[:, :, :, :4] = -9.0
    dl = np.ascontiguousarray(tl[:, :, :K])
    ud = np.full((1, B, K), 0.5, np.float32)
    ud[:, :, 0] = 1e-7
    ua = np.full((1, B, K), np.nextafter(np.float32(1), np.float32(0)), np.float32)
    uf = np.full((1, B, 2), 0.75, np.float32)
    arrays["kat_fallback__draft_logits"], arrays["kat_fallback__target_logits"] = dl, tl
    meta["kat_fallback"] = dict(kind="kat", B=B, K=K, V=V, steps=1, temperature=1.0, top_p=0.9,
                                sha256=digest(dl, tl),
                                step=run_case(ref, "kat_fallback", dl, tl, ud, ua, uf, 1.0, 0.9,
                                              arrays))

    # Known answers at the ratio: u equal to the ratio the reference computed
    # rejects (strict <); one fp32 ulp below accepts; one above rejects.
    B, K, V, T, top_p = 4, 4, 256, 1.0, 0.9
    dl1, tl1, ud1, _, _ = python_step_case(22, B, K, V, 1, noise=0.5)
    ratio = probe_ratios(ref, dl1, tl1, ud1, T, top_p)
    plan = []
    for i_star in (K - 1, 1):
        below = np.flatnonzero(ratio[i_star] < 1.0)
        assert below.size, "the probe found no ratio below 1 at that position"
        b_star = int(below[0])
        r = np.float32(ratio[i_star, b_star])
        for u in (r, np.nextafter(r, np.float32(0)), np.nextafter(r, np.float32(1))):
            plan.append((i_star, b_star, u))
    S = len(plan)
    dl, tl = np.repeat(dl1, S, 0), np.repeat(tl1, S, 0)
    ud = np.repeat(ud1, S, 0)
    ua = np.zeros((S, B, K), np.float32)
    for s, (i_star, b_star, u) in enumerate(plan):
        ua[s, b_star, i_star] = u
    uf = np.random.default_rng(23).random((S, B, 2)).astype(np.float32)
    arrays["kat_u_at_ratio__draft_logits"], arrays["kat_u_at_ratio__target_logits"] = dl, tl
    meta["kat_u_at_ratio"] = dict(kind="kat", B=B, K=K, V=V, steps=S, temperature=T, top_p=top_p,
                                  sha256=digest(dl, tl), plan=[[i, b] for i, b, _ in plan],
                                  step=run_case(ref, "kat_u_at_ratio", dl, tl, ud, ua, uf, T,
                                                top_p, arrays))

    for name, B, K, V in DEGENERATE:
        dl, tl, ud, ua, uf = python_step_case(30 + B + K, B, K, V, 1)
        arrays[name + "__draft_logits"], arrays[name + "__target_logits"] = dl, tl
        meta[name] = dict(kind="degenerate", B=B, K=K, V=V, steps=1, temperature=1.0, top_p=0.9,
                          sha256=digest(dl, tl),
                          step=run_case(ref, name, dl, tl, ud, ua, uf, 1.0, 0.9, arrays))

    with open(os.path.join(HERE, "python_engine.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)
    np.savez_compressed(os.path.join(HERE, "python_engine.npz"), **arrays)
    for name, m in meta.items():
        print(name, [(st.get("num_accepted"), st.get("final_kinds"), st.get("exception"))
                     for st in m["step"]])


if __name__ == "__main__":
    main()
