"""Loader of the python-engine golden vectors (python_engine.json / .npz).

The vectors were written by make_python_golden.py from the reference's own
``cudaforge/speculative.py`` run in the build container; this module only
reads them back and regenerates the logit tables from their recipes,
checking each table's SHA-256.
"""
from __future__ import annotations

import hashlib
import json
import os
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np

from .recipes import python_step_case

HERE = os.path.dirname(os.path.abspath(__file__))

# Draws whose uniform lies closer than this to a boundary of the fp64 CDF of
# the reference's weights are left out of id comparisons: the kernel and the
# oracle form their CDFs in fp32 from probabilities that differ from torch's
# by rounding.
TIE_MARGIN = 1e-5


@dataclass
class Step:
    rec: dict
    arrays: Dict[str, np.ndarray]

    def __getitem__(self, k):
        return self.arrays[k]

    def get(self, k, default=None):
        return self.arrays.get(k, default)

    @property
    def exception(self) -> Optional[List[str]]:
        return self.rec.get("exception")

    @property
    def n_accepted_drafts(self) -> int:
        """Drafts accepted: every acceptance test passed, or all but the last."""
        return self.rec["n_tests"] - (1 if "resample" in self.rec["final_kinds"] else 0)

    def uniforms(self) -> np.ndarray:
        """The step's draws in the kernel's python-mode layout [B, K+2]: the K
        acceptance draws, then the first and second final draws."""
        return np.concatenate([self["acc_u"], self["fin_u"]], axis=1).astype(np.float32)


@dataclass
class Case:
    name: str
    meta: dict
    draft_logits: np.ndarray   # [S, B, K, V]
    target_logits: np.ndarray  # [S, B, K+1, V]
    steps: List[Step] = field(default_factory=list)

    @property
    def B(self): return self.meta["B"]

    @property
    def K(self): return self.meta["K"]

    @property
    def V(self): return self.meta["V"]

    @property
    def temperature(self): return self.meta["temperature"]

    @property
    def top_p(self): return self.meta["top_p"]


def _digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def load(kinds=None) -> List[Case]:
    with open(os.path.join(HERE, "python_engine.json")) as f:
        meta = json.load(f)
    z = np.load(os.path.join(HERE, "python_engine.npz"))
    cases = []
    for name in sorted(meta):
        m = meta[name]
        if kinds is not None and m["kind"] not in kinds:
            continue
        if m["kind"] == "random":
            dl, tl = python_step_case(m["seed"], m["B"], m["K"], m["V"], m["steps"],
                                      sigma=m["sigma"], noise=m["noise"])[:2]
        else:
            dl, tl = z[f"{name}__draft_logits"], z[f"{name}__target_logits"]
        assert _digest(dl, tl) == m["sha256"], f"{name}: the logit recipe changed"
        case = Case(name, m, dl, tl)
        for s, rec in enumerate(m["step"]):
            pre = f"{name}__{s}__"
            arrays = {k[len(pre):]: z[k] for k in z.files if k.startswith(pre)}
            case.steps.append(Step(rec, arrays))
        cases.append(case)
    return cases


def final_columns(step: Step, n: int):
    """(column of the emitted tokens, reference id per row, comparable mask) for
    each final draw: the resample or bonus at column n, a second bonus at n+1."""
    out = []
    for f, kind in enumerate(step.rec["final_kinds"]):
        out.append((n + f, kind, step["final_ids"][f], step["final_margin"][f] >= TIE_MARGIN))
    return out


def knife_edge(step: Step, gap: float = 1e-5) -> bool:
    """Whether some acceptance test the reference ran had its uniform within
    `gap` of a positive ratio: a path that forms the probabilities itself (the
    kernel's fused softmax) may decide such a test either way.  A ratio of
    exactly 0 (a target probability that underflows to 0) is 0 on every path."""
    for i in range(step.rec["n_tests"]):
        r = step["ratio"][i].astype(np.float64)
        gaps = np.abs(step["acc_u"][:, i].astype(np.float64) - r)
        if ((r > 0) & (gaps < gap)).any():
            return True
    return False


def bonus_comparable(case: Case, s: int, ids: np.ndarray, margin: np.ndarray,
                     gap: float = 1e-5) -> np.ndarray:
    """Rows [B] whose bonus id another path must reproduce exactly.

    Paths that form the top-p cumsum in another precision may keep or drop
    the tokens whose mass-above lies within `gap` of top_p (set A).  Changing
    A moves every boundary of the renormalised CDF by at most the mass of A
    over the kept mass, so a draw is fixed when its uniform is farther than
    that (plus TIE_MARGIN) from its boundaries and the drawn token is not in A."""
    if not case.top_p < 1.0:
        return margin >= TIE_MARGIN
    T = max(case.temperature, 1e-5)
    x = case.target_logits[s][:, case.K].astype(np.float64) / T
    p = np.exp(x - x.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ok = np.zeros(case.B, bool)
    for b in range(case.B):
        order = np.argsort(-p[b], kind="stable")
        ps = p[b, order]
        above = np.cumsum(ps) - ps
        near = np.abs(above - case.top_p) < gap
        kept = ps[above <= case.top_p].sum()
        extra = ps[near].sum() / kept
        ok[b] = margin[b] >= TIE_MARGIN + extra and ids[b] not in set(order[near].tolist())
    return ok
