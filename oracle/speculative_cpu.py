"""CPU restatement of one chain speculative step (cudaforge/speculative.py:86-211).

TEST INFRASTRUCTURE ONLY: tests/ and bench.py's cpu_baseline leg use it as
the CPU path of the chain step; the product never imports it.

The same phases as the reference's python engine, on torch-CPU tensors:

1. K autoregressive draft forwards; each draws its token from
   softmax(last logits / T) with torch.multinomial (speculative.py:113-123);
2. one target forward over prompt + drafts; softmax of its last K+1 rows
   (speculative.py:136-145);
3. lock-step rejection sampling with the resample / top-p bonus rules
   (speculative.py:152-195) -- the C oracle's python_verify, fed fp32
   probabilities and uniforms [B, K+2] from the step's generator.

Returns the emitted tokens [B, num_accepted] and num_accepted (which counts
the resampled or bonus token, and reaches K + 1 after a rejection at the
last position, as the reference's does).
"""
from __future__ import annotations

from typing import Any, Optional

import numpy as np
import torch

from . import oracle as O


@torch.no_grad()
def chain_step(draft_runner: Any, target_runner: Any, input_ids: torch.Tensor, K: int,
               temperature: float = 1.0, top_p: float = 0.9,
               generator: Optional[torch.Generator] = None):
    T = max(temperature, 1e-5)
    ids = input_ids.clone()
    drafts, dprobs = [], []
    for _ in range(K):
        logits = draft_runner.forward(ids, None)[:, -1, :].float()
        p = torch.softmax(logits / T, dim=-1)
        tok = torch.multinomial(p, 1, generator=generator)
        drafts.append(tok)
        dprobs.append(p)
        ids = torch.cat([ids, tok], dim=-1)
    B, V = input_ids.shape[0], None
    tok = torch.cat(drafts, dim=-1) if K else input_ids.new_empty(B, 0)
    tlog = target_runner.forward(torch.cat([input_ids, tok], dim=-1), None)
    tp = torch.softmax(tlog[:, -(K + 1):, :].float() / T, dim=-1)
    V = tp.shape[-1]
    dp = torch.stack(dprobs, dim=1) if K else torch.zeros(B, 0, V)
    U = torch.rand(B, K + 2, generator=generator)
    n, ne, toks = O.python_verify(tp.numpy(), dp.numpy(), tok.to(torch.int32).numpy(),
                                  U.numpy(), top_p)
    return torch.from_numpy(np.ascontiguousarray(toks[:, :ne])).long(), ne
