"""Draft-token trees: topology helpers shared by tree attention, tree
acceptance and KV commit.

A tree of N <= 64 nodes is numbered so that parent[i] < i (node 0 is the
root, whose token is the last verified token).  Its ancestor mask holds, for
node i, bit j set iff j is an ancestor of i or i itself; tree attention lets
node i see tree position j exactly when that bit is set.  Node i's position
id for rotary embeddings is ctx_len + depth(i) (the tree's own K/V slots are
ctx_len + i in BFS order; the position id is a property of the token, the slot
is a property of the cache).
"""
from __future__ import annotations

from typing import Sequence

import numpy as np
import torch


def binary_tree_parents(n_nodes: int) -> np.ndarray:
    """BFS-numbered complete binary tree: parent(i) = (i - 1) >> 1, parent(0) = -1."""
    p = (np.arange(n_nodes) - 1) >> 1
    p[0] = -1
    return p.astype(np.int32)


def chain_parents(n_nodes: int) -> np.ndarray:
    """A chain (the reference's K-token speculation): parent(i) = i - 1."""
    p = np.arange(n_nodes) - 1
    return p.astype(np.int32)


def validate_parents(parent: Sequence[int]) -> np.ndarray:
    p = np.asarray(parent, dtype=np.int64).reshape(-1)
    n = p.size
    if n == 0 or n > 64:
        raise ValueError("a tree has 1..64 nodes")
    if p[0] != -1:
        raise ValueError("node 0 must be the root (parent -1)")
    if n > 1 and not np.all((p[1:] >= 0) & (p[1:] < np.arange(1, n))):
        raise ValueError("every non-root node needs a parent with a smaller index")
    return p.astype(np.int32)


def ancestor_masks(parent: Sequence[int]) -> np.ndarray:
    """uint64 per node: bit j set iff j is an ancestor of i or i itself."""
    p = validate_parents(parent)
    m = np.zeros(p.size, np.uint64)
    for i in range(p.size):
        bits = np.uint64(1) << np.uint64(i)
        if p[i] >= 0:
            bits |= m[p[i]]
        m[i] = bits
    return m


def depths(parent: Sequence[int]) -> np.ndarray:
    p = validate_parents(parent)
    d = np.zeros(p.size, np.int32)
    for i in range(1, p.size):
        d[i] = d[p[i]] + 1
    return d


def mask_tensor(masks: np.ndarray, device) -> torch.Tensor:
    """Ancestor masks as an int64 device tensor with the same 64 bits."""
    return torch.from_numpy(np.ascontiguousarray(masks).view(np.int64)).to(device)
