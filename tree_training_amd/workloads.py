"""Synthetic DFS-packed tree topologies used by the benchmark and the tests.

A topology is ``(node_len, parent)`` in DFS pre-order (parent < child, -1 for
a root), the same flattening ``build_dfs_tree_info`` performs
(dfs_tree_forward.py:113-139). Generators are seeded with ``random.Random`` so a
topology depends only on its arguments.
"""
from __future__ import annotations

import random
from typing import List, Tuple

Topology = Tuple[List[int], List[int]]


def agent_tree(seed: int = 0, depth: int = 6, branch=(2, 4), node_len=(64, 512),
               max_tokens: int = 16384) -> Topology:
    """Agent-trajectory tree: root at depth 1, leaves at depth ``depth``,
    branching uniform in ``branch``, node lengths uniform in ``node_len``.
    Generation (depth-first) stops before the first node that would push the
    packed length past ``max_tokens``."""
    rng = random.Random(seed)
    lens: List[int] = []
    par: List[int] = []
    state = {"total": 0, "stop": False}

    def grow(p: int, d: int):
        if state["stop"]:
            return
        L = rng.randint(*node_len)
        if state["total"] + L > max_tokens:
            state["stop"] = True
            return
        me = len(lens)
        lens.append(L)
        par.append(p)
        state["total"] += L
        if d < depth:
            for _ in range(rng.randint(*branch)):
                grow(me, d + 1)

    grow(-1, 1)
    return lens, par


def rollout_tree(seed: int = 0, prompt_len: int = 8192, n_leaves: int = 64,
                 leaf_len=(256, 1024)) -> Topology:
    """GRPO-style rollout: one shared prompt node with ``n_leaves`` leaves."""
    rng = random.Random(seed)
    lens = [prompt_len] + [rng.randint(*leaf_len) for _ in range(n_leaves)]
    par = [-1] + [0] * n_leaves
    return lens, par


def random_forest(seed: int, n_roots=(1, 3), max_depth: int = 5, max_branch: int = 3,
                  node_len=(1, 40)) -> Topology:
    """Small irregular forests for parity sweeps (any lengths, leaves at any depth)."""
    rng = random.Random(seed)
    lens: List[int] = []
    par: List[int] = []

    def grow(p: int, d: int):
        me = len(lens)
        lens.append(rng.randint(*node_len))
        par.append(p)
        if d < max_depth:
            for _ in range(rng.randint(0, max_branch)):
                grow(me, d + 1)

    for _ in range(rng.randint(*n_roots)):
        grow(-1, 1)
    return lens, par


def visible_pairs(topo: Topology) -> int:
    """P = sum over tokens of (depth position + 1): the useful (query, key)
    pairs per head of a DFS-packed tree."""
    lens, par = topo
    off = [0] * len(lens)
    P = 0
    for c, (L, p) in enumerate(zip(lens, par)):
        off[c] = off[p] + lens[p] if p >= 0 else 0
        P += L * off[c] + L * (L + 1) // 2
    return P


def forest_from_topology(topo: Topology, node_cls, vocab: int = 1000, seed: int = 0):
    """TreeNode forest with seeded random token ids; returns (roots, nodes)."""
    rng = random.Random(seed)
    lens, par = topo
    nodes, roots = [], []
    for L, p in zip(lens, par):
        ids = [rng.randrange(1, vocab) for _ in range(L)]
        if p < 0:
            n = node_cls(ids)
            roots.append(n)
        else:
            n = nodes[p].add_child(ids)
        nodes.append(n)
    return roots, nodes
