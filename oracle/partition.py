"""Oracle: greedy partitioning and gateway metadata (test infrastructure only).

Restates tree_grad_hybrid.py:48-153 (``partition_tree``,
``_dfs_info_for_partition``) and the integer part of ``_make_child_gateways``
(tree_grad_hybrid.py:174-209: total length, additive bias and depth offset).

Two bias modes:
  * ``legacy=True`` reproduces the reference literally: the whole inherited
    parent gateway is visible (tree_grad_hybrid.py:207, ``bias[:parent_past_len] = 0``);
  * ``legacy=False`` inherits the parent gateway's own bias, so a chain of
    partitions sees exactly the ancestors of the cut node (the whole-tree mask).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional

from .tree_meta import build_dfs_tree_info_literal


@dataclass
class OraclePartition:
    entry_nodes: list
    dfs_nodes: list = field(default_factory=list)
    cut_node_set: set = field(default_factory=set)
    leaf_node_set: set = field(default_factory=set)
    parent: Optional["OraclePartition"] = None
    parent_cut_node: object = None
    token_count: int = 0


def partition_tree_literal(roots, max_tokens) -> List[OraclePartition]:
    """tree_grad_hybrid.py:60-95 — greedy DFS partitioning, creation order."""
    partitions: List[OraclePartition] = []

    def _build(entry, parent, parent_cut_node):
        p = OraclePartition(entry_nodes=entry, parent=parent, parent_cut_node=parent_cut_node)
        partitions.append(p)
        deferred = []

        def _dfs(node, is_entry):
            L = len(node.token_ids)
            if not is_entry and p.token_count > 0 and p.token_count + L > max_tokens:   # :76
                return False
            p.dfs_nodes.append(node)
            p.token_count += L
            for child in node.children:
                if not _dfs(child, False):                                               # :80-83
                    p.cut_node_set.add(id(node))
                    deferred.append((node, child))
            if not node.children and id(node) not in p.cut_node_set:
                p.leaf_node_set.add(id(node))
            return True

        for r in entry:
            _dfs(r, True)
        for cut_node, cut_child in deferred:                                            # :90-91
            _build([cut_child], p, cut_node)

    for root in roots:                                                                  # :93-94
        _build([root], None, None)
    return partitions


class _Copy:
    __slots__ = ("token_ids", "children")

    def __init__(self, token_ids):
        self.token_ids = list(token_ids)
        self.children = []


def dfs_info_for_partition(partition: OraclePartition):
    """tree_grad_hybrid.py:102-153 — DFS info of the in-partition subtree.

    Returns (info, start, end, par, chunk_idx) where the maps are keyed by id()
    of the original nodes.
    """
    in_part = {id(n) for n in partition.dfs_nodes}
    copies, copy_to_orig = {}, {}

    def _copy(orig):
        if id(orig) in copies:
            return copies[id(orig)]
        c = _Copy(orig.token_ids)
        copies[id(orig)] = c
        copy_to_orig[id(c)] = orig
        for ch in orig.children:
            if id(ch) in in_part:
                c.children.append(_copy(ch))
        return c

    entry_copies = [_copy(n) for n in partition.entry_nodes if id(n) in in_part]
    info = build_dfs_tree_info_literal(entry_copies)
    start, end, par, cidx = {}, {}, {}, {}
    ci = [0]

    def _walk(cn, par_orig):
        idx = ci[0]
        ci[0] += 1
        s, e = info["chunk_boundaries"][idx]
        orig = copy_to_orig[id(cn)]
        start[id(orig)], end[id(orig)] = s, e
        par[id(orig)] = par_orig
        cidx[id(orig)] = idx
        for ch in cn.children:
            _walk(ch, id(orig))

    for ec in entry_copies:
        _walk(ec, -1)
    info["copy_to_orig"] = copy_to_orig
    return info, start, end, par, cidx


def gateway_meta(info, start, end, par, cut_node, parent_pos_offset,
                 parent_past_len, parent_bias=None, legacy=True):
    """tree_grad_hybrid.py:193-209 — (total, bias list, pos_off) for one cut node.

    ``parent_bias`` is the parent partition's own gateway bias (length
    ``parent_past_len``); it is only read when ``legacy`` is False.
    """
    cut_end = end[id(cut_node)]
    total = parent_past_len + cut_end
    cn_start = start[id(cut_node)]
    pos_off = parent_pos_offset + info["dfs_pos_ids"][cn_start] + len(cut_node.token_ids)
    bias = [-math.inf] * total
    if legacy or parent_bias is None:
        for t in range(parent_past_len):
            bias[t] = 0.0
    else:
        for t in range(parent_past_len):
            bias[t] = parent_bias[t]
    nid = id(cut_node)
    while nid != -1 and nid in start:
        s, e = start[nid], end[nid]
        for t in range(parent_past_len + s, parent_past_len + e):
            bias[t] = 0.0
        nid = par.get(nid, -1)
    return total, bias, pos_off


def hybrid_schedule(roots, max_tokens, legacy=True):
    """Top-down walk of tree_grad_hybrid.py:453-499 without a model.

    Returns a list of per-partition dicts (creation order) with the partition,
    its DFS info, its gateway (total, bias, pos_off) or None, and its
    ``pos_offset``.
    """
    parts = partition_tree_literal(roots, max_tokens)
    children_of = {id(p): [] for p in parts}
    for p in parts:
        if p.parent is not None:
            children_of[id(p.parent)].append((p.parent_cut_node, p))
    gw_of = {}
    out = []
    for p in parts:
        gw = gw_of.get(id(p))
        pos_offset = gw["pos_off"] if gw is not None else 0
        info, start, end, par, cidx = dfs_info_for_partition(p)
        out.append(dict(partition=p, info=info, gateway=gw, pos_offset=pos_offset,
                        start=start, end=end, par=par))
        seen = {}
        for cn, child in children_of[id(p)]:
            if id(cn) not in seen:
                total, bias, pos_off = gateway_meta(
                    info, start, end, par, cn, pos_offset,
                    gw["total"] if gw is not None else 0,
                    gw["bias"] if gw is not None else None, legacy=legacy)
                seen[id(cn)] = dict(total=total, bias=bias, pos_off=pos_off, cut=cn)
            gw_of[id(child)] = seen[id(cn)]
    return out
