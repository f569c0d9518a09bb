"""Tree data structure and DFS packing — drop-in for dfs_tree_forward.py Parts 1-2.

``TreeNode`` keeps the reference's fields and methods (dfs_tree_forward.py:46-65).
``build_dfs_tree_info`` keeps its signature and ``DFSTreeInfo`` its fields
(dfs_tree_forward.py:72-184), but the per-token work moves to the GPU: the host
walks the forest once in DFS pre-order (O(nodes) plus the token-id
concatenation), and the HIP metadata kernel produces the depth-based positions
and subtree horizons. ``dfs_pos_ids`` and the dense ``attn_mask_bool`` are
materialised on the host only when read, for compatibility; the attention path
never builds the [N, N] mask.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Sequence, Tuple

import torch


@dataclass
class TreeNode:
    """One node of the generation tree (dfs_tree_forward.py:46-65).

    token_ids : token IDs of this node
    children  : child nodes; empty = leaf
    """
    token_ids: List[int]
    children: List["TreeNode"] = field(default_factory=list)

    def add_child(self, token_ids: List[int]) -> "TreeNode":
        child = TreeNode(token_ids)
        self.children.append(child)
        return child

    @property
    def is_leaf(self) -> bool:
        return len(self.children) == 0


def flatten(roots) -> Tuple[List[int], List[int], list]:
    """DFS pre-order over a forest (parent before children, children left to
    right, dfs_tree_forward.py:113-139). Iterative, so depth is unbounded.
    Returns (node_len, parent, nodes)."""
    node_len: List[int] = []
    parent: List[int] = []
    nodes: list = []
    for root in roots:
        stack = [(root, -1)]
        while stack:
            node, par = stack.pop()
            me = len(nodes)
            nodes.append(node)
            node_len.append(len(node.token_ids))
            parent.append(par)
            for ch in reversed(node.children):
                stack.append((ch, me))
    return node_len, parent, nodes


class DFSTreeInfo:
    """Everything one DFS tree forward needs (dfs_tree_forward.py:72-88).

    Host fields are plain Python (token ids, chunk boundaries, parent map, leaf
    ids and nodes, sizes, per-node depth offsets). Device metadata (positions,
    horizons, tile plan inputs) is built by the HIP kernel on first use and
    cached per (device, pos_offset).
    """

    def __init__(self, dfs_token_ids, chunk_boundaries, chunk_parent_map, leaf_chunk_ids, leaf_nodes,
                 node_len, node_off, nodes):
        self.dfs_token_ids: List[int] = dfs_token_ids
        self.chunk_boundaries: List[Tuple[int, int]] = chunk_boundaries
        self.chunk_parent_map: List[int] = chunk_parent_map
        self.leaf_chunk_ids: List[int] = leaf_chunk_ids
        self.leaf_nodes: list = leaf_nodes
        self.node_len: List[int] = node_len
        self.node_off: List[int] = node_off     # depth offset (position of a node's first token)
        self.nodes: list = nodes
        self.N: int = len(dfs_token_ids)
        self.n_chunks: int = len(chunk_parent_map)
        self._meta = {}
        self._pos_cache = None
        self._mask_cache = None

    # -- device metadata ---------------------------------------------------
    def device_meta(self, device=None, pos_offset: int = 0):
        """TreeMetaDevice for this forest (built once per device/offset)."""
        from .meta import TreeMetaDevice, require_device
        dev = require_device(device)
        key = (str(dev), int(pos_offset))
        if key not in self._meta:
            self._meta[key] = TreeMetaDevice(self.node_len, self.chunk_parent_map, pos_offset=pos_offset,
                                             device=dev)
        return self._meta[key]

    def key_plan(self, device=None, past_bias: Optional[torch.Tensor] = None, pos_offset: int = 0):
        from .meta import KeyPlan
        return KeyPlan(self.device_meta(device, pos_offset).horizon, past_bias,
                       topo=(self.node_len, self.chunk_parent_map))

    # -- compatibility views (host copies, built on access) -------------------
    @property
    def dfs_pos_ids(self) -> List[int]:
        """Depth-based position ids (dfs_tree_forward.py:125-126), from the GPU."""
        if self._pos_cache is None:
            self._pos_cache = self.device_meta().pos.cpu().tolist()
        return self._pos_cache

    @property
    def attn_mask_bool(self) -> torch.Tensor:
        """Dense [N, N] CPU bool mask (dfs_tree_forward.py:161-172), expanded on
        the GPU from the horizons; compatibility only."""
        if self._mask_cache is None:
            self._mask_cache = self.key_plan().dense_mask().cpu()
        return self._mask_cache


def preorder_violation(parent: Sequence[int]) -> Optional[int]:
    """First node index whose parent list position breaks DFS pre-order, or
    None. ``parent[i] < i`` is necessary but not sufficient: in pre-order every
    node between a parent and its child is a descendant of that parent, i.e.
    the parent is still on the open root-to-node path when the child comes."""
    path: List[int] = []
    for i, p in enumerate(parent):
        p = int(p)
        if p < -1 or p >= i:
            return i
        while path and path[-1] != p:
            path.pop()
        if p >= 0 and not path:
            return i
        path.append(i)
    return None


def info_from_flat(node_len: List[int], parent: List[int], nodes: list) -> DFSTreeInfo:
    """DFSTreeInfo from an already flattened DFS pre-order forest."""
    if not nodes:
        raise ValueError("build_dfs_tree_info: empty forest")
    dfs_token_ids: List[int] = []
    bounds: List[Tuple[int, int]] = []
    node_off: List[int] = []
    leaf_ids, leaf_nodes = [], []
    start = 0
    for c, (node, L, p) in enumerate(zip(nodes, node_len, parent)):
        if L < 1:
            raise ValueError(f"TreeNode #{c} in DFS order has no tokens; empty nodes are not supported")
        dfs_token_ids.extend(node.token_ids)
        bounds.append((start, start + L))
        node_off.append(node_off[p] + node_len[p] if p >= 0 else 0)
        if c + 1 >= len(nodes) or parent[c + 1] != c:   # no child follows in pre-order
            leaf_ids.append(c)
            leaf_nodes.append(node)
        start += L
    return DFSTreeInfo(dfs_token_ids, bounds, list(parent), leaf_ids, leaf_nodes, list(node_len), node_off,
                       nodes)


def build_dfs_tree_info(roots: List[TreeNode]) -> DFSTreeInfo:
    """Convert a forest into a DFSTreeInfo (dfs_tree_forward.py:91-184).

    DFS pre-order (chunk_parent_map[i] < i); depth-based positions
    (ancestor tokens + offset in node). Raises ValueError for an empty node
    (it would own no token and break the packed layout).
    """
    return info_from_flat(*flatten(roots))
