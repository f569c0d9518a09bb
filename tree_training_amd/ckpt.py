"""Whole-tree forward + per-leaf backward — drop-in for tree_grad_ckpt.py.

``tree_grad_ckpt_sequential`` (tree_grad_ckpt.py:193-261) runs one forward over
the whole DFS-packed forest, then one backward per leaf in DFS order with
``retain_graph`` for all but the last leaf (tree_grad_ckpt.py:169-186). The
attention backward therefore runs once per leaf with that leaf's partial
upstream gradient, which the tree-attention autograd node supports.
"""
from __future__ import annotations

from typing import Callable, List

import torch
import torch.nn.functional as F

from .dfs_tree_forward import run_tree_model
from .tree import DFSTreeInfo, TreeNode, build_dfs_tree_info


def _build_retain_schedule(info: DFSTreeInfo, leaf_nodes: List[TreeNode]) -> List[bool]:
    """retain_graph for every leaf backward except the last (tree_grad_ckpt.py:169-186)."""
    n = len(leaf_nodes)
    return [True] * (n - 1) + [False]


def tree_grad_ckpt_sequential(model, roots: List[TreeNode],
                              leaf_loss_fn: Callable[[torch.Tensor, TreeNode], torch.Tensor]) -> None:
    """Tree forward + sequential per-leaf backward; grads accumulate in ``.grad``."""
    dev = next(model.parameters()).device
    info = build_dfs_tree_info(roots)
    logits = run_tree_model(model, info, dev).logits
    leaf_logits = [logits[:, s:e, :] for s, e in (info.chunk_boundaries[c] for c in info.leaf_chunk_ids)]
    for lg, node, retain in zip(leaf_logits, info.leaf_nodes, _build_retain_schedule(info, info.leaf_nodes)):
        leaf_loss_fn(lg, node).backward(retain_graph=retain)


def make_tree_loss_fn(leaf_labels: List[torch.Tensor], leaf_nodes: List[TreeNode], n_leaves: int,
                      ignore_index: int = -100) -> Callable:
    """CE(logits[0], labels, ignore_index) / n_leaves per leaf (tree_grad_ckpt.py:279-297)."""
    label_map = {id(n): lab for n, lab in zip(leaf_nodes, leaf_labels)}

    def _loss_fn(logits: torch.Tensor, node: TreeNode) -> torch.Tensor:
        labels = label_map[id(node)].to(logits.device)
        return F.cross_entropy(logits[0], labels, ignore_index=ignore_index) / n_leaves

    return _loss_fn


tree_grad_ckpt_backward = tree_grad_ckpt_sequential
