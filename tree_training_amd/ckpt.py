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

from .dfs_tree_forward import fused_ce_capable, run_tree_model
from .loss import TreeCELoss
from .tree import DFSTreeInfo, TreeNode, build_dfs_tree_info


def _build_retain_schedule(info: DFSTreeInfo, leaf_nodes: List[TreeNode]) -> List[bool]:
    """retain_graph for every leaf backward except the last (tree_grad_ckpt.py:169-186)."""
    n = len(leaf_nodes)
    return [True] * (n - 1) + [False]


def tree_grad_ckpt_sequential(model, roots: List[TreeNode],
                              leaf_loss_fn: Callable[[torch.Tensor, TreeNode], torch.Tensor],
                              fused_leaf_ce: bool = True) -> None:
    """Tree forward + sequential per-leaf backward; grads accumulate in ``.grad``.

    With a ``make_tree_loss_fn`` loss (and ``fused_leaf_ce``) the leaf losses
    come from the final hidden states through the chunked lm_head + fused
    cross-entropy (``loss.fused_linear_ce``, no [T, V] logits), summed over the
    leaves and back-propagated once (the same gradients up to summation order)."""
    dev = next(model.parameters()).device
    info = build_dfs_tree_info(roots)
    spans = [info.chunk_boundaries[c] for c in info.leaf_chunk_ids]
    schedule = _build_retain_schedule(info, info.leaf_nodes)
    if fused_leaf_ce and fused_ce_capable(model, leaf_loss_fn):
        hidden = run_tree_model(model, info, dev, hidden_only=True).last_hidden_state
        leaf_loss_fn.fused_spans(hidden[0], [(s, e, n) for (s, e), n in zip(spans, info.leaf_nodes)],
                                 model.lm_head.weight).backward()
        return
    logits = run_tree_model(model, info, dev).logits
    for (s, e), node, retain in zip(spans, info.leaf_nodes, schedule):
        leaf_loss_fn(logits[:, s:e, :], node).backward(retain_graph=retain)


def make_tree_loss_fn(leaf_labels: List[torch.Tensor], leaf_nodes: List[TreeNode], n_leaves: int,
                      ignore_index: int = -100) -> TreeCELoss:
    """CE(logits[0], labels, ignore_index) / n_leaves per leaf (tree_grad_ckpt.py:279-297)."""
    return TreeCELoss(leaf_labels, leaf_nodes, n_leaves, ignore_index)


tree_grad_ckpt_backward = tree_grad_ckpt_sequential
