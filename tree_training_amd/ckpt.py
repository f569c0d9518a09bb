"""Whole-tree forward + per-leaf backward — drop-in for tree_grad_ckpt.py.

``tree_grad_ckpt_sequential`` (tree_grad_ckpt.py:193-261) runs one forward over
the whole DFS-packed forest, then one backward per leaf in DFS order with
``retain_graph`` for all but the last leaf (tree_grad_ckpt.py:169-186). The
attention backward therefore runs once per leaf with that leaf's partial
upstream gradient, which the tree-attention autograd node supports.
Gated-delta-rule layers of hybrid models (Qwen3.5) run the tree-aware conv and
scan (``gdn_layer._patch_ssm``) for the whole forward and backward, as in
``dfs_tree_forward``: the reference offers this driver for "any HF causal LM
(Qwen3, Qwen3.5, etc.)" (tree_grad_ckpt.py:222) but runs the stock GDN there,
which carries the recurrent state across sibling branches of the DFS order.
"""
from __future__ import annotations

from typing import Callable, List

import torch
import torch.nn.functional as F

from .dfs_tree_forward import fused_ce_capable, literal_options, run_tree_model
from .loss import TreeCELoss
from .tree import DFSTreeInfo, TreeNode, build_dfs_tree_info


def _build_retain_schedule(info: DFSTreeInfo, leaf_nodes: List[TreeNode]) -> List[bool]:
    """retain_graph for every leaf backward except the last (tree_grad_ckpt.py:169-186)."""
    n = len(leaf_nodes)
    return [True] * (n - 1) + [False]


def tree_grad_ckpt_sequential(model, roots: List[TreeNode],
                              leaf_loss_fn: Callable[[torch.Tensor, TreeNode], torch.Tensor],
                              fused_leaf_ce: bool = True, gdn_reference_truncated: bool = False,
                              gdn_per_node_projections: bool = False, fused_prologue: bool = True,
                              reference_literal: bool = False) -> None:
    """Tree forward + sequential per-leaf backward; grads accumulate in ``.grad``.

    With a ``make_tree_loss_fn`` loss (and ``fused_leaf_ce``) the leaf losses
    come from the final hidden states through the chunked lm_head + fused
    cross-entropy (``loss.fused_linear_ce``, no [T, V] logits), summed over the
    leaves and back-propagated once (the same gradients up to summation order).
    ``gdn_reference_truncated`` / ``gdn_per_node_projections`` /
    ``fused_prologue`` as in ``dfs_tree_forward``; ``reference_literal`` sets
    every option to the reference's arithmetic (``literal_options``)."""
    o = literal_options(reference_literal, fused_leaf_ce=fused_leaf_ce,
                        gdn_reference_truncated=gdn_reference_truncated,
                        gdn_per_node_projections=gdn_per_node_projections, fused_prologue=fused_prologue)
    dev = next(model.parameters()).device
    info = build_dfs_tree_info(roots)
    spans = [info.chunk_boundaries[c] for c in info.leaf_chunk_ids]
    schedule = _build_retain_schedule(info, info.leaf_nodes)
    from .gdn_layer import _patch_ssm, _unpatch_ssm
    saved = _patch_ssm(model, info.chunk_boundaries, info.chunk_parent_map, o["gdn_reference_truncated"],
                       o["gdn_per_node_projections"])
    run = dict(linear_attention_patched=True, fused_prologue=o["fused_prologue"])
    try:
        if o["fused_leaf_ce"] and fused_ce_capable(model, leaf_loss_fn):
            hidden = run_tree_model(model, info, dev, hidden_only=True, **run).last_hidden_state
            leaf_loss_fn.fused_spans(hidden[0], [(s, e, n) for (s, e), n in zip(spans, info.leaf_nodes)],
                                     model.lm_head.weight).backward()
            return
        logits = run_tree_model(model, info, dev, **run).logits
        for (s, e), node, retain in zip(spans, info.leaf_nodes, schedule):
            leaf_loss_fn(logits[:, s:e, :], node).backward(retain_graph=retain)
    finally:
        _unpatch_ssm(saved)


def make_tree_loss_fn(leaf_labels: List[torch.Tensor], leaf_nodes: List[TreeNode], n_leaves: int,
                      ignore_index: int = -100) -> TreeCELoss:
    """CE(logits[0], labels, ignore_index) / n_leaves per leaf (tree_grad_ckpt.py:279-297)."""
    return TreeCELoss(leaf_labels, leaf_nodes, n_leaves, ignore_index)


tree_grad_ckpt_backward = tree_grad_ckpt_sequential
