"""Single-pass DFS tree forward — drop-in for dfs_tree_forward.py Parts 7-8.

``dfs_tree_forward(model, roots, dtype=None)`` runs one forward over the whole
DFS-packed forest and returns per-leaf logit views (dfs_tree_forward.py:513-576).
Instead of a dense [1,1,N,N] additive mask the model runs with the
``"tree_hip"`` attention implementation: positions come straight from the GPU
metadata kernel and every layer shares one tile plan. Gated-delta-rule layers
of hybrid models are patched for the duration of the forward (tree conv + tree
scan, ``gdn_layer._patch_ssm``), as the reference does (dfs_tree_forward.py:553-562).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

import torch
import torch.nn.functional as F

from .hf_adapter import TreeAttnContext, tree_attention_mode
from .meta import upload_i32
from .tree import DFSTreeInfo, TreeNode, build_dfs_tree_info


@dataclass
class DFSTreeResult:
    """Output of dfs_tree_forward (dfs_tree_forward.py:474-506).

    leaf_logits : list of [1, Lc, V] views into the single forward's logits, DFS order
    leaf_nodes  : the leaf TreeNodes (same order)
    info        : DFSTreeInfo
    """
    leaf_logits: List[torch.Tensor]
    leaf_nodes: List[TreeNode]
    info: DFSTreeInfo

    def total_loss(self, labels: List[torch.Tensor]) -> torch.Tensor:
        """Sum of per-leaf cross entropies (labels[i]: [Lc] LongTensor)."""
        if len(labels) != len(self.leaf_logits):
            raise AssertionError(f"Expected {len(self.leaf_logits)} label tensors, got {len(labels)}")
        return sum(F.cross_entropy(lg.squeeze(0), lab.to(lg.device))
                   for lg, lab in zip(self.leaf_logits, labels))


def fused_ce_capable(model, leaf_loss_fn) -> bool:
    """True when the leaf loss can be taken from the final hidden states with
    the fused lm_head + cross-entropy (``loss.TreeCELoss`` on a causal LM whose
    logits are plain ``lm_head(hidden)``)."""
    from .loss import TreeCELoss
    head = getattr(model, "lm_head", None)
    return (isinstance(leaf_loss_fn, TreeCELoss) and hasattr(model, "model") and head is not None
            and getattr(head, "bias", None) is None and hasattr(head, "weight")
            and getattr(model.config, "final_logit_softcapping", None) is None)


def run_tree_model(model, info: DFSTreeInfo, dev, pos_offset: int = 0, cache=None, accumulators=None,
                   past_bias: Optional[torch.Tensor] = None, linear_attention_patched: bool = False,
                   hidden_only: bool = False, plan=None, fused_prologue: bool = True):
    """One model forward over a DFS-packed forest (or partition) with tree
    attention. Returns the model output (the decoder's, with the final hidden
    states and no logits, when ``hidden_only``). ``plan``: a KeyPlan already
    built for this tree and gateway (``meta.build_trees``), else built here.
    ``fused_prologue``: the fused q/k RMSNorm + rotary kernel in place of the
    model's own modules (False: transformers' own ops, as the reference)."""
    vocab = getattr(getattr(model, "config", None), "vocab_size", None)
    if vocab is not None and info.dfs_token_ids and not (0 <= min(info.dfs_token_ids) and
                                                         max(info.dfs_token_ids) < vocab):
        # the embedding lookup on the device does not check its indices
        raise ValueError(f"token ids must lie in [0, {vocab}) (the model's vocabulary); got "
                         f"[{min(info.dfs_token_ids)}, {max(info.dfs_token_ids)}]")
    meta = info.device_meta(dev, pos_offset)
    if plan is None:
        plan = info.key_plan(dev, past_bias, pos_offset)
    ids_t = upload_i32([info.dfs_token_ids], dev).long()
    pos_t = meta.pos.long().unsqueeze(0)
    ctx = TreeAttnContext(plan=plan, cache=cache, accumulators=accumulators)
    with tree_attention_mode(model, linear_attention_patched, fused_prologue):
        body = model.model if hidden_only else model
        return body(input_ids=ids_t, attention_mask=None, position_ids=pos_t,
                    past_key_values=cache, use_cache=cache is not None, tree_ctx=ctx)


def literal_options(reference_literal: bool, **opts) -> dict:
    """The drivers' options, with every one that departs from the reference's
    arithmetic switched to the reference's when ``reference_literal``: the
    legacy gateway bias (tree_grad_hybrid.py:206-209), the truncated
    whole-node GDN correction I + R + R^2 (tree_dfs_ssm.py:114-126), node by
    node GDN projections, transformers' own q/k norm + rotary and
    lm_head + cross-entropy instead of the fused kernels, and the reference's
    partition list (no sibling packing)."""
    if reference_literal:
        lit = dict(legacy_gateway_bias=True, gdn_reference_truncated=True, gdn_per_node_projections=True,
                   fused_prologue=False, fused_leaf_ce=False, pack_siblings=False)
        opts.update({k: v for k, v in lit.items() if k in opts})
    return opts


def dfs_tree_forward(model, roots: List[TreeNode], dtype: Optional[torch.dtype] = None,
                     gdn_reference_truncated: bool = False, gdn_per_node_projections: bool = False,
                     fused_prologue: bool = True, reference_literal: bool = False) -> DFSTreeResult:
    """One DFS-packed forward over a forest (dfs_tree_forward.py:513-576).

    ``dtype`` is accepted for signature compatibility; it only set the dense
    mask's dtype in the reference, and no dense mask is built here.
    ``gdn_reference_truncated`` makes the gated-delta-rule layers of hybrid
    models compute what the reference's scan computes (I + R + R^2 per node)
    instead of the exact rule; ``gdn_per_node_projections`` makes them
    project node by node as the reference does (same GEMM shapes as per-path
    runs, so their outputs match those bit for bit) instead of one GEMM per
    projection. ``fused_prologue`` False runs transformers' own q/k norm and
    rotary. ``reference_literal`` sets all three to the reference's arithmetic
    (``literal_options``).
    """
    o = literal_options(reference_literal, gdn_reference_truncated=gdn_reference_truncated,
                        gdn_per_node_projections=gdn_per_node_projections, fused_prologue=fused_prologue)
    dev = next(model.parameters()).device
    info = build_dfs_tree_info(roots)
    # gated-delta-rule layers (hybrid models) run the tree-aware conv + scan
    from .gdn_layer import _patch_ssm, _unpatch_ssm
    saved = _patch_ssm(model, info.chunk_boundaries, info.chunk_parent_map, o["gdn_reference_truncated"],
                       o["gdn_per_node_projections"])
    try:
        out = run_tree_model(model, info, dev, linear_attention_patched=True, fused_prologue=o["fused_prologue"])
    finally:
        _unpatch_ssm(saved)       # always restored, even if the forward raises
    logits = out.logits
    leaf_logits = [logits[:, s:e, :] for s, e in (info.chunk_boundaries[c] for c in info.leaf_chunk_ids)]
    return DFSTreeResult(leaf_logits=leaf_logits, leaf_nodes=info.leaf_nodes, info=info)
