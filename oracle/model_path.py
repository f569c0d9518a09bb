"""Oracle: the reference's whole-tree drivers on a transformers model, on the CPU.

Test infrastructure only. Restates, with the oracle's own literal metadata
(``tree_meta.build_dfs_tree_info_literal``), what the reference drivers do:
  * ``dense_leaf_logits`` — dfs_tree_forward.py:543-570: ids, depth positions,
    the additive [1,1,N,N] mask in the model dtype, one model call with the
    eager attention (the dense-mask path), leaf logit views;
  * ``sequential_param_grads`` — tree_grad_ckpt.py:193-261 with
    make_tree_loss_fn (:279-297) and the fp32 parameter-grad hooks of
    verify_hybrid.py:74-84: one backward per leaf in DFS order.
Run it on a float64 copy of the model for a reference the fp32 engine is
checked against.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .tree_meta import build_dfs_tree_info_literal


def _eager(model):
    cfg = model.config
    saved = cfg._attn_implementation
    cfg._attn_implementation = "eager"
    return saved


def dense_leaf_logits(model, roots):
    """Returns (leaf_logits list of [1, L, V], leaf_nodes)."""
    info = build_dfs_tree_info_literal(roots)
    dev = next(model.parameters()).device
    dtype = next(model.parameters()).dtype
    ids = torch.tensor([info["dfs_token_ids"]], device=dev)
    pos = torch.tensor([info["dfs_pos_ids"]], device=dev)
    N = info["N"]
    mask = torch.full((1, 1, N, N), float("-inf"), dtype=dtype, device=dev)
    mask[0, 0][torch.from_numpy(info["attn_mask_bool"]).to(dev)] = 0.0
    saved = _eager(model)
    try:
        logits = model(input_ids=ids, attention_mask=mask, position_ids=pos, use_cache=False).logits
    finally:
        model.config._attn_implementation = saved
    out = [logits[:, s:e, :] for s, e in (info["chunk_boundaries"][c] for c in info["leaf_chunk_ids"])]
    return out, info["leaf_nodes"]


def sequential_param_grads(model, roots, labels_by_id, n_leaves, ignore_index=-100):
    """fp64/fp32 parameter gradients of the sequential whole-tree run, as a
    dict name -> CPU float64 tensor."""
    model.zero_grad(set_to_none=True)
    acc = {}
    handles = []
    for name, p in model.named_parameters():
        def hook(g, name=name):
            g = g.detach().cpu().double()
            acc[name] = acc[name] + g if name in acc else g.clone()
        handles.append(p.register_hook(hook))
    try:
        leaf_logits, leaf_nodes = dense_leaf_logits(model, roots)
        n = len(leaf_logits)
        for i, (lg, node) in enumerate(zip(leaf_logits, leaf_nodes)):
            lab = labels_by_id[id(node)].to(lg.device)
            loss = F.cross_entropy(lg[0], lab, ignore_index=ignore_index) / n_leaves
            loss.backward(retain_graph=i < n - 1)
    finally:
        for h in handles:
            h.remove()
    return acc
