"""Oracle: the reference's whole-tree drivers on a transformers model, on the CPU.

Test infrastructure only. Restates, with the oracle's own literal metadata
(``tree_meta.build_dfs_tree_info_literal``), what the reference drivers do:
  * ``dense_leaf_logits`` — dfs_tree_forward.py:543-570: ids, depth positions,
    the additive [1,1,N,N] mask in the model dtype, one model call with the
    eager attention (the dense-mask path), leaf logit views;
  * ``sequential_param_grads`` — tree_grad_ckpt.py:193-261 with
    make_tree_loss_fn (:279-297) and the fp32 parameter-grad hooks of
    verify_hybrid.py:74-84: one backward per leaf in DFS order;
  * ``tree_gdn_layers`` — the GatedDeltaNet patch the reference installs around
    its whole-tree forward (dfs_tree_forward.py:442-467, tree_dfs_ssm.py:432-445):
    every linear-attention layer computes ``gdn.gdn_layer_torch`` over the DFS
    forest (the exact rule, or with ``reference_truncated`` the reference's own
    I + R + R^2 scan), so the two functions above become the reference's
    drivers on hybrid (Qwen3.5) models;
  * ``hybrid_param_grads`` — tree_grad_hybrid.py:434-539 (attention models):
    partitions forwarded top-down, each over its gateway KV with the gateway
    bias in the additive mask, then per partition bottom-up one backward per
    leaf and one chaining backward per unique gateway (the gateway gradients
    kept in the model dtype instead of the reference's fp32 host copy, so a
    float64 run is exact to its own rounding).
Run it on a float64 copy of the model for a reference the fp32 engine is
checked against.
"""
from __future__ import annotations

import contextlib

import torch
import torch.nn.functional as F

from .gdn import gdn_layer_torch
from .partition import hybrid_schedule
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


@contextlib.contextmanager
def tree_gdn_layers(model, roots, reference_truncated=False):
    """Within the block every GatedDeltaNet layer of ``model`` (modules with
    ``in_proj_qkv`` and ``A_log``, called as ``linear_attn(hidden_states=...)``)
    runs ``gdn_layer_torch`` over the DFS-packed forest of ``roots``."""
    info = build_dfs_tree_info_literal(roots)
    lens = [e - s for s, e in info["chunk_boundaries"]]
    par = list(info["chunk_parent_map"])
    layers = [m for m in model.modules() if hasattr(m, "in_proj_qkv") and hasattr(m, "A_log")]

    def make(ssm):
        def forward(hidden_states=None, *args, **kwargs):
            assert hidden_states.shape[0] == 1 and hidden_states.shape[1] == sum(lens)
            return gdn_layer_torch(ssm, hidden_states[0], lens, par, reference_truncated)[None]
        return forward

    for m in layers:
        m.forward = make(m)
    try:
        yield
    finally:
        for m in layers:
            del m.forward


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


class _GatewayCache:
    """The gateway cache of tree_grad_ckpt_opath.py:66-133 in the duck type the
    transformers model calls: each layer's gateway K/V ([1, Hkv, past, D]) in
    front of the partition's own, the concatenation kept per layer."""

    is_compileable = False

    def __init__(self, gate_kv):
        self.gate_kv = list(gate_kv)
        self.full_kv = {}

    def update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        if layer_idx < len(self.gate_kv):
            gk, gv = self.gate_kv[layer_idx]
            key_states = torch.cat([gk, key_states], dim=-2)
            value_states = torch.cat([gv, value_states], dim=-2)
        self.full_kv[layer_idx] = (key_states, value_states)
        return key_states, value_states

    def get_seq_length(self, layer_idx=0):
        return self.gate_kv[layer_idx][0].shape[-2] if layer_idx < len(self.gate_kv) else 0

    def get_mask_sizes(self, query, layer_idx=0):
        q_len = query.shape[0] if isinstance(query, torch.Tensor) else int(query)
        return self.get_seq_length(layer_idx) + q_len, 0

    def get_query_offset(self, layer_idx=0):
        return self.get_seq_length(layer_idx)


def hybrid_param_grads(model, roots, labels_by_id, n_leaves, max_tokens, legacy=True, ignore_index=-100):
    """Parameter gradients of tree_grad_hybrid (tree_grad_hybrid.py:434-539) as
    a dict name -> CPU float64 tensor. ``legacy`` selects the gateway bias of
    tree_grad_hybrid.py:207 (the whole parent gateway visible) or the
    inherited one (the cut node's ancestors only; partition.gateway_meta)."""
    model.zero_grad(set_to_none=True)
    acc = {}
    handles = []
    for name, p in model.named_parameters():
        def hook(g, name=name):
            g = g.detach().cpu().double()
            acc[name] = acc[name] + g if name in acc else g.clone()
        handles.append(p.register_hook(hook))
    dev = next(model.parameters()).device
    dtype = next(model.parameters()).dtype
    sched = hybrid_schedule(roots, max_tokens, legacy=legacy)
    entry_of = {id(e["partition"]): e for e in sched}
    children_of = {id(e["partition"]): [] for e in sched}
    for e in sched:
        p = e["partition"]
        if p.parent is not None:
            children_of[id(p.parent)].append((p.parent_cut_node, p))
    gates, fwd = {}, {}
    saved = _eager(model)
    try:
        # top-down forward (tree_grad_hybrid.py:465-499, _subtree_forward :303-405)
        for e in sched:
            p, info = e["partition"], e["info"]
            gw = gates.get(id(p))
            N, past = info["N"], (gw["total"] if gw is not None else 0)
            ids = torch.tensor([info["dfs_token_ids"]], device=dev)
            pos = torch.tensor([[x + e["pos_offset"] for x in info["dfs_pos_ids"]]], device=dev)
            mask = torch.full((1, 1, N, past + N), float("-inf"), dtype=dtype, device=dev)
            if past:
                mask[0, 0, :, :past] = torch.tensor(gw["bias"], dtype=dtype, device=dev)
            own = torch.from_numpy(info["attn_mask_bool"]).to(dev)
            mask[0, 0, :, past:] = torch.where(own, torch.zeros((), dtype=dtype, device=dev), mask[0, 0, :, past:])
            cache = _GatewayCache(gw["gates"] if gw is not None else [])
            logits = model(input_ids=ids, attention_mask=mask, position_ids=pos, past_key_values=cache,
                           use_cache=True).logits
            fwd[id(p)] = (logits, info)
            # child gateways, one per unique cut node (_make_child_gateways :174-250)
            made = {}
            for cn, child in children_of[id(p)]:
                if id(cn) not in made:
                    total = entry_of[id(child)]["gateway"]["total"]
                    gl, raws, sums = [], [], []
                    for layer in range(len(cache.full_kv)):
                        fk, fv = cache.full_kv[layer]
                        pair = []
                        for raw in (fk[:, :, :total, :], fv[:, :, :total, :]):
                            leaf = raw.detach().requires_grad_(True)
                            box = [None]

                            def h(g, box=box):
                                box[0] = g.detach().clone() if box[0] is None else box[0] + g.detach()
                                return torch.zeros_like(g)
                            leaf.register_hook(h)
                            pair.append(leaf)
                            raws.append(raw)
                            sums.append(box)
                        gl.append(tuple(pair))
                    made[id(cn)] = dict(entry_of[id(child)]["gateway"], gates=gl, raws=raws, sums=sums)
                gates[id(child)] = made[id(cn)]
        # bottom-up backward (:501-539, _chain_gateway_grads :253-272)
        for e in reversed(sched):
            p = e["partition"]
            logits, info = fwd[id(p)]
            leaf_chunks = []
            for i, lc in enumerate(info["leaf_chunk_ids"]):
                s, t = info["chunk_boundaries"][lc]
                orig = info["copy_to_orig"][id(info["leaf_nodes"][i])]
                if id(orig) in p.leaf_node_set:
                    leaf_chunks.append((s, t, orig))
            chains, seen = [], set()
            for _, child in children_of[id(p)]:
                gw = gates[id(child)]
                if id(gw) not in seen:
                    seen.add(id(gw))
                    chains.append(gw)
            remaining = len(leaf_chunks) + len(chains)
            for s, t, orig in leaf_chunks:
                remaining -= 1
                loss = F.cross_entropy(logits[0, s:t], labels_by_id[id(orig)].to(dev),
                                       ignore_index=ignore_index) / n_leaves
                loss.backward(retain_graph=remaining > 0)
            for gw in chains:
                remaining -= 1
                raws = [r for r, b in zip(gw["raws"], gw["sums"]) if b[0] is not None]
                grads = [b[0] for b in gw["sums"] if b[0] is not None]
                if raws:
                    torch.autograd.backward(raws, grads, retain_graph=remaining > 0)
    finally:
        model.config._attn_implementation = saved
        for hd in handles:
            hd.remove()
    return acc
