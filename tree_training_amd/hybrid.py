"""Partitioned tree training with gateway KV — drop-in for tree_grad_hybrid.py.

Same API and schedule as the reference (tree_grad_hybrid.py:48-558):
  * ``partition_tree`` — greedy DFS partitioning to ``max_tokens`` (:60-95);
  * top-down forward of each partition with its parent's gateway KV (:468-499);
  * bottom-up per-leaf backward, then one gradient chain per unique gateway
    (:502-539).

What changes underneath:
  * each partition runs the HIP tree attention with the gateway as a second key
    segment (no dense [N, past+N] mask, no per-layer ``cat``);
  * gateway gradients are accumulated in float32 on the device by the attention
    backward (the reference's hooks copy every gradient to the host,
    tree_grad_hybrid.py:220-225), and chaining hands the own-token part to
    autograd and adds the inherited part straight into the parent gateway's
    fp32 accumulators;
  * the gateway bias is *inherited* through partition chains by default, so a
    partition sees exactly the ancestors of its cut node at every depth and
    the result equals the whole-tree run. ``legacy_gateway_bias=True``
    reproduces the reference literally, where a second-level gateway exposes
    the parent's whole gateway (``bias[:parent_past_len] = 0``,
    tree_grad_hybrid.py:207), DFS siblings included.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Tuple

import torch
import torch.nn.functional as F

from .dfs_tree_forward import fused_ce_capable, literal_options, run_tree_model
from .loss import TreeCELoss
from .gateway import GatewayAccumulator, GatewayCache
from .tree import DFSTreeInfo, TreeNode, info_from_flat


# ---------------------------------------------------------------------------
# 1. partitioning
# ---------------------------------------------------------------------------
@dataclass
class SubtreePartition:
    """One partition (tree_grad_hybrid.py:48-57)."""
    entry_nodes: List[TreeNode]
    dfs_nodes: List[TreeNode] = field(default_factory=list)
    cut_node_set: set = field(default_factory=set)
    leaf_node_set: set = field(default_factory=set)
    parent: Optional["SubtreePartition"] = None
    parent_cut_node: Optional[TreeNode] = None
    pos_offset: int = 0
    token_count: int = 0


def partition_tree(roots: List[TreeNode], max_tokens: int) -> List[SubtreePartition]:
    """Greedy DFS partitioning (tree_grad_hybrid.py:60-95).

    A node joins the current partition unless it is not the entry, the
    partition already holds tokens, and it would exceed ``max_tokens``; then its
    parent becomes a cut node and the node starts a child partition. Each forest
    root starts its own top-level partition. Partitions are listed parent
    before child, in the pre-order of the partition tree. Both walks are
    iterative, so tree depth is unbounded.
    """
    partitions: List[SubtreePartition] = []
    work = [([root], None, None) for root in reversed(roots)]
    while work:
        entry, parent, cut = work.pop()
        p = SubtreePartition(entry_nodes=entry, parent=parent, parent_cut_node=cut)
        partitions.append(p)
        deferred: List[Tuple[TreeNode, TreeNode]] = []
        stack = [(n, None) for n in reversed(entry)]
        while stack:
            node, par = stack.pop()
            L = len(node.token_ids)
            if par is not None and p.token_count > 0 and p.token_count + L > max_tokens:
                p.cut_node_set.add(id(par))
                deferred.append((par, node))
                continue
            p.dfs_nodes.append(node)
            p.token_count += L
            if not node.children:
                p.leaf_node_set.add(id(node))
            for ch in reversed(node.children):
                stack.append((ch, node))
        for cut_node, child in reversed(deferred):
            work.append(([child], p, cut_node))
    return partitions


def pack_sibling_partitions(partitions: List[SubtreePartition], max_tokens: int) -> List[SubtreePartition]:
    """Merges partitions that hang off the same cut node of the same parent
    partition into one partition with several entry nodes (the reference's
    ``SubtreePartition.entry_nodes`` is a list), consecutive siblings while
    their token counts sum to at most ``max_tokens``. Siblings see the same
    gateway, so a merged partition computes what its members compute, in one
    model pass instead of several small ones (the reference gives every
    over-budget child of a cut node a partition of its own,
    tree_grad_hybrid.py:93-94). Parents still precede children; the merged
    partition takes the place of its first member. The partitions are updated
    in place (a merged partition is its first member, extended; the children
    of any member point at it), so pass a fresh ``partition_tree`` list."""
    out: List[SubtreePartition] = []
    holder: Dict[int, SubtreePartition] = {}     # id(original) -> partition that holds it now
    open_bin: Dict[Tuple[int, int], SubtreePartition] = {}
    for p in partitions:
        if p.parent is not None:
            p.parent = holder[id(p.parent)]
            key = (id(p.parent), id(p.parent_cut_node))
            b = open_bin.get(key)
            if b is not None and b.token_count + p.token_count <= max_tokens:
                b.entry_nodes = list(b.entry_nodes) + list(p.entry_nodes)
                b.dfs_nodes.extend(p.dfs_nodes)
                b.cut_node_set |= p.cut_node_set
                b.leaf_node_set |= p.leaf_node_set
                b.token_count += p.token_count
                holder[id(p)] = b
                continue
            open_bin[key] = p
        holder[id(p)] = p
        out.append(p)
    return out


# ---------------------------------------------------------------------------
# 2. DFS info of one partition
# ---------------------------------------------------------------------------
def _flatten_partition(partition: SubtreePartition):
    members = {id(n) for n in partition.dfs_nodes}
    node_len, parent, nodes = [], [], []
    for entry in partition.entry_nodes:
        if id(entry) not in members:
            continue
        stack = [(entry, -1)]
        while stack:
            node, par = stack.pop()
            me = len(nodes)
            nodes.append(node)
            node_len.append(len(node.token_ids))
            parent.append(par)
            for ch in reversed(node.children):
                if id(ch) in members:
                    stack.append((ch, me))
    return node_len, parent, nodes


def _dfs_info_for_partition(partition: SubtreePartition):
    """DFS info of the in-partition subtree (tree_grad_hybrid.py:102-153).

    Returns (dfs_info, start, end, par, chunk_idx, copy_to_orig) keyed by
    id() of the original nodes. No nodes are copied: ``copy_to_orig`` maps each
    node's id to itself, so code written against the reference still works.
    """
    node_len, parent, nodes = _flatten_partition(partition)
    info = info_from_flat(node_len, parent, nodes)
    start, end, par, cidx = {}, {}, {}, {}
    for c, node in enumerate(nodes):
        s, e = info.chunk_boundaries[c]
        start[id(node)], end[id(node)] = s, e
        par[id(node)] = id(nodes[parent[c]]) if parent[c] >= 0 else -1
        cidx[id(node)] = c
    copy_to_orig = {id(n): n for n in nodes}
    return info, start, end, par, cidx, copy_to_orig


# ---------------------------------------------------------------------------
# 3. gateways
# ---------------------------------------------------------------------------
@dataclass
class SubtreeGateway:
    """Gateway from a parent partition to the partitions of one cut node
    (tree_grad_hybrid.py:160-171).

    ``key_gates/val_gates`` are detached leaves [1, Hkv, past_len, D]: the
    parent's own gateway followed by the parent's own tokens up to the cut
    node's end. ``raw_keys/raw_vals`` are the own-token parts with autograd
    history; ``fp32_acc`` receives the children's gateway gradients in float32;
    ``parent_acc`` / ``parent_past_len`` route the inherited part back into the
    parent gateway's accumulators at chaining.
    """
    key_gates: List[torch.Tensor]
    val_gates: List[torch.Tensor]
    raw_keys: List[torch.Tensor]
    raw_vals: List[torch.Tensor]
    fp32_acc: List[GatewayAccumulator]
    past_len: int
    attn_bias: torch.Tensor
    pos_offset: int
    parent_past_len: int = 0
    parent_acc: Optional[List[GatewayAccumulator]] = None
    ssm: Optional[object] = None

    @property
    def fp32_k(self):
        return [[a.k if a.touched else None] for a in self.fp32_acc]

    @property
    def fp32_v(self):
        return [[a.v if a.touched else None] for a in self.fp32_acc]


def _ancestor_ranges(cut_node, start, end, par):
    ranges = []
    nid = id(cut_node)
    while nid != -1 and nid in start:
        ranges.append((start[nid], end[nid]))
        nid = par.get(nid, -1)
    return ranges


def gateway_bias_and_offset(info: DFSTreeInfo, start, end, par, cidx, cut_node, parent_pos_offset: int,
                            parent_past_len: int, parent_bias: Optional[torch.Tensor],
                            legacy: bool = False):
    """(total, bias [total] float32 CPU, pos_off) of one cut node
    (tree_grad_hybrid.py:193-209). With ``legacy`` False the first
    ``parent_past_len`` entries copy the parent gateway's bias; with ``legacy``
    True they are all 0 as in the reference."""
    cut_end = end[id(cut_node)]
    total = parent_past_len + cut_end
    pos_off = parent_pos_offset + info.node_off[cidx[id(cut_node)]] + len(cut_node.token_ids)
    bias = torch.full((total,), float("-inf"))
    if parent_past_len:
        if legacy or parent_bias is None:
            bias[:parent_past_len] = 0.0
        else:
            bias[:parent_past_len] = parent_bias.detach().float().cpu()[:parent_past_len]
    for s, e in _ancestor_ranges(cut_node, start, end, par):
        bias[parent_past_len + s: parent_past_len + e] = 0.0
    return total, bias, pos_off


def _make_child_gateways(own_kv, dfs_info, orig_id_to_start, orig_id_to_end, orig_id_to_par,
                         orig_id_to_chunk_idx, cut_nodes, parent_pos_offset, parent_gateway=None,
                         legacy: bool = False) -> Dict[int, SubtreeGateway]:
    """One gateway per unique cut node (tree_grad_hybrid.py:174-250).

    ``own_kv[l] = (k, v)`` are the parent partition's own keys/values of layer
    l ([1, Hkv, N, D], with autograd history)."""
    gateways: Dict[int, SubtreeGateway] = {}
    ppl = parent_gateway.past_len if parent_gateway is not None else 0
    pbias = parent_gateway.attn_bias if parent_gateway is not None else None
    for cn in cut_nodes:
        total, bias, pos_off = gateway_bias_and_offset(
            dfs_info, orig_id_to_start, orig_id_to_end, orig_id_to_par, orig_id_to_chunk_idx, cn,
            parent_pos_offset, ppl, pbias, legacy)
        cut_end = orig_id_to_end[id(cn)]
        kg, vg, rk, rv, accs = [], [], [], [], []
        for l, (k, v) in enumerate(own_kv):
            rk_l, rv_l = k[:, :, :cut_end], v[:, :, :cut_end]
            with torch.no_grad():
                if ppl:
                    gk = torch.cat([parent_gateway.key_gates[l].detach(), rk_l], dim=2)
                    gv = torch.cat([parent_gateway.val_gates[l].detach(), rv_l], dim=2)
                else:
                    gk, gv = rk_l.detach(), rv_l.detach()
            gk.requires_grad_(True)
            gv.requires_grad_(True)
            kg.append(gk)
            vg.append(gv)
            rk.append(rk_l)
            rv.append(rv_l)
            accs.append(GatewayAccumulator(gk))
        gateways[id(cn)] = SubtreeGateway(
            key_gates=kg, val_gates=vg, raw_keys=rk, raw_vals=rv, fp32_acc=accs, past_len=total,
            attn_bias=bias, pos_offset=pos_off, parent_past_len=ppl,
            parent_acc=parent_gateway.fp32_acc if parent_gateway is not None else None)
    return gateways


def _chain_gateway_grads(gw: SubtreeGateway, retain_graph: bool = False, collect: Optional[list] = None) -> None:
    """Chain a gateway's fp32 gradients into the parent (tree_grad_hybrid.py:253-272).

    The own-token part goes through autograd into the parent partition's graph
    (autograd casts it to the K/V dtype, as in the reference); the inherited
    part is added to the parent gateway's fp32 accumulators. With ``collect``
    the (tensor, gradient) pairs are appended there instead of run."""
    raws, grads = [], []
    ppl = gw.parent_past_len
    for l, acc in enumerate(gw.fp32_acc):
        if not acc.touched:
            continue
        if ppl and gw.parent_acc is not None:
            pa = gw.parent_acc[l]
            pa.k[:ppl] += acc.k[:ppl]
            pa.v[:ppl] += acc.v[:ppl]
            pa.touched = True
        raws += [gw.raw_keys[l], gw.raw_vals[l]]
        grads += [acc.as_hf("k")[:, :, ppl:], acc.as_hf("v")[:, :, ppl:]]
    if collect is not None:
        collect.extend(zip(raws, grads))
    elif raws:
        torch.autograd.backward(raws, grads, retain_graph=retain_graph)


# ---------------------------------------------------------------------------
# 4. one partition forward
# ---------------------------------------------------------------------------
def _subtree_forward(model, partition: SubtreePartition, gateway: Optional[SubtreeGateway], dev, dtype,
                     hidden_only: bool = False, prebuilt=None, fused_prologue: bool = True):
    """Forward of one partition with its gateway (tree_grad_hybrid.py:279-427).
    ``prebuilt``: (DFS info tuple, KeyPlan) from ``_prebuild_partitions``.

    Returns (logits, or the final hidden states when ``hidden_only``, dfs_info,
    own_kv, start, end, par, chunk_idx, copy_to_orig)."""
    if prebuilt is not None:
        (info, start, end, par, cidx, c2o), plan = prebuilt
    else:
        (info, start, end, par, cidx, c2o), plan = _dfs_info_for_partition(partition), None
    gate_kv = list(zip(gateway.key_gates, gateway.val_gates)) if gateway is not None else []
    cache = GatewayCache(gate_kv, segmented=True)
    out = run_tree_model(model, info, dev, pos_offset=partition.pos_offset, cache=cache,
                         accumulators=gateway.fp32_acc if gateway is not None else None,
                         past_bias=gateway.attn_bias if gateway is not None else None, hidden_only=hidden_only,
                         plan=plan, fused_prologue=fused_prologue)
    own_kv = [cache.own_kv(l) for l in sorted(cache._segments)]
    res = out.last_hidden_state if hidden_only else out.logits
    return res, info, own_kv, start, end, par, cidx, c2o


def _prebuild_partitions(partitions, children_of, dev, legacy: bool):
    """Host DFS info of every partition and, in one ``meta.build_trees`` call,
    their device metadata and tile plans (positions, horizons, gateway key
    intervals): all of it depends on the topology alone, so the whole step's
    metadata is built up front in a few launches instead of per partition.
    Returns {id(partition): ((info, start, end, par, cidx, c2o), KeyPlan)}."""
    from .meta import build_trees
    infos, gws, specs = {}, {}, []
    for p in partitions:                                   # parents before children
        gw = gws.get(id(p))
        pos_offset = gw[2] if gw is not None else 0
        infos[id(p)] = _dfs_info_for_partition(p)
        info, start, end, par, cidx, _ = infos[id(p)]
        specs.append((info.node_len, info.chunk_parent_map, pos_offset, gw[1] if gw is not None else None))
        made = {}
        for cn, child in children_of[id(p)]:
            if id(cn) not in made:
                made[id(cn)] = gateway_bias_and_offset(info, start, end, par, cidx, cn, pos_offset,
                                                       gw[0] if gw else 0, gw[1] if gw else None, legacy)
            gws[id(child)] = made[id(cn)]
    built = build_trees(specs, dev)
    out = {}
    for p, spec, (meta, plan) in zip(partitions, specs, built):
        info = infos[id(p)][0]
        info._meta[(str(meta.device), spec[2])] = meta
        out[id(p)] = (infos[id(p)], plan)
    return out


# ---------------------------------------------------------------------------
# 5. driver
# ---------------------------------------------------------------------------
def tree_grad_hybrid(model, roots: List[TreeNode], leaf_loss_fn: Callable[[torch.Tensor, TreeNode], torch.Tensor],
                     max_tokens: int, legacy_gateway_bias: bool = False, summed_backward: bool = False,
                     fused_leaf_ce: bool = True, fused_prologue: bool = True,
                     reference_literal: bool = False, pack_siblings: bool = True) -> None:
    """Hybrid tree training (tree_grad_hybrid.py:434-539); grads accumulate in ``.grad``.

    model        : HF causal LM (Qwen3 family), train mode, zero_grad() already called
    roots        : forest roots
    leaf_loss_fn : loss = leaf_loss_fn(logits [1, L, V], node) -> scalar
    max_tokens   : max DFS token count per partition
    summed_backward : False (default) keeps the reference's schedule, one
                   ``retain_graph`` backward per leaf and per gateway chain
                   (:526-539), each running the partition's whole backward
                   graph; True runs ONE backward per partition over the sum of
                   its leaf losses and its chain gradients (the same gradients
                   up to summation order).
    fused_leaf_ce : with a ``make_tree_loss_fn`` loss, take the leaf losses from
                   the final hidden states through the chunked lm_head + fused
                   cross-entropy (no [T, V] logits), one backward per partition
                   as with ``summed_backward``; other losses get logits.
    fused_prologue : the fused q/k RMSNorm + rotary kernel (False: transformers'
                   own modules).
    pack_siblings : merge the partitions of one cut node while they fit
                   ``max_tokens`` (``pack_sibling_partitions``; the same
                   gradients up to summation order, fewer and larger model
                   passes); False keeps the reference's partition list.
    reference_literal : every option at the reference's arithmetic — the legacy
                   gateway bias, transformers' prologue and logits + CE, the
                   per-leaf backward schedule (``literal_options``).
    """
    o = literal_options(reference_literal, legacy_gateway_bias=legacy_gateway_bias,
                        fused_leaf_ce=fused_leaf_ce, fused_prologue=fused_prologue, pack_siblings=pack_siblings)
    legacy_gateway_bias, fused_leaf_ce = o["legacy_gateway_bias"], o["fused_leaf_ce"]
    if reference_literal:
        summed_backward = False
    dev = next(model.parameters()).device
    dtype = next(model.parameters()).dtype
    fused = fused_leaf_ce and fused_ce_capable(model, leaf_loss_fn)
    partitions = partition_tree(roots, max_tokens)
    if o["pack_siblings"]:
        partitions = pack_sibling_partitions(partitions, max_tokens)
    children_of: Dict[int, List[Tuple[TreeNode, SubtreePartition]]] = {id(p): [] for p in partitions}
    for p in partitions:
        if p.parent is not None:
            children_of[id(p.parent)].append((p.parent_cut_node, p))

    prebuilt = _prebuild_partitions(partitions, children_of, dev, legacy_gateway_bias)
    gateways: Dict[int, Optional[SubtreeGateway]] = {}
    fwd_cache: Dict[int, tuple] = {}
    for p in partitions:                                   # top-down forward
        gw = gateways.get(id(p))
        p.pos_offset = gw.pos_offset if gw is not None else 0
        logits, info, own_kv, s_map, e_map, par_map, ci_map, c2o = _subtree_forward(
            model, p, gw, dev, dtype, hidden_only=fused, prebuilt=prebuilt.pop(id(p)),
            fused_prologue=o["fused_prologue"])
        fwd_cache[id(p)] = (logits, info, c2o)
        seen, cuts = set(), []
        for cn, _ in children_of[id(p)]:
            if id(cn) not in seen:
                seen.add(id(cn))
                cuts.append(cn)
        if cuts:
            child_gws = _make_child_gateways(own_kv, info, s_map, e_map, par_map, ci_map, cuts, p.pos_offset,
                                             gw, legacy=legacy_gateway_bias)
            for cn, child_p in children_of[id(p)]:
                gateways[id(child_p)] = child_gws[id(cn)]

    for p in reversed(partitions):                         # bottom-up backward
        logits, info, c2o = fwd_cache.pop(id(p))
        leaf_chunks = []
        for i, lc in enumerate(info.leaf_chunk_ids):
            s, e = info.chunk_boundaries[lc]
            leaf = c2o[id(info.leaf_nodes[i])]
            if id(leaf) in p.leaf_node_set:
                leaf_chunks.append((s, e, leaf))
        seen_gw, chains = set(), []
        for cut_node, child_p in children_of[id(p)]:
            cgw = gateways.get(id(child_p))
            if cgw is not None and id(cgw) not in seen_gw:
                seen_gw.add(id(cgw))
                chains.append(cgw)
        if summed_backward or fused:
            pairs = []
            for cgw in chains:
                _chain_gateway_grads(cgw, collect=pairs)
            roots_, grads_ = [t for t, _ in pairs], [g for _, g in pairs]
            if leaf_chunks and fused:
                roots_.append(leaf_loss_fn.fused_spans(logits[0], leaf_chunks, model.lm_head.weight))
                grads_.append(None)
            elif leaf_chunks:
                roots_.append(sum(leaf_loss_fn(logits[:, s:e, :], leaf) for s, e, leaf in leaf_chunks))
                grads_.append(None)
            if roots_:
                torch.autograd.backward(roots_, grads_)
            continue
        remaining = [len(leaf_chunks) + len(chains)]

        def _retain():
            remaining[0] -= 1
            return remaining[0] > 0

        for s, e, leaf in leaf_chunks:
            leaf_loss_fn(logits[:, s:e, :], leaf).backward(retain_graph=_retain())
        for cgw in chains:
            _chain_gateway_grads(cgw, retain_graph=_retain())


def make_tree_loss_fn(leaf_labels: List[torch.Tensor], leaf_nodes: List[TreeNode], n_leaves: int,
                      ignore_index: int = -100) -> TreeCELoss:
    """CE(logits[0], labels, ignore_index) / n_leaves (tree_grad_hybrid.py:546-558)."""
    return TreeCELoss(leaf_labels, leaf_nodes, n_leaves, ignore_index)


# ---------------------------------------------------------------------------
# 6. model-free schedule (benchmarks, inspection)
# ---------------------------------------------------------------------------
def hybrid_plan(roots: List[TreeNode], max_tokens: int, legacy: bool = False,
                pack_siblings: bool = True) -> List[dict]:
    """Per-partition attention problems of ``tree_grad_hybrid`` without a model:
    partition-local (node_len, parent), pos_offset, and the gateway length and
    bias each partition attends to, in creation order (``pack_siblings`` as in
    ``tree_grad_hybrid``)."""
    partitions = partition_tree(roots, max_tokens)
    if pack_siblings:
        partitions = pack_sibling_partitions(partitions, max_tokens)
    gw_of: Dict[int, dict] = {}
    children_of: Dict[int, list] = {id(p): [] for p in partitions}
    for p in partitions:
        if p.parent is not None:
            children_of[id(p.parent)].append((p.parent_cut_node, p))
    out = []
    for p in partitions:
        gw = gw_of.get(id(p))
        pos_offset = gw["pos_off"] if gw is not None else 0
        node_len, parent, nodes = _flatten_partition(p)
        info, start, end, par, cidx, _ = _dfs_info_for_partition(p)
        out.append(dict(node_len=node_len, parent=parent, pos_offset=pos_offset,
                        past_len=gw["total"] if gw is not None else 0,
                        bias=gw["bias"] if gw is not None else None, n_tokens=info.N))
        made = {}
        for cn, child in children_of[id(p)]:
            if id(cn) not in made:
                total, bias, pos_off = gateway_bias_and_offset(
                    info, start, end, par, cidx, cn, pos_offset, gw["total"] if gw else 0,
                    gw["bias"] if gw else None, legacy)
                made[id(cn)] = dict(total=total, bias=bias, pos_off=pos_off)
            gw_of[id(child)] = made[id(cn)]
    return out
