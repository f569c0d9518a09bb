"""Tree gated delta rule (linear-attention layers) on the GPU.

Drop-in for ``torch_chunk_gated_delta_rule_tree_varlen`` (tree_dfs_ssm.py:38-156,
twin ``_tree_gated_delta_net_varlen`` in dfs_tree_forward.py:253-353): the same
inputs — q, k ``[B=1, T, Hk, D]``, v ``[1, T, Hv, D]``, g, beta ``[1, T, Hv]``,
``chunk_boundaries`` (one (start, end) per tree node, DFS order) and
``chunk_parent_map`` (parent node index, -1 for a root), the optional
``initial_state`` every root starts from and ``output_final_state`` (the last
node's state, differentiable like the output) — computed through
``tt_gdn_tree_fwd``: one parallel HIP launch over all 32-token chunks for the
state-independent terms, then one scan launch per tree level.

Semantics: by default the exact gated delta rule along every root-to-leaf
path (what the reference function states it computes, tree_dfs_ssm.py:49-52).
With ``reference_truncated=True`` it returns what the reference function itself
computes: every whole node one chunk, the within-node correction built from
the uncorrected rows, A = I + R + R^2 (tree_dfs_ssm.py:120-126). The two agree
for nodes of at most three tokens and differ for longer ones.
"""
from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib
from .meta import _ptr, _stream, require_device, upload_i32

HEAD_DIM = 128
CHUNK = 32        # TT_GDN_CHUNK


class GdnTree:
    """Node ranges, parents and per-depth node groups of a DFS-packed forest,
    resident on the device (level offsets stay on the host: one launch per
    level)."""

    def __init__(self, node_len: Sequence[int], parent: Sequence[int], device):
        n = len(node_len)
        if n < 1 or len(parent) != n:
            raise ValueError("node_len and parent must be non-empty and of equal length")
        start, s = [], 0
        depth = []
        for i, (L, p) in enumerate(zip(node_len, parent)):
            if L < 1:
                raise ValueError(f"node {i} is empty")
            if not (-1 <= p < i):
                raise ValueError(f"node {i}: parent {p} does not precede it (DFS pre-order expected)")
            start.append(s)
            s += int(L)
            depth.append(0 if p < 0 else depth[p] + 1)
        self.n_nodes = n
        self.n_tokens = s
        self.node_len = [int(x) for x in node_len]
        self.parent = [int(x) for x in parent]
        self.node_start = start
        levels: List[List[int]] = [[] for _ in range(max(depth) + 1)]
        for i, d in enumerate(depth):
            levels[d].append(i)
        for lv in levels:   # longest nodes first: the scan of a level dispatches them (all heads) first
            lv.sort(key=lambda i: -self.node_len[i])
        order = [i for lv in levels for i in lv]
        offs = [0]
        for lv in levels:
            offs.append(offs[-1] + len(lv))
        self.n_levels = len(levels)
        self.level_offsets = (ctypes.c_int32 * len(offs))(*offs)
        kids: List[List[int]] = [[] for _ in range(n)]
        for i, par in enumerate(self.parent):
            if par >= 0:
                kids[par].append(i)
        child_off = [0]
        for ks in kids:
            child_off.append(child_off[-1] + len(ks))
        child = [c for ks in kids for c in ks] or [0]
        chunk0, chunk_node = [], []
        for i, L in enumerate(self.node_len):
            chunk0.append(len(chunk_node))
            chunk_node.extend([i] * ((L + CHUNK - 1) // CHUNK))
        self.n_chunks = len(chunk_node)
        dev = require_device(device)
        parts = [start, self.node_len, self.parent, order, chunk0, chunk_node, child_off, child]
        flat = upload_i32(np.concatenate([np.asarray(x, dtype=np.int32) for x in parts]), dev)
        (self.d_start, self.d_len, self.d_parent, self.d_levels, self.d_chunk0, self.d_chunk_node,
         self.d_child_off, self.d_child) = torch.split(flat, [len(x) for x in parts])
        self.device = dev

    def token_links(self):
        """Device (tok_prev [T], tok_next_off [T + 1], tok_next) of the tree's
        tokens: the path predecessor of each token and the successor lists
        (built once, on first use)."""
        if getattr(self, "_links", None) is None:
            T = self.n_tokens
            prev = np.arange(-1, T - 1, dtype=np.int64)
            for i, (st, par) in enumerate(zip(self.node_start, self.parent)):
                prev[st] = self.node_start[par] + self.node_len[par] - 1 if par >= 0 else -1
            has = prev >= 0
            order = np.argsort(prev[has], kind="stable")
            nxt = np.arange(T, dtype=np.int64)[has][order]
            off = np.zeros(T + 1, dtype=np.int64)
            np.cumsum(np.bincount(prev[has], minlength=T), out=off[1:])
            nxt = nxt if len(nxt) else np.zeros(1, np.int64)
            flat = upload_i32(np.concatenate([prev, off, nxt]), self.device)
            self._links = tuple(torch.split(flat, [len(prev), len(off), len(nxt)]))
        return self._links

    @classmethod
    def from_boundaries(cls, chunk_boundaries: Sequence[Tuple[int, int]], chunk_parent_map: Sequence[int],
                        device) -> "GdnTree":
        """From the reference's ``chunk_boundaries`` / ``chunk_parent_map``."""
        s = 0
        for a, b in chunk_boundaries:
            if a != s or b <= a:
                raise ValueError("chunk_boundaries must tile [0, T) in order with non-empty chunks")
            s = b
        return cls([b - a for a, b in chunk_boundaries], list(chunk_parent_map), device)


def _tok_heads(x: torch.Tensor, name: str) -> torch.Tensor:
    if x.dim() == 4:
        if x.shape[0] != 1:
            raise ValueError(f"{name}: batch size must be 1 (one packed tree)")
        x = x[0]
    if x.dim() != 3 or x.shape[-1] != HEAD_DIM:
        raise ValueError(f"{name}: expected [T, H, {HEAD_DIM}], got {tuple(x.shape)}")
    if x.stride(-1) != 1:
        x = x.contiguous()
    return x


def _tok_vec(x: torch.Tensor, name: str) -> torch.Tensor:
    if x.dim() == 3:
        if x.shape[0] != 1:
            raise ValueError(f"{name}: batch size must be 1")
        x = x[0]
    if x.dim() != 2:
        raise ValueError(f"{name}: expected [T, H], got {tuple(x.shape)}")
    x = x.float()
    if x.stride(-1) != 1:
        x = x.contiguous()
    return x


def _f32_block(x: Optional[torch.Tensor], shape: Tuple[int, ...], name: str) -> Optional[torch.Tensor]:
    """x (None passes through) as a contiguous float32 tensor of ``shape``."""
    if x is None:
        return None
    if tuple(x.shape) != shape:
        raise ValueError(f"{name}: expected {shape}, got {tuple(x.shape)}")
    return x.float().contiguous()


def _problem(q, k, v, g, beta, tree: GdnTree, scale, l2norm, reference_truncated=False, initial_state=None):
    q, k, v = _tok_heads(q, "q"), _tok_heads(k, "k"), _tok_heads(v, "v")
    g, beta = _tok_vec(g, "g"), _tok_vec(beta, "beta")
    T, Hk, _ = q.shape
    Hv = v.shape[1]
    if k.shape != q.shape or v.shape[0] != T or g.shape != (T, Hv) or beta.shape != (T, Hv):
        raise ValueError("q/k/v/g/beta shapes disagree")
    if T != tree.n_tokens:
        raise ValueError(f"{T} tokens but the tree holds {tree.n_tokens}")
    if v.dtype not in (torch.bfloat16, torch.float32) or q.dtype != v.dtype or k.dtype != v.dtype:
        raise ValueError("q, k, v must share dtype bfloat16 or float32")
    if initial_state is not None and initial_state.dim() == 4 and initial_state.shape[0] == 1:
        initial_state = initial_state[0]          # the reference's [B = 1, Hv, 128, 128]
    s0 = _f32_block(initial_state, (Hv, HEAD_DIM, HEAD_DIM), "initial_state")
    if s0 is not None and s0.device != v.device:
        raise ValueError("initial_state must be on the device of q, k, v")
    p = _lib.TTGdnProblem(
        dtype=_lib.TT_DTYPE_BF16 if v.dtype == torch.bfloat16 else _lib.TT_DTYPE_F32,
        n_tokens=T, n_nodes=tree.n_nodes, n_heads_k=Hk, n_heads_v=Hv, head_dim=HEAD_DIM,
        l2norm=1 if l2norm else 0, scale=float(scale if scale is not None else HEAD_DIM ** -0.5),
        q=_lib.TTTensor(q.data_ptr(), q.stride(0), q.stride(1)),
        k=_lib.TTTensor(k.data_ptr(), k.stride(0), k.stride(1)),
        v=_lib.TTTensor(v.data_ptr(), v.stride(0), v.stride(1)),
        g=g.data_ptr(), g_stride_tok=g.stride(0), beta=beta.data_ptr(), beta_stride_tok=beta.stride(0),
        node_start=_ptr(tree.d_start), node_len=_ptr(tree.d_len), node_parent=_ptr(tree.d_parent),
        level_nodes=_ptr(tree.d_levels), level_offsets=tree.level_offsets, n_levels=tree.n_levels,
        n_chunks=tree.n_chunks, node_chunk0=_ptr(tree.d_chunk0), chunk_node=_ptr(tree.d_chunk_node),
        node_child_off=_ptr(tree.d_child_off), node_child=_ptr(tree.d_child),
        reference_truncated=1 if reference_truncated else 0,
        initial_state=s0.data_ptr() if s0 is not None else None)
    return p, (q, k, v, g, beta, s0)


# Whether the autograd Function keeps the forward's per-chunk terms and states
# for the backward (tt_gdn_tree_fwd_save / tt_gdn_tree_bwd_saved: about 123 KiB
# per (32-token chunk, v head) held from forward to backward, 2.1 GB for a
# 16K-token tree with 32 v heads) instead of recomputing them in the backward.
KEEP_FORWARD_STATES = True


def _gdn_forward(q, k, v, g, beta, tree: GdnTree, scale, l2norm, keep: bool, reference_truncated=False,
                 initial_state=None):
    p, (q, k, v, g, beta, _s0) = _problem(q, k, v, g, beta, tree, scale, l2norm, reference_truncated,
                                          initial_state)
    T, Hv = v.shape[0], v.shape[1]
    dev = require_device(q.device)
    o = torch.empty((T, Hv, HEAD_DIM), dtype=v.dtype, device=dev)
    states = torch.empty((tree.n_nodes, Hv, HEAD_DIM, HEAD_DIM), dtype=torch.float32, device=dev)
    lib = _lib.lib()
    if keep:
        saved_bytes = lib.tt_gdn_saved_bytes(ctypes.byref(p))
        saved = torch.empty(saved_bytes, dtype=torch.uint8, device=dev)
        _lib.check(lib.tt_gdn_tree_fwd_save(ctypes.byref(p), _ptr(o), _ptr(states), _ptr(saved), saved_bytes,
                                            _stream(dev)), "tt_gdn_tree_fwd_save")
        return o, states, saved
    ws_bytes = lib.tt_gdn_workspace_bytes(ctypes.byref(p))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    _lib.check(lib.tt_gdn_tree_fwd(ctypes.byref(p), _ptr(o), _ptr(states), _ptr(ws), ws_bytes, _stream(dev)),
               "tt_gdn_tree_fwd")
    return o, states, None


def gdn_tree_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
                     tree: GdnTree, scale: Optional[float] = None, l2norm: bool = True,
                     reference_truncated: bool = False, initial_state: Optional[torch.Tensor] = None):
    """o [T, Hv, 128] (dtype of v) and node_states [n_nodes, Hv, 128, 128]
    (float32; the state after each node). ``initial_state`` [Hv, 128, 128]:
    the state every root starts from (zero when None)."""
    o, states, _ = _gdn_forward(q, k, v, g, beta, tree, scale, l2norm, False, reference_truncated, initial_state)
    return o, states


def _packed_qkv_width(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> Optional[int]:
    """Row width W when q, k, v [T, H, 128] are the consecutive column blocks
    [q | k | v] of one row-major [T, W] buffer (a conv output split three
    ways) with contiguous heads, else None."""
    st, e = q.stride(0), q.element_size()
    widths = [t.shape[1] * t.shape[2] for t in (q, k, v)]
    if any(t.stride(0) != st or t.stride(2) != 1 or t.stride(1) != t.shape[2] for t in (q, k, v)):
        return None
    if st != sum(widths) or len({t.untyped_storage().data_ptr() for t in (q, k, v)}) != 1:
        return None
    if k.data_ptr() != q.data_ptr() + widths[0] * e or v.data_ptr() != k.data_ptr() + widths[1] * e:
        return None
    return st


def _tt(t: torch.Tensor):
    return _lib.TTTensor(t.data_ptr(), t.stride(0), t.stride(1))


def gdn_tree_backward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
                      d_o: torch.Tensor, tree: GdnTree, scale: Optional[float] = None, l2norm: bool = True,
                      saved: Optional[torch.Tensor] = None, reference_truncated: bool = False,
                      initial_state: Optional[torch.Tensor] = None, d_states: Optional[torch.Tensor] = None,
                      initial_state_grad: bool = False, d_last_state: Optional[torch.Tensor] = None):
    """Gradients of sum(o * d_o) + sum(node_states * d_states) for
    ``gdn_tree_forward``'s outputs: dq, dk [T, Hk, 128] and dv [T, Hv, 128]
    in the dtype of v, dg and dbeta [T, Hv] float32, and with
    ``initial_state_grad`` also that of the initial state [Hv, 128, 128]
    (float32). ``d_states`` [n_nodes, Hv, 128, 128] may be None (no gradient
    reaches the node states); ``d_last_state`` [Hv, 128, 128] instead gives
    the gradient of the last node's state alone (no [n_nodes, ...] buffer).
    When q, k, v are the column blocks of one packed row buffer (the q/k/v
    split of a conv output), dq, dk, dv are the same column blocks of one new
    buffer, so the split's backward needs no concatenation. Recomputes the
    forward internally (tt_gdn_tree_bwd) unless ``saved`` holds what
    tt_gdn_tree_fwd_save kept for the same inputs (tt_gdn_tree_bwd_saved)."""
    p, (q, k, v, g, beta, _s0) = _problem(q, k, v, g, beta, tree, scale, l2norm, reference_truncated,
                                          initial_state)
    d_o = _tok_heads(d_o, "d_o").to(v.dtype)
    T, Hk, Hv = q.shape[0], q.shape[1], v.shape[1]
    if d_o.shape != v.shape:
        raise ValueError(f"d_o: expected {tuple(v.shape)}, got {tuple(d_o.shape)}")
    dev = require_device(q.device)
    W = _packed_qkv_width(q, k, v)
    if W is not None:
        rows = torch.empty((T, W), dtype=v.dtype, device=dev)
        nk = Hk * HEAD_DIM
        dq = rows[:, :nk].view(T, Hk, HEAD_DIM)
        dk = rows[:, nk:2 * nk].view(T, Hk, HEAD_DIM)
        dv = rows[:, 2 * nk:].view(T, Hv, HEAD_DIM)
    else:
        dq = torch.empty((T, Hk, HEAD_DIM), dtype=v.dtype, device=dev)
        dk = torch.empty_like(dq)
        dv = torch.empty((T, Hv, HEAD_DIM), dtype=v.dtype, device=dev)
    dg = torch.empty((T, Hv), dtype=torch.float32, device=dev)
    dbeta = torch.empty_like(dg)
    if d_states is not None and d_last_state is not None:
        raise ValueError("give d_states or d_last_state, not both")
    if d_last_state is not None:
        ds = _f32_block(d_last_state, (Hv, HEAD_DIM, HEAD_DIM), "d_last_state")
        p.d_states_last_only = 1
    else:
        ds = _f32_block(d_states, (tree.n_nodes, Hv, HEAD_DIM, HEAD_DIM), "d_states")
    if ds is not None and ds.device != dev:
        raise ValueError("d_states must be on the device of q, k, v")
    d_init = torch.empty((Hv, HEAD_DIM, HEAD_DIM), dtype=torch.float32, device=dev) if initial_state_grad else None
    lib = _lib.lib()
    outs = (_tt(d_o), _tt(dq), _tt(dk), _tt(dv), _ptr(dg), _ptr(dbeta), _ptr(ds), _ptr(d_init))
    if saved is not None:
        ws_bytes = lib.tt_gdn_bwd_saved_workspace_bytes(ctypes.byref(p))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        _lib.check(lib.tt_gdn_tree_bwd_saved(ctypes.byref(p), *outs, _ptr(saved), saved.numel(), _ptr(ws), ws_bytes,
                                             _stream(dev)), "tt_gdn_tree_bwd_saved")
    else:
        ws_bytes = lib.tt_gdn_bwd_workspace_bytes(ctypes.byref(p))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        _lib.check(lib.tt_gdn_tree_bwd(ctypes.byref(p), *outs, _ptr(ws), ws_bytes, _stream(dev)), "tt_gdn_tree_bwd")
    return (dq, dk, dv, dg, dbeta, d_init) if initial_state_grad else (dq, dk, dv, dg, dbeta)


class GdnTreeFunction(torch.autograd.Function):
    """Differentiable tree GDN: forward ``tt_gdn_tree_fwd_save`` (or
    ``tt_gdn_tree_fwd``), backward ``tt_gdn_tree_bwd_saved`` (or the
    recomputing ``tt_gdn_tree_bwd``), as ``KEEP_FORWARD_STATES`` says. Both
    outputs (o and the node states) carry gradients, and so does the
    optional initial state. With ``last_only`` the second output is the last
    node's state alone ([Hv, 128, 128]), whose gradient goes to the kernel as
    it is, without a zero-filled [n_nodes, ...] buffer around it."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, initial_state, tree, scale, l2norm, reference_truncated, last_only=False):
        keep = bool(KEEP_FORWARD_STATES)
        o, states, saved = _gdn_forward(q, k, v, g, beta, tree, scale, l2norm, keep, reference_truncated,
                                        initial_state)
        # The kept forward terms go through save_for_backward as well: autograd
        # then frees them with the graph (after a backward without retain_graph,
        # or when the graph is dropped), and every backward of a graph run
        # with retain_graph (the reference's per-leaf schedule) reuses them.
        ctx.save_for_backward(q, k, v, g, beta, initial_state, *(() if saved is None else (saved,)))
        ctx.tree, ctx.scale, ctx.l2norm, ctx.trunc = tree, scale, l2norm, reference_truncated
        ctx.last_only = last_only
        # No zero-filled gradient is made for an output the loss does not use.
        ctx.set_materialize_grads(False)
        return o, (states[-1].clone() if last_only else states)

    @staticmethod
    def backward(ctx, d_o, d_states):
        if d_o is None and d_states is None:
            return (None,) * 11
        q, k, v, g, beta, s0, *kept = ctx.saved_tensors
        if d_o is None:
            d_o = torch.zeros(v.shape, dtype=v.dtype, device=v.device)
        want_init = s0 is not None and ctx.needs_input_grad[5]
        res = gdn_tree_backward(q, k, v, g, beta, d_o, ctx.tree, ctx.scale, ctx.l2norm,
                                saved=kept[0] if kept else None, reference_truncated=ctx.trunc, initial_state=s0,
                                d_states=None if ctx.last_only else d_states, initial_state_grad=want_init,
                                d_last_state=d_states if ctx.last_only else None)
        dq, dk, dv, dg, dbeta = res[:5]
        d_init = res[5].reshape(s0.shape).to(s0.dtype) if want_init else None
        return (dq.reshape(q.shape).to(q.dtype), dk.reshape(k.shape).to(k.dtype), dv.reshape(v.shape).to(v.dtype),
                dg.reshape(g.shape).to(g.dtype), dbeta.reshape(beta.shape).to(beta.dtype), d_init,
                None, None, None, None, None)


def gdn_tree(q, k, v, g, beta, tree: GdnTree, scale: Optional[float] = None, l2norm: bool = True,
             reference_truncated: bool = False, initial_state: Optional[torch.Tensor] = None,
             last_state_only: bool = False):
    """Autograd-aware ``gdn_tree_forward``: (o, node_states), differentiable
    in q, k, v, g, beta and ``initial_state`` ([Hv, 128, 128], or [1, Hv,
    128, 128]; every root's state, zero when None). When any input requires
    a gradient and ``KEEP_FORWARD_STATES`` is set, the forward keeps its chunk
    terms and states for the backward. ``last_state_only``: the second output
    is the last node's state [Hv, 128, 128] instead of all node states."""
    ins = (q, k, v, g, beta) + (() if initial_state is None else (initial_state,))
    if not (torch.is_grad_enabled() and any(t.requires_grad for t in ins)):
        o, states = gdn_tree_forward(q, k, v, g, beta, tree, scale, l2norm, reference_truncated, initial_state)
        return o, (states[-1] if last_state_only else states)
    return GdnTreeFunction.apply(q, k, v, g, beta, initial_state, tree, scale, l2norm, bool(reference_truncated),
                                 bool(last_state_only))


def torch_chunk_gated_delta_rule_tree_varlen(query, key, value, g, beta, chunk_boundaries, chunk_parent_map,
                                             initial_state=None, output_final_state=False,
                                             use_qk_l2norm_in_kernel=False, reference_truncated=False):
    """Signature of tree_dfs_ssm.py:38-46, differentiable in q, k, v, g, beta
    and ``initial_state`` ([1, Hv, 128, 128], the state every root starts
    from; zero when None, tree_dfs_ssm.py:84-86). Returns (core_out [1, T, Hv,
    128], None or the last node's state [1, Hv, 128, 128], float32 and
    differentiable as tree_dfs_ssm.py:155). ``reference_truncated=True``
    gives the reference function's own numbers (I + R + R^2 per node) instead
    of the exact rule."""
    tree = GdnTree.from_boundaries(chunk_boundaries, chunk_parent_map, query.device)
    o, last = gdn_tree(query, key, value, g, beta, tree, l2norm=use_qk_l2norm_in_kernel,
                       reference_truncated=reference_truncated, initial_state=initial_state, last_state_only=True)
    last = last[None] if output_final_state else None
    return o[None], last
