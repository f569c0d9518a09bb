"""Tree gated-delta-rule (GDN) oracle, float64 numpy — test infrastructure only.

What the reference computes for the linear-attention layers of a DFS-packed
tree, restated on the CPU:

* ``tree_conv`` — tree-correct depthwise causal conv + SiLU:
  R/tree_dfs_ssm.py:284-346 (twin R/dfs_tree_forward.py:191-246). Each node's
  left context is its parent's last K-1 *effective* inputs, zeros for a root.
* ``gdn_tree(mode="reference")`` — literal restatement of
  ``torch_chunk_gated_delta_rule_tree_varlen`` (R/tree_dfs_ssm.py:38-156, twin
  R/dfs_tree_forward.py:253-353): each whole node is one chunk, its state
  comes from the parent node's final state (`all_states[parent+1]`, :131-132),
  and the within-node correction is built from the *uncorrected* rows
  (:114-121), i.e. A = I + R + R^2.
* ``gdn_tree(mode="exact")`` — the gated delta rule itself, token by token, on
  every root-to-leaf path (the semantics the reference's docstring states,
  R/tree_dfs_ssm.py:49-52): the transformers recurrence
  ``torch_recurrent_gated_delta_rule`` (HF/models/qwen3_5_moe/
  modeling_qwen3_5_moe.py) continued from the parent's final state.
* ``gdn_tree(mode="chunked")`` — the exact rule in fixed-size chunks with the
  forward-substitution inverse T = (I - N)^-1 (the algebra of transformers'
  ``torch_chunk_gated_delta_rule``), which is what the HIP scan evaluates.

The two differ: (I - R)^-1 = I + R + R^2 + R^3 (I - R)^-1, so the reference
equals the exact rule for nodes of at most 3 tokens (R^3 = 0) and deviates by
the R^3 term otherwise.

Pinned by (tests/test_oracle_gdn.py): transformers' recurrent and chunked
gated-delta-rule routines (library; the recurrent one also from a given
initial state), per-path equivalence of the tree outputs, chunk-size
independence, the R^3 identity above, a tree cut below its root equalling its
subtrees run from the root's final state, central finite differences for the
torch restatements' gradients, and torch.nn.functional.conv1d on every
root-to-leaf path for the conv.
"""
from __future__ import annotations

import numpy as np


def l2norm(x, eps=1e-6):
    """x / sqrt(sum(x^2) + eps) over the last axis (transformers' l2norm)."""
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + eps)


def node_starts(node_len):
    s = np.zeros(len(node_len), dtype=np.int64)
    if len(node_len) > 1:
        s[1:] = np.cumsum(node_len)[:-1]
    return s


def gdn_recurrent(q, k, v, g, beta, state):
    """Token-by-token gated delta rule for one head.

    q, k [L, Dk] (normalised, q already scaled); v [L, Dv]; g, beta [L];
    state [Dk, Dv]. Returns (o [L, Dv], final state). Follows the per-token
    update of transformers' torch_recurrent_gated_delta_rule:
    S <- S e^g; S <- S + k (beta (v - S^T k))^T; o = S^T q.
    """
    S = np.array(state, dtype=np.float64, copy=True)
    o = np.zeros((q.shape[0], v.shape[1]))
    for t in range(q.shape[0]):
        S = S * np.exp(g[t])
        delta = (v[t] - k[t] @ S) * beta[t]
        S = S + np.outer(k[t], delta)
        o[t] = q[t] @ S
    return o, S


def _decay(G):
    """D[i, j] = exp(G_i - G_j) for j <= i, 0 above the diagonal."""
    diff = G[:, None] - G[None, :]
    return np.where(np.tril(np.ones((len(G), len(G)), dtype=bool)), np.exp(np.tril(diff)), 0.0)


def _chunk_step(q, k, v, g, beta, S, correction):
    """One chunk of the chunked gated delta rule for one head (q scaled).

    correction(N) returns the matrix applied to beta*v and beta*k*e^G; the
    exact rule uses (I - N)^-1, the reference uses I + N + N^2 (with N the
    strictly lower matrix -(beta k k^T) * D).
    """
    L = q.shape[0]
    G = np.cumsum(g)
    D = _decay(G)
    N = -np.tril((beta[:, None] * k) @ k.T * D, -1)
    A = correction(N)
    u = A @ (beta[:, None] * v)
    w = A @ (beta[:, None] * k * np.exp(G)[:, None])
    vn = u - w @ S
    att = np.tril(q @ k.T * D)
    o = (q * np.exp(G)[:, None]) @ S + att @ vn
    S_new = S * np.exp(G[-1]) + (k * np.exp(G[-1] - G)[:, None]).T @ vn
    return o, S_new


def exact_correction(N):
    return np.linalg.inv(np.eye(N.shape[0]) - N)


def truncated_correction(N):
    """I + N + N^2: R/tree_dfs_ssm.py:114-121 (row j += raw[j,:j] @ raw[:j,:])."""
    L = N.shape[0]
    rows = [N[0:1, :]]
    for j in range(1, L):
        rows.append(N[j:j + 1, :] + N[j:j + 1, :j] @ N[:j, :])
    return np.concatenate(rows, axis=0) + np.eye(L)


def gdn_tree(q, k, v, g, beta, node_len, parent, mode="exact", chunk=64, l2=True, initial_state=None):
    """Tree gated delta rule over a DFS-packed forest.

    q, k [T, Hk, Dk]; v [T, Hv, Dv]; g, beta [T, Hv]; nodes in DFS pre-order
    (parent[i] < i, -1 for roots). v head h reads q/k head h // (Hv // Hk)
    (the reference's repeat_interleave). q, k are l2-normalised when ``l2``
    and q is scaled by Dk^-1/2 (R/tree_dfs_ssm.py:70-90). ``initial_state``
    [Hv, Dk, Dv]: the state every root starts from (zeros when None; the
    reference's ``all_states[0]``, R/tree_dfs_ssm.py:84-90).

    Returns (o [T, Hv, Dv], final states [n_nodes, Hv, Dk, Dv]).
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    g = np.asarray(g, np.float64)
    beta = np.asarray(beta, np.float64)
    T, Hk, Dk = q.shape
    Hv, Dv = v.shape[1], v.shape[2]
    rep = Hv // Hk
    if l2:
        q, k = l2norm(q), l2norm(k)
    q = q * Dk ** -0.5
    starts = node_starts(node_len)
    n = len(node_len)
    o = np.zeros((T, Hv, Dv))
    finals = np.zeros((n, Hv, Dk, Dv))
    for i in range(n):
        s0, L = int(starts[i]), int(node_len[i])
        sl = slice(s0, s0 + L)
        for h in range(Hv):
            hk = h // rep
            if parent[i] >= 0:
                S = finals[parent[i], h]
            elif initial_state is not None:
                S = np.asarray(initial_state[h], np.float64)
            else:
                S = np.zeros((Dk, Dv))
            qi, ki, vi, gi, bi = q[sl, hk], k[sl, hk], v[sl, h], g[sl, h], beta[sl, h]
            if mode == "exact":
                oi, S = gdn_recurrent(qi, ki, vi, gi, bi, S)
            elif mode == "reference":
                oi, S = _chunk_step(qi, ki, vi, gi, bi, S, truncated_correction)
            elif mode == "chunked":
                parts = []
                for c0 in range(0, L, chunk):
                    c1 = min(L, c0 + chunk)
                    oc, S = _chunk_step(qi[c0:c1], ki[c0:c1], vi[c0:c1], gi[c0:c1], bi[c0:c1], S,
                                        exact_correction)
                    parts.append(oc)
                oi = np.concatenate(parts, axis=0)
            else:
                raise ValueError(mode)
            o[sl, h] = oi
            finals[i, h] = S
    return o, finals


def tree_conv(x, weight, bias, node_len, parent):
    """Tree-correct depthwise causal conv + SiLU.

    x [T, C] (token-major), weight [C, K], bias [C] or None. Each node sees
    [parent's last K-1 effective inputs | its own inputs] (zeros before a
    root); out[t, c] = silu(bias[c] + sum_i weight[c, i] * ext[t + i]) with
    ext the K-1 context followed by the node (R/tree_dfs_ssm.py:306-346).
    """
    x = np.asarray(x, np.float64)
    w = np.asarray(weight, np.float64)
    C, K = w.shape
    starts = node_starts(node_len)
    out = np.zeros_like(x)
    ctx = {}
    for i in range(len(node_len)):
        s0, L = int(starts[i]), int(node_len[i])
        c = ctx[parent[i]] if parent[i] >= 0 else np.zeros((K - 1, C))
        ext = np.concatenate([c, x[s0:s0 + L]], axis=0)
        y = np.zeros((L, C))
        for j in range(K):
            y += ext[j:j + L] * w[:, j]
        if bias is not None:
            y += np.asarray(bias, np.float64)
        out[s0:s0 + L] = y / (1.0 + np.exp(-y))
        # the last K-1 rows (the reference slices ext[-(K-1):], which for K = 1
        # is the whole of ext: its kernel-size-1 case is not well formed, so the
        # empty context is taken explicitly here)
        ctx[i] = ext[len(ext) - (K - 1):]
    return out


def gdn_gates(a, b, A_log, dt_bias):
    """beta = sigmoid(b), g = -exp(A_log) * softplus(a + dt_bias)
    (R/tree_dfs_ssm.py:396-397)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    beta = 1.0 / (1.0 + np.exp(-b))
    z = a + np.asarray(dt_bias, np.float64)
    sp = np.where(z > 20.0, z, np.log1p(np.exp(np.minimum(z, 20.0))))
    g = -np.exp(np.asarray(A_log, np.float64)) * sp
    return g, beta


def gdn_tree_torch(q, k, v, g, beta, node_len, parent, l2=True, eps=1e-6, initial_state=None,
                   return_states=False):
    """The exact tree gated delta rule (token recurrence, as ``gdn_tree``
    mode="exact") in torch, differentiable: the backward oracle (autograd on
    float64). q, k [T, Hk, Dk]; v [T, Hv, Dv]; g, beta [T, Hv];
    ``initial_state`` [Hv, Dk, Dv] (every root's state, zeros when None, as
    R/tree_dfs_ssm.py:84-86). Returns o, and with ``return_states`` also the
    node final states [n_nodes, Hv, Dk, Dv]."""
    import torch
    T, Hk, Dk = q.shape
    Hv, Dv = v.shape[1], v.shape[2]
    rep = Hv // Hk
    if l2:
        q = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + eps)
        k = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + eps)
    q = q * Dk ** -0.5
    q = q.repeat_interleave(rep, dim=1)
    k = k.repeat_interleave(rep, dim=1)
    starts = node_starts(node_len)
    finals = [None] * len(node_len)
    outs = []
    for i in range(len(node_len)):
        S = finals[parent[i]] if parent[i] >= 0 else _root_state(initial_state, Hv, Dk, Dv, q.dtype)
        for t in range(int(starts[i]), int(starts[i] + node_len[i])):
            S = S * torch.exp(g[t])[:, None, None]
            delta = (v[t] - torch.einsum("hk,hkv->hv", k[t], S)) * beta[t][:, None]
            S = S + k[t][:, :, None] * delta[:, None, :]
            outs.append(torch.einsum("hk,hkv->hv", q[t], S))
        finals[i] = S
    out = torch.stack(outs, 0)
    return (out, torch.stack(finals)) if return_states else out


def _root_state(initial_state, Hv, Dk, Dv, dtype):
    import torch
    if initial_state is None:
        return torch.zeros(Hv, Dk, Dv, dtype=dtype)
    return initial_state


def gdn_tree_reference_torch(q, k, v, g, beta, node_len, parent, l2=True, eps=1e-6, return_states=False,
                             initial_state=None):
    """The reference's own evaluation (``gdn_tree`` mode="reference": every
    whole node one chunk, within-node correction A = I + R + R^2 built from
    the uncorrected rows, R/tree_dfs_ssm.py:100-150) in torch, differentiable:
    the backward oracle of that mode (autograd on float64). Same arguments and
    result as ``gdn_tree_torch`` (plus the node final states [n_nodes, Hv, Dk,
    Dv] with ``return_states``; ``initial_state`` as there); in the inputs'
    dtype, so float32 inputs give the precision the reference's own float32
    code reaches."""
    import torch
    T, Hk, Dk = q.shape
    Hv, Dv = v.shape[1], v.shape[2]
    rep = Hv // Hk
    if l2:
        q = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + eps)
        k = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + eps)
    q = (q * Dk ** -0.5).repeat_interleave(rep, dim=1).transpose(0, 1)    # [Hv, T, Dk]
    k = k.repeat_interleave(rep, dim=1).transpose(0, 1)
    v = v.transpose(0, 1)
    g, beta = g.transpose(0, 1), beta.transpose(0, 1)                     # [Hv, T]
    starts = node_starts(node_len)
    finals = [None] * len(node_len)
    outs = []
    for i in range(len(node_len)):
        s0, L = int(starts[i]), int(node_len[i])
        qi, ki, vi = q[:, s0:s0 + L], k[:, s0:s0 + L], v[:, s0:s0 + L]
        gi, bi = g[:, s0:s0 + L], beta[:, s0:s0 + L]
        S = finals[parent[i]] if parent[i] >= 0 else _root_state(initial_state, Hv, Dk, Dv, q.dtype)
        G = gi.cumsum(-1)
        lower = torch.tril(torch.ones(L, L, dtype=torch.bool))
        D = torch.where(lower, torch.exp(torch.where(lower, G[:, :, None] - G[:, None, :], 0.0)), 0.0)
        R = -torch.tril((bi[:, :, None] * ki) @ ki.transpose(1, 2) * D, -1)
        A = torch.eye(L, dtype=q.dtype) + R + R @ R
        u = A @ (bi[:, :, None] * vi)
        w = A @ (bi[:, :, None] * ki * torch.exp(G)[:, :, None])
        vn = u - w @ S
        o = (qi * torch.exp(G)[:, :, None]) @ S + (qi @ ki.transpose(1, 2) * D) @ vn
        finals[i] = S * torch.exp(G[:, -1])[:, None, None] + \
            (ki * torch.exp(G[:, -1:] - G)[:, :, None]).transpose(1, 2) @ vn
        outs.append(o)
    out = torch.cat(outs, 1).transpose(0, 1)
    return (out, torch.stack(finals)) if return_states else out


def token_prev(node_len, parent):
    """Path predecessor of every token: t - 1 inside a node, the parent's
    last token for a node's first token, -1 before a root."""
    starts = node_starts(node_len)
    prev = np.arange(-1, int(sum(node_len)) - 1)
    for i, p in enumerate(parent):
        prev[starts[i]] = starts[p] + node_len[p] - 1 if p >= 0 else -1
    return prev


def tree_conv_torch(x, weight, bias, node_len, parent):
    """``tree_conv`` written over token predecessor chains in torch,
    differentiable (the backward oracle): y[t] = silu(b + sum_i w[:, i] *
    x[prev^(K-1-i)(t)]). x [T, C], weight [C, K], bias [C] or None."""
    import torch
    T, C = x.shape
    K = weight.shape[1]
    prev = torch.from_numpy(token_prev(node_len, parent))
    idx = torch.arange(T)
    acc = bias.expand(T, C) if bias is not None else torch.zeros(T, C, dtype=x.dtype)
    xz = torch.cat([x, torch.zeros(1, C, dtype=x.dtype)], 0)      # row T is the zero row
    for m in range(K):
        sel = torch.where(idx >= 0, idx, torch.full_like(idx, T))
        acc = acc + weight[:, K - 1 - m] * xz[sel]
        idx = torch.where(idx >= 0, prev[idx.clamp(min=0)], idx)
    return acc * torch.sigmoid(acc)


def gdn_layer_torch(ssm, hidden, node_len, parent, reference_truncated=False):
    """The tree-aware GatedDeltaNet layer in float64 torch, differentiable:
    projections, ``tree_conv_torch``, gates, ``gdn_tree_torch`` (exact rule,
    q/k heads shared by Hv/Hk v heads), gated RMSNorm and out_proj, with the
    parameters of ``ssm`` (a transformers Qwen3_5MoeGatedDeltaNet, whose
    attributes this reads: the layer of R/tree_dfs_ssm.py:355-423 and
    R/dfs_tree_forward.py:360-435). hidden [T, d] float64; the module's
    parameters are used in float64. ``reference_truncated`` takes the
    reference's own I + R + R^2 scan instead of the exact rule. Returns [T, d]."""
    import torch
    P = {n: p.double() for n, p in ssm.named_parameters()}
    lin = lambda x, n: x @ P[n + ".weight"].T
    mixed = lin(hidden, "in_proj_qkv")
    z = lin(hidden, "in_proj_z")
    b = lin(hidden, "in_proj_b")
    a = lin(hidden, "in_proj_a")
    cb = P.get("conv1d.bias")
    mixed = tree_conv_torch(mixed, P["conv1d.weight"][:, 0, :], cb, node_len, parent)
    T = hidden.shape[0]
    q, k, v = torch.split(mixed, [ssm.key_dim, ssm.key_dim, ssm.value_dim], dim=-1)
    q = q.reshape(T, -1, ssm.head_k_dim)
    k = k.reshape(T, -1, ssm.head_k_dim)
    v = v.reshape(T, -1, ssm.head_v_dim)
    beta = torch.sigmoid(b)
    g = -torch.exp(P["A_log"]) * torch.nn.functional.softplus(a + P["dt_bias"])
    scan = gdn_tree_reference_torch if reference_truncated else gdn_tree_torch
    o = scan(q, k, v, g, beta, node_len, parent)
    o = o.reshape(-1, ssm.head_v_dim)
    zz = z.reshape(-1, ssm.head_v_dim)
    o = o * torch.rsqrt(o.pow(2).mean(-1, keepdim=True) + ssm.norm.variance_epsilon)
    o = P["norm.weight"] * o * (zz * torch.sigmoid(zz))
    return lin(o.reshape(T, -1), "out_proj")
