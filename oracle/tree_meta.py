"""Oracle: DFS tree metadata (test infrastructure only).

Restates ``build_dfs_tree_info`` of the reference two ways:
  * ``build_dfs_tree_info_literal`` — the literal loops of
    dfs_tree_forward.py:91-184 (pure Python; small trees only);
  * ``meta_closed_form`` — numpy closed form  mask[i, j] <=> j <= i < h[j],
    where h[j] is the exclusive end token of the subtree of the node holding
    token j (DFS pre-order makes every subtree one contiguous token range).

Both accept any duck-typed node with ``token_ids`` and ``children``.
"""
from __future__ import annotations

import numpy as np


def flatten_forest(roots):
    """DFS pre-order flattening, dfs_tree_forward.py:113-139.

    Returns (node_len, parent, nodes) with parent[c] < c, -1 for a root.
    """
    node_len, parent, nodes = [], [], []

    def _dfs(node, par):
        me = len(nodes)
        nodes.append(node)
        node_len.append(len(node.token_ids))
        parent.append(par)
        for ch in node.children:
            _dfs(ch, me)

    for r in roots:
        _dfs(r, -1)
    return node_len, parent, nodes


def build_dfs_tree_info_literal(roots):
    """Literal restatement of build_dfs_tree_info, dfs_tree_forward.py:91-184.

    Returns a dict with the reference's DFSTreeInfo fields; ``attn_mask_bool``
    is a numpy bool [N, N] array built by the reference's per-pair loop
    (dfs_tree_forward.py:161-172).
    """
    dfs_token_ids, dfs_pos_ids = [], []
    chunk_boundaries, chunk_parent_map = [], []
    leaf_chunk_ids, leaf_nodes = [], []
    counter = [0]

    def _dfs(node, parent_chunk, depth_offset):          # :113-136
        my_chunk = counter[0]
        counter[0] += 1
        c_start = len(dfs_token_ids)
        dfs_token_ids.extend(node.token_ids)
        L = len(node.token_ids)
        for j in range(L):
            dfs_pos_ids.append(depth_offset + j)        # :125-126
        chunk_parent_map.append(parent_chunk)
        chunk_boundaries.append((c_start, c_start + L))
        if len(node.children) == 0:
            leaf_chunk_ids.append(my_chunk)
            leaf_nodes.append(node)
        else:
            for child in node.children:
                _dfs(child, my_chunk, depth_offset + L)

    for root in roots:                                   # :138-139
        _dfs(root, -1, 0)

    N = len(dfs_token_ids)
    n_chunks = len(chunk_parent_map)

    ancestors = [None] * n_chunks                        # :145-155

    def _anc(c):
        if ancestors[c] is not None:
            return ancestors[c]
        p = chunk_parent_map[c]
        ancestors[c] = [c] if p == -1 else _anc(p) + [c]
        return ancestors[c]

    for c in range(n_chunks):
        _anc(c)

    mask = np.zeros((N, N), dtype=bool)                  # :161-172
    for c in range(n_chunks):
        c_start, c_end = chunk_boundaries[c]
        for anc in ancestors[c]:
            a_start, a_end = chunk_boundaries[anc]
            for i in range(c_start, c_end):
                if anc == c:
                    for j in range(c_start, i + 1):
                        mask[i, j] = True
                else:
                    for j in range(a_start, a_end):
                        mask[i, j] = True

    return dict(dfs_token_ids=dfs_token_ids, dfs_pos_ids=dfs_pos_ids,
                chunk_boundaries=chunk_boundaries, chunk_parent_map=chunk_parent_map,
                attn_mask_bool=mask, leaf_chunk_ids=leaf_chunk_ids,
                leaf_nodes=leaf_nodes, N=N, n_chunks=n_chunks)


def meta_closed_form(node_len, parent, pos_offset=0):
    """Closed-form metadata from DFS pre-order (node_len, parent).

    Returns dict of numpy int64 arrays:
      node_start[n], node_off[n] (depth offset), node_hend[n] (subtree end token),
      pos[T] (= pos_offset + node_off + j), node_of[T], horizon[T].
    Follows dfs_tree_forward.py:113-139 (positions) and the subtree-contiguity of
    pre-order for the horizon.
    """
    node_len = np.asarray(node_len, dtype=np.int64)
    parent = np.asarray(parent, dtype=np.int64)
    n = len(node_len)
    start = np.concatenate([[0], np.cumsum(node_len)[:-1]]) if n else np.zeros(0, np.int64)
    T = int(node_len.sum())
    off = np.zeros(n, np.int64)
    for c in range(n):                 # parent < child, so one forward pass
        p = parent[c]
        if p >= 0:
            off[c] = off[p] + node_len[p]
    hend = start + node_len            # subtree end: max end over descendants
    for c in range(n - 1, -1, -1):
        p = parent[c]
        if p >= 0:
            hend[p] = max(hend[p], hend[c])
    node_of = np.repeat(np.arange(n, dtype=np.int64), node_len)
    j_in = np.arange(T, dtype=np.int64) - start[node_of]
    pos = pos_offset + off[node_of] + j_in
    horizon = hend[node_of]
    return dict(node_start=start, node_off=off, node_hend=hend, pos=pos,
                node_of=node_of, horizon=horizon, T=T)


def mask_from_horizon(horizon):
    """Dense [T, T] bool mask from the closed form  j <= i < h[j]."""
    h = np.asarray(horizon)
    T = len(h)
    i = np.arange(T)[:, None]
    j = np.arange(T)[None, :]
    return (j <= i) & (i < h[None, :])


def brute_force_mask(node_len, parent):
    """Mask by walking ancestor chains per token pair (tiny trees only)."""
    m = meta_closed_form(node_len, parent)
    node_of = m["node_of"]
    T = m["T"]

    def anc_or_self(c):
        out = set()
        while c >= 0:
            out.add(int(c))
            c = parent[c]
        return out

    anc = [anc_or_self(c) for c in range(len(node_len))]
    mask = np.zeros((T, T), dtype=bool)
    for i in range(T):
        for j in range(T):
            a, b = node_of[i], node_of[j]
            if b in anc[a] and (b != a or j <= i):
                mask[i, j] = True
    return mask
