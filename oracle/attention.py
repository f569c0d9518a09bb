"""Oracle: dense-mask GQA attention forward/backward in float64 numpy.

Test infrastructure only. Restates the attention arithmetic the reference
hands to transformers: ``eager_attention_forward`` /
``sdpa_attention_forward`` (transformers models/qwen3/modeling_qwen3.py:185-207,
integrations/sdpa_attention.py:79-175) fed with the reference's dense additive
tree mask (dfs_tree_forward.py:548-550, tree_grad_hybrid.py:312-317):

    O_h = softmax(Q_h K_g^T * scale + M) V_g,   g = h // (Hq / Hkv)   (repeat_kv)

with the closed-form backward of softmax attention. Layouts are token-major:
q [N, Hq, D], k/v [Lk, Hkv, D], mask [N, Lk] bool (True = visible).
"""
from __future__ import annotations

import numpy as np


def _groups(Hq, Hkv):
    assert Hq % Hkv == 0
    return Hq // Hkv


def attn_fwd(q, k, v, mask, scale):
    """Returns (o [N,Hq,D] float64, lse [Hq,N] float64, natural log)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    N, Hq, D = q.shape
    Hkv = k.shape[1]
    rep = _groups(Hq, Hkv)
    o = np.zeros((N, Hq, D))
    lse = np.full((Hq, N), -np.inf)
    neg = ~mask
    for h in range(Hq):
        g = h // rep
        s = (q[:, h, :] @ k[:, g, :].T) * scale
        s[neg] = -np.inf
        m = s.max(axis=1, keepdims=True)
        m_safe = np.where(np.isfinite(m), m, 0.0)
        p = np.exp(s - m_safe)
        l = p.sum(axis=1, keepdims=True)
        l_safe = np.where(l > 0, l, 1.0)
        p = p / l_safe
        o[:, h, :] = p @ v[:, g, :]
        lse[h] = np.where(l[:, 0] > 0, m_safe[:, 0] + np.log(l_safe[:, 0]), -np.inf)
    return o, lse


def attn_bwd(q, k, v, mask, scale, do):
    """Returns (dq, dk, dv) in float64 for upstream gradient ``do`` [N,Hq,D]."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    do = np.asarray(do, np.float64)
    N, Hq, D = q.shape
    Hkv = k.shape[1]
    rep = _groups(Hq, Hkv)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    neg = ~mask
    for h in range(Hq):
        g = h // rep
        s = (q[:, h, :] @ k[:, g, :].T) * scale
        s[neg] = -np.inf
        m = s.max(axis=1, keepdims=True)
        m = np.where(np.isfinite(m), m, 0.0)
        p = np.exp(s - m)
        l = p.sum(axis=1, keepdims=True)
        p = p / np.where(l > 0, l, 1.0)
        dv[:, g, :] += p.T @ do[:, h, :]
        dp = do[:, h, :] @ v[:, g, :].T
        delta = (p * dp).sum(axis=1, keepdims=True)
        ds = p * (dp - delta)
        dq[:, h, :] = (ds @ k[:, g, :]) * scale
        dk[:, g, :] += (ds.T @ q[:, h, :]) * scale
    return dq, dk, dv


def key_interval_mask(key_lo, key_hi, n_q):
    """Dense [n_q, Lk] mask for per-key visible query intervals [lo, hi)."""
    lo = np.asarray(key_lo)[None, :]
    hi = np.asarray(key_hi)[None, :]
    i = np.arange(n_q)[:, None]
    return (lo <= i) & (i < hi)


def gateway_mask(own_mask, bias):
    """[N, Lp+N] mask: the gateway bias row broadcast over queries, then the
    in-partition mask (tree_grad_hybrid.py:312-317)."""
    N = own_mask.shape[0]
    bias = np.asarray(bias, dtype=np.float64)
    past = np.broadcast_to(np.isfinite(bias)[None, :], (N, len(bias)))
    return np.concatenate([past, own_mask], axis=1)


def max_rel(ref, new):
    """max|new - ref| / (max|ref| + 1e-12), the reference's metric
    (verify_hybrid.py:129-132)."""
    ref = np.asarray(ref, np.float64)
    new = np.asarray(new, np.float64)
    return float(np.abs(ref - new).max() / (np.abs(ref).max() + 1e-12))
