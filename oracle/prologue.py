"""Attention prologue oracle (q/k RMSNorm + rotary embedding), float64 torch —
test infrastructure only.

What transformers' Qwen3Attention does to the projected q and k before the
attention call (HF/models/qwen3/modeling_qwen3.py:252-257): per head,
``y = w * x / sqrt(mean(x^2) + eps)`` (Qwen3RMSNorm, :59-64), then
``y * cos + rotate_half(y) * sin`` with ``rotate_half(y) = [-y[64:], y[:64]]``
(:140-170), cos/sin being the model's rotary table at each token's position.
The reference feeds it the depth positions of the DFS tree
(R/dfs_tree_forward.py:543-560). Differentiable (autograd gives the backward).

Pinned by tests/test_oracle_prologue.py against transformers' own
Qwen3RMSNorm and apply_rotary_pos_emb (library) in float64, values and
gradients.
"""
from __future__ import annotations


def qk_prologue(x, weight, eps, cos, sin):
    """x [T, H, D] (projected q or k), weight [D], cos/sin [T, D]. Returns the
    normalised, rotated [T, H, D]."""
    import torch
    y = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * weight
    half = x.shape[-1] // 2
    rot = torch.cat([-y[..., half:], y[..., :half]], dim=-1)
    return y * cos[:, None, :] + rot * sin[:, None, :]
