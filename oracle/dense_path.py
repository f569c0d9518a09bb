"""Oracle: the reference's dense-mask attention path on the CPU, in torch.

Test infrastructure and CPU baseline only. Restates, op for op, what one
attention layer of the reference executes for a DFS-packed tree:
  1. additive mask [1,1,N,Lp+N] in the model dtype: -inf everywhere, the
     gateway bias broadcast over rows, 0 on the in-partition tree mask
     (dfs_tree_forward.py:548-550; tree_grad_hybrid.py:312-317);
  2. repeat_kv 8 -> 32 heads and F.scaled_dot_product_attention with the
     float mask and scale = d**-0.5 (transformers integrations/sdpa_attention.py:79-175,
     models/qwen3/modeling_qwen3.py:173-182);
  3. autograd for the backward.
Inputs use the transformers layout: q [1,Hq,N,D], k/v [1,Hkv,Lk,D].
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def additive_mask(mask_bool, dtype, past_bias=None):
    """[1,1,N,Lp+N] additive mask (0 visible, -inf blocked)."""
    N = mask_bool.shape[0]
    Lp = 0 if past_bias is None else int(past_bias.numel())
    m = torch.full((1, 1, N, Lp + N), float("-inf"), dtype=dtype)
    if Lp:
        m[0, 0, :, :Lp] = past_bias.to(dtype)
    m[0, 0, :, Lp:][mask_bool] = 0.0
    return m


def repeat_kv(x, n_rep):
    """transformers models/qwen3/modeling_qwen3.py:173-182."""
    b, hkv, s, d = x.shape
    if n_rep == 1:
        return x
    return x[:, :, None, :, :].expand(b, hkv, n_rep, s, d).reshape(b, hkv * n_rep, s, d)


def dense_tree_attention(q, k, v, add_mask, scale):
    """Forward of the dense path; returns [1, N, Hq, D] like the HF bridge."""
    rep = q.shape[1] // k.shape[1]
    kk = repeat_kv(k, rep)
    vv = repeat_kv(v, rep)
    o = F.scaled_dot_product_attention(q, kk, vv, attn_mask=add_mask, scale=scale)
    return o.transpose(1, 2).contiguous()


def dense_fwd_bwd(q, k, v, add_mask, scale, do):
    """One forward + full backward of the dense path (the timed CPU baseline)."""
    q = q.detach().requires_grad_(True)
    k = k.detach().requires_grad_(True)
    v = v.detach().requires_grad_(True)
    o = dense_tree_attention(q, k, v, add_mask, scale)
    o.backward(do)
    return o.detach(), q.grad, k.grad, v.grad
