"""Fused attention prologue: q/k RMSNorm + rotary embedding in one HIP pass.

Qwen3Attention (HF/models/qwen3/modeling_qwen3.py:241-280) normalises the
projected q and k per head (q_norm / k_norm, :252-253), rotates them with the
model's cos/sin table (:256-257) and hands [B, H, T, D] transposed views to the
attention function: several elementwise passes over q and k in each direction.
``fused_qwen3_attention_forward`` replaces that stretch with
``tt_qk_prologue_fwd`` / ``tt_qk_prologue_bwd`` (include/tree_attn.h), which
read the projections once and write q and k in the [T, H, 128] layout the tree
attention kernels read; the projections, the cache update and o_proj are the
module's own. ``tree_attention_mode`` installs it on every Qwen3Attention for
the duration of a tree forward.
"""
from __future__ import annotations

import ctypes
import types
from typing import Optional

import torch

from . import _lib
from .meta import _ptr, _stream, require_device

HEAD_DIM = 128


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return _lib.TT_DTYPE_BF16
    if t.dtype == torch.float32:
        return _lib.TT_DTYPE_F32
    raise ValueError(f"unsupported dtype {t.dtype} (bfloat16 or float32)")


def _rows(x: torch.Tensor, name: str) -> torch.Tensor:
    if x.dim() != 3 or x.shape[-1] != HEAD_DIM:
        raise ValueError(f"{name}: expected [T, H, {HEAD_DIM}], got {tuple(x.shape)}")
    if x.stride(-1) != 1 or x.data_ptr() % 16 or x.stride(0) % 8 or x.stride(1) % 8:
        x = x.contiguous()
    return x


def _tensor(x: torch.Tensor):
    return _lib.TTTensor(x.data_ptr(), x.stride(0), x.stride(1))


def _problem(q, k, qw, kw, eps_q, eps_k, cos, sin):
    q, k = _rows(q, "q"), _rows(k, "k")
    if k.shape[0] != q.shape[0] or k.dtype != q.dtype:
        raise ValueError("q and k disagree in tokens or dtype")
    T = q.shape[0]
    cos = cos.reshape(-1, HEAD_DIM)
    sin = sin.reshape(-1, HEAD_DIM)
    if cos.shape[0] != T or sin.shape[0] != T:
        raise ValueError(f"cos/sin: expected [{T}, {HEAD_DIM}], got {tuple(cos.shape)}")
    cos = cos.to(q.dtype).contiguous()
    sin = sin.to(q.dtype).contiguous()
    qw = qw.to(q.dtype).contiguous()
    kw = kw.to(q.dtype).contiguous()
    p = _lib.TTPrologueProblem(dtype=_dtype_code(q), n_tokens=T, n_heads_q=q.shape[1], n_heads_kv=k.shape[1],
                               head_dim=HEAD_DIM, eps_q=float(eps_q), eps_k=float(eps_k), q=_tensor(q),
                               k=_tensor(k), q_weight=qw.data_ptr(), k_weight=kw.data_ptr(), cos=cos.data_ptr(),
                               sin=sin.data_ptr(), cs_stride_tok=HEAD_DIM)
    return p, (q, k, qw, kw, cos, sin)


def qk_prologue_forward(q, k, q_weight, k_weight, eps_q, eps_k, cos, sin):
    """(q_out [T, Hq, 128], k_out [T, Hkv, 128]) contiguous, dtype of q."""
    p, keep = _problem(q, k, q_weight, k_weight, eps_q, eps_k, cos, sin)
    q, k = keep[0], keep[1]
    dev = require_device(q.device)
    qo = torch.empty(q.shape, dtype=q.dtype, device=dev)
    ko = torch.empty(k.shape, dtype=k.dtype, device=dev)
    _lib.check(_lib.lib().tt_qk_prologue_fwd(ctypes.byref(p), _ptr(qo), _ptr(ko), _stream(dev)),
               "tt_qk_prologue_fwd")
    return qo, ko


def qk_prologue_backward(q, k, q_weight, k_weight, eps_q, eps_k, cos, sin, dq_out, dk_out):
    """(dq [T, Hq, 128], dk [T, Hkv, 128] in q's dtype, dq_weight, dk_weight
    [128] float32)."""
    p, keep = _problem(q, k, q_weight, k_weight, eps_q, eps_k, cos, sin)
    q, k = keep[0], keep[1]
    dq_out, dk_out = _rows(dq_out.to(q.dtype), "dq_out"), _rows(dk_out.to(q.dtype), "dk_out")
    dev = require_device(q.device)
    dq = torch.empty(q.shape, dtype=q.dtype, device=dev)
    dk = torch.empty(k.shape, dtype=k.dtype, device=dev)
    dqw = torch.empty(HEAD_DIM, dtype=torch.float32, device=dev)
    dkw = torch.empty(HEAD_DIM, dtype=torch.float32, device=dev)
    lib = _lib.lib()
    ws_bytes = lib.tt_qk_prologue_bwd_workspace_bytes(ctypes.byref(p))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    _lib.check(lib.tt_qk_prologue_bwd(ctypes.byref(p), _tensor(dq_out), _tensor(dk_out), _ptr(dq), _ptr(dk),
                                      _ptr(dqw), _ptr(dkw), _ptr(ws), ws_bytes, _stream(dev)), "tt_qk_prologue_bwd")
    return dq, dk, dqw, dkw


class QKPrologueFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, q_weight, k_weight, eps_q, eps_k, cos, sin):
        ctx.save_for_backward(q, k, q_weight, k_weight, cos, sin)
        ctx.eps = (eps_q, eps_k)
        return qk_prologue_forward(q, k, q_weight, k_weight, eps_q, eps_k, cos, sin)

    @staticmethod
    def backward(ctx, dq_out, dk_out):
        q, k, qw, kw, cos, sin = ctx.saved_tensors
        dq, dk, dqw, dkw = qk_prologue_backward(q, k, qw, kw, ctx.eps[0], ctx.eps[1], cos, sin, dq_out, dk_out)
        return (dq.reshape(q.shape), dk.reshape(k.shape), dqw.to(qw.dtype), dkw.to(kw.dtype), None, None, None,
                None)


def qk_prologue(q, k, q_weight, k_weight, eps_q, eps_k, cos, sin):
    """Autograd-aware fused prologue: (q_out, k_out) [T, H, 128]."""
    return QKPrologueFunction.apply(q, k, q_weight, k_weight, eps_q, eps_k, cos, sin)


def fused_qwen3_attention_forward(self, hidden_states, position_embeddings, attention_mask, past_key_values=None,
                                  **kwargs):
    """Qwen3Attention.forward with the fused prologue (signature of
    HF/models/qwen3/modeling_qwen3.py:241-248); the attention call goes to the
    model's configured attention implementation, as in the original."""
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    B, T = hidden_states.shape[:2]
    if B != 1:
        raise ValueError("the tree forward packs one forest per batch row; batch size must be 1")
    h = hidden_states[0]
    q_raw = self.q_proj(h).view(T, -1, self.head_dim)
    k_raw = self.k_proj(h).view(T, -1, self.head_dim)
    v = self.v_proj(h).view(T, -1, self.head_dim)
    cos, sin = position_embeddings
    q, k = qk_prologue(q_raw, k_raw, self.q_norm.weight, self.k_norm.weight, self.q_norm.variance_epsilon,
                       self.k_norm.variance_epsilon, cos[0], sin[0])
    query_states = q[None].transpose(1, 2)
    key_states = k[None].transpose(1, 2)
    value_states = v[None].transpose(1, 2)
    if past_key_values is not None:
        key_states, value_states = past_key_values.update(key_states, value_states, self.layer_idx)
    from transformers.models.qwen3.modeling_qwen3 import eager_attention_forward
    attention_interface = ALL_ATTENTION_FUNCTIONS.get_interface(self.config._attn_implementation,
                                                               eager_attention_forward)
    attn_output, attn_weights = attention_interface(
        self, query_states, key_states, value_states, attention_mask,
        dropout=0.0 if not self.training else self.attention_dropout, scaling=self.scaling,
        sliding_window=getattr(self, "sliding_window", None), **kwargs)
    attn_output = attn_output.reshape(B, T, -1).contiguous()
    return self.o_proj(attn_output), attn_weights


def _is_qwen3_attention(m) -> bool:
    return (type(m).__name__ == "Qwen3Attention" and hasattr(m, "q_norm") and hasattr(m, "k_norm")
            and getattr(m, "head_dim", None) == HEAD_DIM)


def patch_attention_prologue(model) -> list:
    """Installs the fused forward on every Qwen3Attention of ``model``;
    returns what ``unpatch_attention_prologue`` restores."""
    saved = []
    for m in model.modules():
        if _is_qwen3_attention(m):
            saved.append((m, m.__dict__.get("forward")))
            m.forward = types.MethodType(fused_qwen3_attention_forward, m)
    return saved


def unpatch_attention_prologue(saved: list) -> None:
    for m, orig in saved:
        if orig is None:
            m.__dict__.pop("forward", None)
        else:
            m.forward = orig
