"""Tree-masked GQA attention as a torch.autograd.Function over the HIP kernels.

Drop-in replacement for the attention core the reference hands to
transformers — ``repeat_kv`` + ``F.scaled_dot_product_attention`` with the dense
additive tree mask, and autograd's backward of it (transformers
integrations/sdpa_attention.py:79-175 as called by Qwen3Attention,
models/qwen3/modeling_qwen3.py:262-276) — plus the gateway concatenation of
``GatewayCache.update`` (tree_grad_ckpt_opath.py:92-114): the gateway K/V are
a second key segment read in place.

Layouts follow transformers: q [1, Hq, N, D], k/v [1, Hkv, N, D] (any strides
with D contiguous), output [1, N, Hq, D] contiguous. Gateway K/V are
[1, Hkv, Lp, D]. When a gateway accumulator is given, gateway gradients are
added to it in float32 on the device and no gradient is returned for the
gateway tensors — the contract of the fp32 hooks of tree_grad_hybrid.py:220-225
(accumulate in fp32, suppress the low-precision ``.grad``), without the host
round trip.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from ._lib import (TT_BWD_DETERMINISTIC, TT_DTYPE_BF16, TT_DTYPE_F32, TreeAttnError, TTAttnProblem, TTTensor,
                   check, lib)
from .meta import KeyPlan, _ptr, _stream

_DTYPES = {torch.bfloat16: TT_DTYPE_BF16, torch.float32: TT_DTYPE_F32}


def _layout(x: torch.Tensor, tok_dim: int, head_dim: int) -> Tuple[torch.Tensor, int, int]:
    """4-D tensor with a contiguous last (head-dim) axis -> (tensor,
    stride_tok, stride_head) in elements; copies only when the kernels' 16-byte
    vector alignment would not hold. Strides of size-1 axes are never used."""
    if x.dim() != 4 or x.shape[0] != 1:
        raise TreeAttnError(f"expected a 4-D tensor with batch 1, got shape {tuple(x.shape)}")

    def stride(t, d):
        return t.stride(d) if t.shape[d] > 1 else t.shape[3]

    def ok(t):
        return (t.stride(3) == 1 and t.data_ptr() % 16 == 0
                and all(stride(t, d) % 8 == 0 and stride(t, d) >= t.shape[3] for d in (tok_dim, head_dim)))

    if not ok(x):
        x = x.contiguous()
    return x, stride(x, tok_dim), stride(x, head_dim)


def _hf_view(x: torch.Tensor) -> Tuple[torch.Tensor, int, int]:
    """[1, H, T, D] (transformers layout)."""
    return _layout(x, 2, 1)


def _tok_view(x: torch.Tensor) -> Tuple[torch.Tensor, int, int]:
    """[1, T, H, D] (attention-output layout)."""
    return _layout(x, 1, 2)


class _Problem:
    """Builds the C problem struct for one call (keeps tensors alive)."""

    def __init__(self, q, k, v, kp, vp, plan: KeyPlan, scale: float):
        if q.dtype not in _DTYPES:
            raise TreeAttnError(f"unsupported dtype {q.dtype}; the engine is built for bf16 and fp32")
        for t in (k, v, kp, vp):
            if t is not None and t.dtype != q.dtype:
                raise TreeAttnError("q, k, v and gateway tensors must share one dtype")
        q, qst, qsh = _hf_view(q)
        k, kst, ksh = _hf_view(k)
        v, vst, vsh = _hf_view(v)
        n_past = 0
        kpt = vpt = TTTensor(None, 128, 128)
        if kp is not None:
            kp, kpst, kpsh = _hf_view(kp)
            vp, vpst, vpsh = _hf_view(vp)
            n_past = kp.shape[2]
            kpt = TTTensor(kp.data_ptr(), kpst, kpsh)
            vpt = TTTensor(vp.data_ptr(), vpst, vpsh)
        N, Hq, D = q.shape[2], q.shape[1], q.shape[3]
        if k.shape[2] != N or v.shape[2] != N:
            raise TreeAttnError("k/v must have the same token count as q (own segment)")
        if n_past != plan.n_past or N != plan.n_q:
            raise TreeAttnError(f"plan built for n_q={plan.n_q}, n_past={plan.n_past}; "
                                f"got n_q={N}, n_past={n_past}")
        self.keep = (q, k, v, kp, vp, plan)
        self.N, self.Hq, self.Hkv, self.D, self.n_past = N, Hq, k.shape[1], D, n_past
        self.dtype = q.dtype
        self.s = TTAttnProblem(
            dtype=_DTYPES[q.dtype], n_q=N, n_past=n_past, n_heads_q=Hq, n_heads_kv=k.shape[1],
            head_dim=D, scale=float(scale), bwd_parts=0,
            q=TTTensor(q.data_ptr(), qst, qsh), k=TTTensor(k.data_ptr(), kst, ksh),
            v=TTTensor(v.data_ptr(), vst, vsh), k_past=kpt, v_past=vpt,
            key_lo=plan.key_lo.data_ptr(), key_hi=plan.key_hi.data_ptr(), plan=plan.plan.data_ptr(),
            plan_bytes=plan.plan_bytes)


def fwd_workspace(pb: "_Problem", device) -> Optional[torch.Tensor]:
    """The forward's workspace (key-split partials of small bf16 problems), or
    None when the problem needs none."""
    n = lib().tt_attn_fwd_workspace_bytes(ctypes.byref(pb.s))
    return torch.empty(n, dtype=torch.uint8, device=device) if n else None


def attn_forward(q, k, v, plan: KeyPlan, scale: float, k_past=None, v_past=None):
    """Returns (o [N, Hq, D], lse [Hq, N] float32)."""
    pb = _Problem(q, k, v, k_past, v_past, plan, scale)
    o = torch.empty((pb.N, pb.Hq, pb.D), dtype=pb.dtype, device=q.device)
    lse = torch.empty((pb.Hq, pb.N), dtype=torch.float32, device=q.device)
    ws = fwd_workspace(pb, q.device)
    check(lib().tt_attn_fwd(ctypes.byref(pb.s), _ptr(o), _ptr(lse), _ptr(ws) if ws is not None else None,
                            ws.numel() if ws is not None else 0, _stream(q.device)), "tt_attn_fwd")
    return o, lse


def attn_backward(q, k, v, plan: KeyPlan, scale: float, o, lse, d_o, k_past=None, v_past=None,
                  gate_acc=None, parts=(0,), deterministic: Optional[bool] = None):
    """Returns (dq [N,Hq,D], dk [N,Hkv,D], dv [N,Hkv,D]); gateway grads are
    added to ``gate_acc`` when given. ``parts``: the ``bwd_parts`` of one
    ``tt_attn_bwd`` call each, run in order (default: one call, every part).
    ``deterministic`` (default: ``torch.are_deterministic_algorithms_enabled()``)
    adds TT_BWD_DETERMINISTIC: bitwise-repeatable dk/dv and gateway sums (both dtypes)."""
    if deterministic is None:
        deterministic = torch.are_deterministic_algorithms_enabled()
    det = TT_BWD_DETERMINISTIC if deterministic else 0
    pb = _Problem(q, k, v, k_past, v_past, plan, scale)
    pb.s.bwd_parts = det
    pb.s.split_tiles = plan.split_tiles()
    if det:
        pb.s.det_slots = plan.det_slots()
    dev = q.device
    d_o = d_o.reshape(1, pb.N, pb.Hq, pb.D) if d_o.dim() != 4 else d_o
    d_o, dst, dsh = _tok_view(d_o)
    dq = torch.empty((pb.N, pb.Hq, pb.D), dtype=pb.dtype, device=dev)
    dk = torch.empty((pb.N, pb.Hkv, pb.D), dtype=pb.dtype, device=dev)
    dv = torch.empty((pb.N, pb.Hkv, pb.D), dtype=pb.dtype, device=dev)
    # the workspace a call needs depends on its parts (the dQ pass's key-split
    # partials, the deterministic slots of the dK/dV pass): size it for the
    # largest of the calls
    ws_bytes = 0
    for part in parts:
        pb.s.bwd_parts = part | det
        ws_bytes = max(ws_bytes, lib().tt_attn_bwd_workspace_bytes(ctypes.byref(pb.s)))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    acc_k = acc_v = None
    if gate_acc is not None and pb.n_past > 0:
        acc_k, acc_v = gate_acc
        for a in (acc_k, acc_v):
            if a.dtype != torch.float32 or not a.is_contiguous() or a.numel() != pb.n_past * pb.Hkv * pb.D:
                raise TreeAttnError("gateway accumulators must be contiguous float32 [Lp, Hkv, D]")
    for part in parts:
        pb.s.bwd_parts = part | det
        rc = lib().tt_attn_bwd(ctypes.byref(pb.s), _ptr(o), _ptr(lse), TTTensor(d_o.data_ptr(), dst, dsh),
                               _ptr(dq), _ptr(dk), _ptr(dv), _ptr(acc_k), _ptr(acc_v), _ptr(ws), ws_bytes,
                               _stream(dev))
        check(rc, "tt_attn_bwd")
    return dq, dk, dv


class TreeAttnFunction(torch.autograd.Function):
    """Autograd node of one tree-attention call; re-entrant under repeated
    ``backward(retain_graph=True)`` with partial upstream gradients."""

    @staticmethod
    def forward(ctx, q, k, v, k_past, v_past, plan, scale, gate_acc):
        o, lse = attn_forward(q, k, v, plan, scale, k_past, v_past)
        ctx.save_for_backward(q, k, v, k_past, v_past, o, lse)
        ctx.plan, ctx.scale, ctx.gate_acc = plan, scale, gate_acc
        return o.view(1, *o.shape)

    @staticmethod
    def backward(ctx, g_o):
        q, k, v, k_past, v_past, o, lse = ctx.saved_tensors
        N, Hq, D = o.shape
        Hkv = k.shape[1]
        gate_acc = ctx.gate_acc
        acc = None
        own_acc = False
        if k_past is not None:
            if gate_acc is not None:
                gate_acc.touched = True
                acc = (gate_acc.k, gate_acc.v)
            elif ctx.needs_input_grad[3] or ctx.needs_input_grad[4]:
                Lp = k_past.shape[2]
                acc = (torch.zeros((Lp, Hkv, D), dtype=torch.float32, device=q.device),
                       torch.zeros((Lp, Hkv, D), dtype=torch.float32, device=q.device))
                own_acc = True
        dq, dk, dv = attn_backward(q, k, v, ctx.plan, ctx.scale, o, lse, g_o, k_past, v_past, acc)
        dq = dq.view(1, N, Hq, D).transpose(1, 2)
        dk = dk.view(1, N, Hkv, D).transpose(1, 2)
        dv = dv.view(1, N, Hkv, D).transpose(1, 2)
        dkp = dvp = None
        if own_acc:
            Lp = k_past.shape[2]
            dkp = acc[0].to(k_past.dtype).view(1, Lp, Hkv, D).transpose(1, 2)
            dvp = acc[1].to(v_past.dtype).view(1, Lp, Hkv, D).transpose(1, 2)
        return dq, dk, dv, dkp, dvp, None, None, None


def tree_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, plan: KeyPlan, scale: float,
                   k_past: Optional[torch.Tensor] = None, v_past: Optional[torch.Tensor] = None,
                   gate_acc=None) -> torch.Tensor:
    """Tree-masked attention: returns [1, N, Hq, D] (the HF attention output).

    ``gate_acc`` (a ``gateway.GatewayAccumulator``) receives the gateway
    gradients in float32; without it, gateway tensors that require grad get
    their gradient through autograd in their own dtype."""
    return TreeAttnFunction.apply(q, k, v, k_past, v_past, plan, float(scale), gate_acc)
