"""Leaf loss without [T, V] logits: chunked lm_head + fused cross-entropy.

The reference scores leaves with ``F.cross_entropy(logits[0], labels,
ignore_index) / n_leaves`` (tree_grad_hybrid.py:546-558,
tree_grad_ckpt.py:280-297) on logits the model computed for every token of
the packed tree ([T, V]: ~5 GB in bf16 for a 16K tree and V = 151,936, plus
float32 temporaries). ``fused_linear_ce`` takes the final hidden states of the
leaf tokens only and, chunk by chunk, runs the lm_head GEMM, ``tt_ce_rows``
(loss and logit gradient in one HIP kernel, in place) and the two gradient
GEMMs, so at most one [chunk, V] block exists; the gradients of the hidden
states and of the lm_head weight are formed during the forward and scaled by
the incoming gradient in the backward.

``TreeCELoss`` is what ``make_tree_loss_fn`` returns: called as
``loss_fn(logits, node)`` it is exactly the reference's loss; the drivers
recognise it and take the fused path instead (``fused_leaf_ce``).
"""
from __future__ import annotations

import ctypes
from typing import List

import torch
import torch.nn.functional as F

from . import _lib
from .meta import _ptr, _stream, require_device, to_device


def ce_rows(logits: torch.Tensor, labels: torch.Tensor, row_scale: torch.Tensor, ignore_index: int = -100,
            grad: torch.Tensor = None) -> torch.Tensor:
    """Per-row weighted CE loss [N] (float32) of logits [N, V]; writes the
    logit gradient into ``grad`` (default: in place over ``logits``)."""
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits: expected [N, V] with unit column stride")
    N, V = logits.shape
    grad = logits if grad is None else grad
    dev = require_device(logits.device)
    lab = to_device(labels, dev, torch.int32)
    sc = to_device(row_scale, dev, torch.float32)
    loss = torch.empty(N, dtype=torch.float32, device=dev)
    code = _lib.TT_DTYPE_BF16 if logits.dtype == torch.bfloat16 else _lib.TT_DTYPE_F32
    if logits.dtype not in (torch.bfloat16, torch.float32) or grad.dtype != logits.dtype:
        raise ValueError("logits and grad must be bfloat16 or float32, the same")
    _lib.check(_lib.lib().tt_ce_rows(code, _ptr(logits), logits.stride(0), N, V, _ptr(lab), _ptr(sc), ignore_index,
                                     _ptr(loss), _ptr(grad), grad.stride(0), _stream(dev)), "tt_ce_rows")
    return loss


def _mm_f32(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a @ b with a float32 result straight from the GEMM (no rounding to the
    inputs' dtype in between)."""
    if a.dtype == torch.float32:
        return a @ b
    try:
        return torch.mm(a, b, out_dtype=torch.float32)
    except (RuntimeError, NotImplementedError, TypeError):
        return (a @ b).float()


class FusedLinearCE(torch.autograd.Function):
    """sum_r c_r CE(hidden_r W^T, y_r) with the gradients formed in the forward."""

    @staticmethod
    def forward(ctx, hidden, weight, labels, row_scale, ignore_index, chunk):
        N = hidden.shape[0]
        gh = torch.empty_like(hidden)
        gw = torch.zeros(weight.shape, dtype=torch.float32, device=weight.device)
        total = torch.zeros((), dtype=torch.float32, device=hidden.device)
        for c0 in range(0, N, chunk):
            h = hidden[c0:c0 + chunk]
            logits = h @ weight.t()                      # [n, V], the model dtype
            total += ce_rows(logits, labels[c0:c0 + chunk], row_scale[c0:c0 + chunk], ignore_index).sum()
            gh[c0:c0 + chunk] = logits @ weight          # logits now hold dL/dlogits
            gw += _mm_f32(logits.t(), h)
        ctx.save_for_backward(gh, gw)
        ctx.weight_dtype = weight.dtype
        return total

    @staticmethod
    def backward(ctx, g):
        gh, gw = ctx.saved_tensors
        return (gh * g.to(gh.dtype), (gw * g).to(ctx.weight_dtype), None, None, None, None)


def fused_linear_ce(hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor, row_scale: torch.Tensor,
                    ignore_index: int = -100, chunk: int = 4096) -> torch.Tensor:
    """Scalar sum_r row_scale[r] * CE(hidden[r] @ weight.T, labels[r])."""
    return FusedLinearCE.apply(hidden, weight, labels, row_scale, ignore_index, chunk)


class TreeCELoss:
    """``make_tree_loss_fn``'s result: CE(logits[0], labels, ignore_index) /
    n_leaves per leaf (tree_grad_hybrid.py:546-558)."""

    def __init__(self, leaf_labels: List[torch.Tensor], leaf_nodes, n_leaves: int, ignore_index: int = -100):
        self.label_map = {id(n): lab for n, lab in zip(leaf_nodes, leaf_labels)}
        self.n_leaves = n_leaves
        self.ignore_index = ignore_index

    def __call__(self, logits: torch.Tensor, node) -> torch.Tensor:
        labels = self.label_map[id(node)].to(logits.device)
        return F.cross_entropy(logits[0], labels, ignore_index=self.ignore_index) / self.n_leaves

    def fused_spans(self, hidden: torch.Tensor, spans, lm_head_weight: torch.Tensor) -> torch.Tensor:
        """Sum of the loss over leaves ``spans`` = [(start, end, node)] of the
        final hidden states ``hidden`` [T, H], through ONE ``fused_linear_ce``
        call over all their rows (one weight-gradient buffer, full chunks)."""
        dev = hidden.device
        rows, labels, scales, empty = [], [], [], False
        for s, e, node in spans:
            lab = self.label_map[id(node)].reshape(-1)
            n_valid = int((lab != self.ignore_index).sum())   # no device round trip for host labels
            empty = empty or n_valid == 0
            rows.append(torch.arange(s, e, device=dev))
            labels.append(lab)
            scales.append(torch.full((e - s,), 1.0 / (max(n_valid, 1) * self.n_leaves), dtype=torch.float32,
                                     device=dev))
        idx = torch.cat(rows)
        if all(lab.device.type == "cpu" for lab in labels):
            lab_all = to_device(torch.cat(labels), dev, torch.int32)
        else:
            lab_all = torch.cat([lab.to(dev) for lab in labels])
        loss = fused_linear_ce(hidden.index_select(0, idx), lm_head_weight, lab_all, torch.cat(scales),
                               self.ignore_index)
        return loss * float("nan") if empty else loss    # F.cross_entropy's mean over no tokens is NaN
