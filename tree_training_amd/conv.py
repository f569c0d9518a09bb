"""Tree-correct short convolution (depthwise causal conv + SiLU) on the GPU.

Drop-in for ``_tree_correct_conv_varlen`` (tree_dfs_ssm.py:284-346; twin
dfs_tree_forward.py:191-246): every node's conv window reaches into its
ancestors' last K-1 inputs (zeros before a root), as a run of its
root-to-node path alone would, computed by ``tt_tree_conv_fwd`` in one launch
over all tokens instead of one ``cat`` + conv launch per node. The backward
(``tt_tree_conv_bwd``) gives dx, dweight and dbias.

Rows are tokens (channels contiguous); the reference's [B, C, T] layout is
accepted by the drop-in and its result is returned as a [1, C, T] view of the
token-major output, the layout the q/k/v split after it reads.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import torch

from . import _lib
from .gdn import GdnTree
from .meta import _ptr, _stream, require_device


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return _lib.TT_DTYPE_BF16
    if t.dtype == torch.float32:
        return _lib.TT_DTYPE_F32
    raise ValueError(f"unsupported dtype {t.dtype} (bfloat16 or float32)")


def _rows(x: torch.Tensor, name: str) -> torch.Tensor:
    if x.dim() != 2:
        raise ValueError(f"{name}: expected [T, C], got {tuple(x.shape)}")
    if x.stride(1) != 1 or x.stride(0) % 4 or x.data_ptr() % 16:
        x = x.contiguous()
    return x


def _problem(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], tree: GdnTree):
    x = _rows(x, "x")
    T, C = x.shape
    if T != tree.n_tokens:
        raise ValueError(f"{T} tokens but the tree holds {tree.n_tokens}")
    w = weight.reshape(C, -1).to(x.dtype).contiguous()
    b = bias.to(x.dtype).contiguous() if bias is not None else None
    prev, off, nxt = tree.token_links()
    p = _lib.TTConvProblem(dtype=_dtype_code(x), n_tokens=T, n_channels=C, kernel_size=w.shape[1],
                           x=x.data_ptr(), x_stride_tok=x.stride(0), weight=w.data_ptr(),
                           bias=b.data_ptr() if b is not None else None, tok_prev=_ptr(prev),
                           tok_next_off=_ptr(off), tok_next=_ptr(nxt))
    return p, x, w, b


def tree_conv_forward(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                      tree: GdnTree) -> torch.Tensor:
    """y [T, C] = silu(tree-correct depthwise causal conv of x [T, C]); weight
    [C, K] or [C, 1, K], bias [C] or None."""
    p, x, w, b = _problem(x, weight, bias, tree)
    dev = require_device(x.device)
    y = torch.empty_like(x, memory_format=torch.contiguous_format)
    _lib.check(_lib.lib().tt_tree_conv_fwd(ctypes.byref(p), _ptr(y), y.stride(0), _stream(dev)), "tt_tree_conv_fwd")
    return y


def tree_conv_backward(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], dy: torch.Tensor,
                       tree: GdnTree):
    """(dx [T, C] in x's dtype, dweight [C, K] float32, dbias [C] float32 or None)."""
    p, x, w, b = _problem(x, weight, bias, tree)
    dy = _rows(dy.to(x.dtype), "dy")
    if dy.shape != x.shape:
        raise ValueError(f"dy: expected {tuple(x.shape)}, got {tuple(dy.shape)}")
    dev = require_device(x.device)
    T, C = x.shape
    dx = torch.empty((T, C), dtype=x.dtype, device=dev)
    dw = torch.empty((C, w.shape[1]), dtype=torch.float32, device=dev)
    db = torch.empty((C,), dtype=torch.float32, device=dev) if b is not None else None
    lib = _lib.lib()
    ws_bytes = lib.tt_tree_conv_bwd_workspace_bytes(ctypes.byref(p))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    _lib.check(lib.tt_tree_conv_bwd(ctypes.byref(p), _ptr(dy), dy.stride(0), _ptr(dx), _ptr(dw),
                                    _ptr(db) if db is not None else None, _ptr(ws), ws_bytes, _stream(dev)),
               "tt_tree_conv_bwd")
    return dx, dw, db


class TreeConvFunction(torch.autograd.Function):
    """Differentiable tree conv: forward ``tt_tree_conv_fwd``, backward
    ``tt_tree_conv_bwd``."""

    @staticmethod
    def forward(ctx, x, weight, bias, tree):
        ctx.save_for_backward(x, weight, bias)
        ctx.tree = tree
        return tree_conv_forward(x, weight, bias, tree)

    @staticmethod
    def backward(ctx, dy):
        x, weight, bias = ctx.saved_tensors
        dx, dw, db = tree_conv_backward(x, weight, bias, dy, ctx.tree)
        return (dx.to(x.dtype), dw.reshape(weight.shape).to(weight.dtype),
                db.to(bias.dtype) if bias is not None else None, None)


def _join_columns(grads, sizes: Sequence[int], like: torch.Tensor) -> torch.Tensor:
    """dy [T, sum(sizes)] from the gradients of the column blocks: read in
    place when they already are those blocks of one row-major buffer (what
    gdn_tree_backward writes for a q/k/v split), else concatenated (zeros for
    a block without a gradient)."""
    T, W = like.shape[0], sum(sizes)
    if all(g is not None for g in grads):
        g0 = grads[0]
        e, off, ok = g0.element_size(), 0, True
        for g, n in zip(grads, sizes):
            ok = ok and (g.dim() == 2 and g.shape == (T, n) and g.stride(1) == 1 and g.stride(0) == W and
                         g.dtype == g0.dtype and g.untyped_storage().data_ptr() == g0.untyped_storage().data_ptr()
                         and g.data_ptr() == g0.data_ptr() + off * e)
            off += n
        if ok and (g0.storage_offset() + T * W) * e <= g0.untyped_storage().nbytes():
            return g0.as_strided((T, W), (W, 1))
    return torch.cat([g if g is not None else torch.zeros((T, n), dtype=like.dtype, device=like.device)
                      for g, n in zip(grads, sizes)], dim=1)


class TreeConvSplitFunction(torch.autograd.Function):
    """Tree conv whose output rows are handed out as column blocks (the q/k/v
    split after the conv); the backward takes the blocks' gradients back as
    one dy through ``_join_columns``."""

    @staticmethod
    def forward(ctx, x, weight, bias, tree, sizes):
        ctx.save_for_backward(x, weight, bias)
        ctx.tree, ctx.sizes = tree, tuple(sizes)
        ctx.set_materialize_grads(False)
        y = tree_conv_forward(x, weight, bias, tree)
        if y.shape[1] != sum(ctx.sizes):
            raise ValueError(f"split sizes {ctx.sizes} do not add up to the {y.shape[1]} channels")
        return tuple(torch.split(y, ctx.sizes, dim=1))

    @staticmethod
    def backward(ctx, *grads):
        if all(g is None for g in grads):
            return None, None, None, None, None
        x, weight, bias = ctx.saved_tensors
        dy = _join_columns(grads, ctx.sizes, x)
        dx, dw, db = tree_conv_backward(x, weight, bias, dy, ctx.tree)
        return (dx.to(x.dtype), dw.reshape(weight.shape).to(weight.dtype),
                db.to(bias.dtype) if bias is not None else None, None, None)


def tree_conv(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], tree: GdnTree,
              split_sizes: Optional[Sequence[int]] = None):
    """Autograd-aware ``tree_conv_forward``. With ``split_sizes`` the output
    comes back as the tuple ``torch.split(y, split_sizes, dim=1)`` would give
    (views of one [T, C] buffer), and the backward reads the blocks'
    gradients in place when they are the matching blocks of one buffer (as
    ``gdn_tree`` gives for q, k, v taken from those blocks) instead of
    concatenating them."""
    if split_sizes is None:
        return TreeConvFunction.apply(x, weight, bias, tree)
    return TreeConvSplitFunction.apply(x, weight, bias, tree, tuple(int(n) for n in split_sizes))


def _tree_correct_conv_varlen(ssm, mixed_qkv_raw: torch.Tensor, chunk_boundaries, chunk_parent_map):
    """Signature of tree_dfs_ssm.py:284: ``mixed_qkv_raw`` [1, conv_dim, N]
    (raw projections), the ssm module supplies ``conv1d`` (weight [C, 1, K],
    bias or None). Returns [1, conv_dim, N] (a view of token-major rows)."""
    if mixed_qkv_raw.dim() != 3 or mixed_qkv_raw.shape[0] != 1:
        raise ValueError("mixed_qkv_raw: expected [1, conv_dim, N] (one packed tree)")
    if getattr(ssm, "activation", "silu") not in ("silu", "swish"):
        raise NotImplementedError(f"activation {ssm.activation!r}: only SiLU is built")
    tree = GdnTree.from_boundaries(chunk_boundaries, chunk_parent_map, mixed_qkv_raw.device)
    y = tree_conv(mixed_qkv_raw[0].transpose(0, 1), ssm.conv1d.weight, ssm.conv1d.bias, tree)
    return y.transpose(0, 1)[None]
