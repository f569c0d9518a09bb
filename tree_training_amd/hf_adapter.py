"""transformers integration: the ``"tree_hip"`` attention implementation.

The reference feeds transformers a dense additive 4-D mask and lets
``Qwen3Attention`` call SDPA (dfs_tree_forward.py:548-560,
tree_grad_hybrid.py:312-317,396-402). Here the drivers switch the model's
``config._attn_implementation`` to ``"tree_hip"`` for the duration of the call
(restored in ``finally``, as the reference restores its SSM patches) and pass a
``TreeAttnContext`` through ``model(..., tree_ctx=ctx)``. transformers builds no
mask for an implementation it has no mask function for
(masking_utils.py ``_preprocess_mask_arguments``), and forwards the keyword to
every attention call (models/qwen3/modeling_qwen3.py:266-276), which lands in
``tree_hip_attention``.
"""
from __future__ import annotations

import contextlib
from dataclasses import dataclass
from typing import Optional

from ._lib import TreeAttnError
from .attention import tree_attention
from .meta import KeyPlan

ATTN_IMPL = "tree_hip"
_registered = False


@dataclass
class TreeAttnContext:
    """Per-forward state shared by every attention layer."""
    plan: KeyPlan
    cache: Optional[object] = None          # GatewayCache (segmented) or None
    accumulators: Optional[list] = None     # per-layer GatewayAccumulator for the gateway grads


def tree_hip_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """transformers attention-interface function (returns (out [1,N,Hq,D], None))."""
    ctx = kwargs.get("tree_ctx")
    if ctx is None:
        raise TreeAttnError("the tree_hip attention needs tree metadata: call it through "
                            "dfs_tree_forward / tree_grad_ckpt_sequential / tree_grad_hybrid")
    if dropout:
        raise TreeAttnError("attention dropout is not supported by the tree attention kernels")
    layer = getattr(module, "layer_idx", 0)
    kp = vp = acc = None
    if ctx.cache is not None:
        kp, vp = ctx.cache.gate(layer)
        if kp is not None and ctx.accumulators is not None:
            acc = ctx.accumulators[layer]
    scale = scaling if scaling is not None else query.shape[-1] ** -0.5
    out = tree_attention(query, key, value, ctx.plan, scale, kp, vp, acc)
    return out, None


def register():
    """Registers ``"tree_hip"`` with transformers' AttentionInterface (idempotent)."""
    global _registered
    if _registered:
        return
    from transformers import AttentionInterface
    AttentionInterface.register(ATTN_IMPL, tree_hip_attention)
    _registered = True


def _has_linear_attention(model) -> bool:
    for m in model.modules():
        if hasattr(m, "linear_attn"):
            return True
    return False


@contextlib.contextmanager
def tree_attention_mode(model, linear_attention_patched: bool = False, fused_prologue: bool = True):
    """Switches every attention layer of ``model`` to the tree kernels for the
    duration of the block, and (``fused_prologue``) every Qwen3Attention to the
    fused q/k RMSNorm + rotary prologue (``prologue.py``). Gated-delta-rule
    (linear_attn) layers must have been patched with the tree-aware forward
    (``gdn_layer._patch_ssm``, done by dfs_tree_forward); the partitioned
    drivers do not carry their recurrent state across partitions and refuse
    such models (dfs_tree_forward and tree_grad_ckpt_sequential patch them)."""
    from .prologue import patch_attention_prologue, unpatch_attention_prologue
    register()
    if not linear_attention_patched and _has_linear_attention(model):
        raise NotImplementedError("gated-delta-rule (linear_attn) layers are supported by dfs_tree_forward and "
                                  "tree_grad_ckpt_sequential, not by the partitioned drivers")
    cfg = model.config
    saved = cfg._attn_implementation
    cfg._attn_implementation = ATTN_IMPL
    patched = patch_attention_prologue(model) if fused_prologue else []
    try:
        yield
    finally:
        unpatch_attention_prologue(patched)
        cfg._attn_implementation = saved
