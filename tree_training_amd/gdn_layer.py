"""Tree-aware forward for the gated-delta-rule (linear-attention) layers.

Drop-in for the reference's SSM layer patch: ``_make_dfs_ssm_forward`` /
``_patch_ssm`` / ``_unpatch_ssm`` (dfs_tree_forward.py:360-467) and
``_make_dfs_ssm_forward`` / ``patch_ssm_for_dfs`` / ``unpatch_ssm``
(tree_dfs_ssm.py:355-445). A patched ``Qwen3_5MoeGatedDeltaNet`` (or any
module with the same attributes: in_proj_qkv/z/b/a, conv1d, A_log, dt_bias,
norm, out_proj, key_dim, value_dim, head_k_dim, head_v_dim) runs:

  projections   one GEMM per projection over all T tokens (torch), or with
                per_node_projections one per tree node, as the reference
  conv          tt_tree_conv_fwd / _bwd (each node's window reaches into its
                ancestors' last K-1 inputs), token-major rows; q, k, v are
                its column blocks and their gradients come back as the same
                blocks of one buffer (no concatenation)
  gates         beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias) (torch)
  scan          tt_gdn_tree_fwd / _bwd (exact gated delta rule per root-to-leaf
                path, or with reference_truncated the reference function's
                own I + R + R^2 per node; v head h reads q/k head h / (Hv/Hk),
                the reference's repeat_interleave, without materialising it)
  output        the module's own RMSNormGated and out_proj over all tokens
                (per node with per_node_projections)

The reference projects node by node so that bf16 GEMM shapes match separate
per-path runs bit for bit (tree_dfs_ssm.py:369-373, 416-428). By default each
projection here is one GEMM over all tokens (fewer, larger GEMMs), so the tree
output agrees with per-path runs to bf16 rounding; ``per_node_projections=True``
runs them node by node as the reference does, and the tree output then equals
per-path runs of the same nodes bit for bit (the conv and the scan already do).
``cache_params`` is ignored, as in the reference (the tree forward runs with
use_cache=False).
"""
from __future__ import annotations

from typing import Dict, Sequence, Tuple

import torch
import torch.nn.functional as F

from .conv import tree_conv
from .gdn import GdnTree, gdn_tree


def _per_node(fn, tree: GdnTree, *xs: torch.Tensor) -> torch.Tensor:
    """fn applied to each node's rows of xs [T, ...], the results stacked back
    in token order (one GEMM shape per node, as a per-path run has)."""
    return torch.cat([fn(*(x[s:s + n] for x in xs)) for s, n in zip(tree.node_start, tree.node_len)], dim=0)


def _tree_ssm_forward(ssm, hidden_states: torch.Tensor, tree: GdnTree, reference_truncated: bool = False,
                      per_node_projections: bool = False) -> torch.Tensor:
    B, S, _ = hidden_states.shape
    if B != 1:
        raise ValueError("the tree forward packs one forest per batch row; batch size must be 1")
    if S != tree.n_tokens:
        raise ValueError(f"{S} tokens but the tree holds {tree.n_tokens}")
    h = hidden_states[0]
    if per_node_projections:
        mixed = _per_node(ssm.in_proj_qkv, tree, h)              # [T, conv_dim]
        z = _per_node(ssm.in_proj_z, tree, h)                    # [T, value_dim]
        b = _per_node(ssm.in_proj_b, tree, h)
        a = _per_node(ssm.in_proj_a, tree, h)
    else:
        mixed = ssm.in_proj_qkv(h)
        z = ssm.in_proj_z(h)
        b = ssm.in_proj_b(h)
        a = ssm.in_proj_a(h)
    q, k, v = tree_conv(mixed, ssm.conv1d.weight, ssm.conv1d.bias, tree,
                        split_sizes=(ssm.key_dim, ssm.key_dim, ssm.value_dim))
    q = q.reshape(S, -1, ssm.head_k_dim)
    k = k.reshape(S, -1, ssm.head_k_dim)
    v = v.reshape(S, -1, ssm.head_v_dim)
    beta = b.sigmoid()
    g = -ssm.A_log.float().exp() * F.softplus(a.float() + ssm.dt_bias)
    o, _ = gdn_tree(q, k, v, g, beta, tree, None, True, reference_truncated)   # [T, Hv, Dv]
    Dv = ssm.head_v_dim
    if per_node_projections:
        def node_out(o_n, z_n):
            return ssm.out_proj(ssm.norm(o_n.reshape(-1, Dv), z_n.reshape(-1, Dv)).reshape(len(o_n), -1))
        return _per_node(node_out, tree, o, z)[None]
    o = ssm.norm(o.reshape(-1, Dv), z.reshape(-1, Dv))
    return ssm.out_proj(o.reshape(1, S, -1))


class _LazyTree:
    """The GdnTree of a forest, built on the device of the first call and
    shared by every layer patched together."""

    def __init__(self, chunk_boundaries, chunk_parent_map):
        self.bounds = [tuple(b) for b in chunk_boundaries]
        self.parent = list(chunk_parent_map)
        self.trees = {}

    def on(self, device) -> GdnTree:
        key = str(device)
        if key not in self.trees:
            self.trees[key] = GdnTree.from_boundaries(self.bounds, self.parent, device)
        return self.trees[key]


def _make_dfs_ssm_forward(ssm_layer, chunk_boundaries: Sequence[Tuple[int, int]], chunk_parent_map: Sequence[int],
                          tree: _LazyTree = None, reference_truncated: bool = False,
                          per_node_projections: bool = False):
    """Patched forward for one GatedDeltaNet layer (dfs_tree_forward.py:360,
    tree_dfs_ssm.py:355). ``tree`` may be shared by all layers of a model."""
    tree = tree or _LazyTree(chunk_boundaries, chunk_parent_map)

    def patched_forward(hidden_states, cache_params=None, cache_position=None, attention_mask=None, **kwargs):
        return _tree_ssm_forward(ssm_layer, hidden_states, tree.on(hidden_states.device), reference_truncated,
                                 per_node_projections)

    return patched_forward


def _ssm_layers(model):
    return [layer.linear_attn for layer in model.model.layers if hasattr(layer, "linear_attn")]


def _patch_ssm(model, chunk_boundaries, chunk_parent_map, reference_truncated: bool = False,
               per_node_projections: bool = False) -> Dict:
    """Patch every GatedDeltaNet layer (dfs_tree_forward.py:442-462): the
    accelerate-wrapped ``_old_forward`` when present, else ``forward``.
    Returns what ``_unpatch_ssm`` restores."""
    saved = {}
    tree = _LazyTree(chunk_boundaries, chunk_parent_map)
    for ssm in _ssm_layers(model):
        patched = _make_dfs_ssm_forward(ssm, chunk_boundaries, chunk_parent_map, tree, reference_truncated,
                                        per_node_projections)
        attr = "_old_forward" if hasattr(ssm, "_old_forward") else "forward"
        saved[ssm] = (attr, ssm.__dict__.get(attr, None))
        setattr(ssm, attr, patched)
    return saved


def _unpatch_ssm(saved: Dict) -> None:
    """Restore what ``_patch_ssm`` replaced (dfs_tree_forward.py:465-467)."""
    for ssm, (attr, orig) in saved.items():
        if orig is None:
            ssm.__dict__.pop(attr, None)       # the class method shows through again
        else:
            setattr(ssm, attr, orig)


def patch_ssm_for_dfs(model, chunk_boundaries, chunk_parent_map, reference_truncated: bool = False,
                      per_node_projections: bool = False) -> Dict:
    """tree_dfs_ssm.py:432 name for ``_patch_ssm``."""
    return _patch_ssm(model, chunk_boundaries, chunk_parent_map, reference_truncated, per_node_projections)


def unpatch_ssm(saved: Dict) -> None:
    """tree_dfs_ssm.py:442 name for ``_unpatch_ssm``."""
    _unpatch_ssm(saved)
