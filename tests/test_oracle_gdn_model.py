"""CPU pins of oracle.model_path.tree_gdn_layers on a two-layer Qwen3.5-MoE
text model (one gated-delta-rule layer, one full-attention layer), float64.

With the GatedDeltaNet layers patched over the DFS forest, the dense-mask
whole-tree forward (oracle.model_path.dense_leaf_logits) must give every leaf
the logits of a separate forward over its root-to-leaf path through
transformers' own modules, whose GDN core is the float64 exact recurrence
(pinned against transformers' own routines in tests/test_oracle_gdn.py).
The truncated scan (the reference's I + R + R^2 per node) equals the exact
rule when no node is longer than 3 tokens (R is strictly lower triangular,
R^3 = 0), so on such a forest the reference_truncated patch must match the
per-path forwards too; on longer nodes, with nearly parallel keys and slow
decay (gdn_layer_util.strong_recurrence), it must not.
Bar 1e-6: transformers' eager attention takes its softmax in float32 even in a
float64 model, which leaves ~1e-7 between two float64 runs that order the
attention differently (dense tree mask vs one path).
"""
import copy

import pytest
import torch

from oracle import gdn as ogdn
from oracle.attention import max_rel
from oracle.model_path import dense_leaf_logits, tree_gdn_layers
from tests.conftest import forest_from_spec, load_golden

qmod = pytest.importorskip("transformers.models.qwen3_5_moe.modeling_qwen3_5_moe")
from tests.gdn_layer_util import small_hybrid_model, strong_recurrence  # noqa: E402


def _gdn64(query, key, value, g, beta, initial_state=None, output_final_state=False, use_qk_l2norm_in_kernel=False,
           **kwargs):
    T = query.shape[1]
    o = ogdn.gdn_tree_torch(query[0].double(), key[0].double(), value[0].double(), g[0].double(),
                            beta[0].double(), [T], [-1], l2=use_qk_l2norm_in_kernel)
    return o[None].to(value.dtype), None


def _forest(short):
    from tests.conftest import Node
    spec = load_golden("c1_tree.json")
    nodes_spec = spec["nodes"]
    if short:   # every node cut to at most 3 tokens
        nodes_spec = [dict(n, len=min(n["len"], 3)) for n in nodes_spec]
    roots, nodes = forest_from_spec(nodes_spec)
    for n in nodes:
        n.token_ids = [t % 64 for t in n.token_ids]
    return roots, nodes


def _per_path(model, nodes):
    parent_of = {id(c): n for n in nodes for c in n.children}
    out = {}
    for n in nodes:
        if n.children:
            continue
        toks, m = [], n
        while m is not None:
            toks = list(m.token_ids) + toks
            m = parent_of.get(id(m))
        lg = model(input_ids=torch.tensor([toks]), position_ids=torch.arange(len(toks))[None], use_cache=False).logits
        out[id(n)] = lg[0, len(toks) - len(n.token_ids):]
    return out


@pytest.mark.parametrize("short,truncated", [(False, False), (True, True)])
def test_tree_gdn_oracle_matches_per_path(monkeypatch, short, truncated):
    roots, nodes = _forest(short)
    model = strong_recurrence(small_hybrid_model(3)).double()
    with torch.no_grad():
        with tree_gdn_layers(model, roots, reference_truncated=truncated):
            leaf_logits, leaf_nodes = dense_leaf_logits(model, roots)
        monkeypatch.setattr(qmod, "torch_chunk_gated_delta_rule", _gdn64)
        ref = _per_path(model, nodes)
    worst = max(max_rel(ref[id(n)].numpy(), lg[0].numpy()) for lg, n in zip(leaf_logits, leaf_nodes))
    assert worst < 1e-6, worst


def test_tree_gdn_oracle_truncated_differs_on_long_nodes():
    roots, nodes = _forest(False)
    model = strong_recurrence(small_hybrid_model(3)).double()
    with torch.no_grad():
        with tree_gdn_layers(model, roots, reference_truncated=True):
            trunc, _ = dense_leaf_logits(model, roots)
        with tree_gdn_layers(model, roots, reference_truncated=False):
            exact, _ = dense_leaf_logits(model, roots)
    assert max(max_rel(a[0].numpy(), b[0].numpy()) for a, b in zip(exact, trunc)) > 1e-4
