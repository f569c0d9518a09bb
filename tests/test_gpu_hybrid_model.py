"""End to end on a hybrid model: dfs_tree_forward over a two-layer
Qwen3.5-MoE text model (one gated-delta-rule layer, one full-attention layer)
against separate per-path forwards of the same model in float64 on the CPU,
the equivalence the reference's tree forward is built to keep (every leaf
sees exactly its root-to-leaf path).

The per-path oracle runs transformers' own modules with its gated-delta-rule
core (``torch_chunk_gated_delta_rule``, float32 inside) replaced by the
float64 exact recurrence of oracle/gdn.py (pinned against that routine in
tests/test_oracle_gdn.py). Checked: leaf logits and the gradients of the sum
of leaf cross entropies with respect to every parameter.

Bars: float32 leaf logits and parameter gradients max_rel < 1e-5, except the
two per-head gate parameters A_log and dt_bias (4 values each), < 5e-5: each is
a full reduction over tokens and heads of terms of both signs that carry the
float32 rounding of both layers, so cancellation magnifies it (measured
1.9e-5 and 1.3e-5 here; the single-layer test holds them to 1e-5).
"""
import copy

import pytest
import torch
import torch.nn.functional as F

from oracle import gdn as ogdn
from oracle.attention import max_rel
from tests.conftest import forest_from_spec, load_golden

pytestmark = pytest.mark.gpu
qmod = pytest.importorskip("transformers.models.qwen3_5_moe.modeling_qwen3_5_moe")
from tests.gdn_layer_util import small_hybrid_model  # noqa: E402

DEV = torch.device("cuda", 0)


def _gdn64(query, key, value, g, beta, initial_state=None, output_final_state=False, use_qk_l2norm_in_kernel=False,
           **kwargs):
    assert initial_state is None and query.shape[0] == 1
    T = query.shape[1]
    o = ogdn.gdn_tree_torch(query[0].double(), key[0].double(), value[0].double(), g[0].double(),
                            beta[0].double(), [T], [-1], l2=use_qk_l2norm_in_kernel)
    return o[None].to(value.dtype), None


def _path_tokens(node, parent_of):
    toks = []
    while node is not None:
        toks = list(node.token_ids) + toks
        node = parent_of.get(id(node))
    return toks


def test_hybrid_model_dfs_tree_forward_matches_per_path_fp32(monkeypatch):
    from tree_training_amd.dfs_tree_forward import dfs_tree_forward
    from tree_training_amd.tree import TreeNode
    spec = load_golden("c1_tree.json")
    roots, nodes = forest_from_spec(spec["nodes"], TreeNode)
    leaves = [n for n in nodes if not n.children]
    parent_of = {id(c): n for n in nodes for c in n.children}
    base = small_hybrid_model(3)
    ref = copy.deepcopy(base).double()
    model = base.to(DEV)
    for n in nodes:                      # token ids inside the small vocabulary
        n.token_ids = [t % 64 for t in n.token_ids]
    g = torch.Generator().manual_seed(7)
    labels = {id(n): torch.randint(0, 64, (len(n.token_ids),), generator=g) for n in leaves}
    print(f"hybrid model tree: {sum(len(n.token_ids) for n in nodes)} tokens, {len(leaves)} leaves", flush=True)

    res = dfs_tree_forward(model, roots)
    assert [id(n) for n in res.leaf_nodes] == [id(n) for n in leaves]
    loss = sum(F.cross_entropy(lg[0], labels[id(n)].to(DEV)) for lg, n in zip(res.leaf_logits, res.leaf_nodes))
    model.zero_grad(set_to_none=True)
    loss.backward()

    monkeypatch.setattr(qmod, "torch_chunk_gated_delta_rule", _gdn64)
    ref.zero_grad(set_to_none=True)
    worst = 0.0
    for lg, n in zip(res.leaf_logits, res.leaf_nodes):
        toks = _path_tokens(n, parent_of)
        out = ref(input_ids=torch.tensor([toks]), position_ids=torch.arange(len(toks))[None], use_cache=False)
        leaf = out.logits[0, len(toks) - len(n.token_ids):]
        worst = max(worst, max_rel(leaf.detach().numpy(), lg[0].detach().double().cpu().numpy()))
        F.cross_entropy(leaf, labels[id(n)]).backward()
    print(f"  leaf logits max_rel {worst:.3e}", flush=True)
    assert worst < 1e-5
    gw = 0.0
    for (name, p), (_, pr) in zip(model.named_parameters(), ref.named_parameters()):
        if pr.grad is None:
            assert p.grad is None or not p.grad.any(), name
            continue
        r = max_rel(pr.grad.numpy(), p.grad.double().cpu().numpy())
        gw = max(gw, r)
        if r > 5e-6:
            print(f"  {name}: {r:.3e}", flush=True)
        bar = 5e-5 if name.endswith(("linear_attn.A_log", "linear_attn.dt_bias")) else 1e-5
        assert r < bar, (name, r)
    print(f"  param grads max_rel {gw:.3e}", flush=True)
