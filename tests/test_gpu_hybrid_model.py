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

Bars: float32 leaf logits and every parameter gradient max_rel < 1e-5,
the gate parameters A_log, dt_bias and in_proj_a included: they are
reductions over tokens of the decay gradient dg, which the scan's backward
forms from exactly the pair terms that reach each token (no cancelling row
and column sums), so it keeps float32 accuracy relative to its own size.
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
        assert r < 1e-5, (name, r)
    print(f"  param grads max_rel {gw:.3e}", flush=True)


def _c1_forest():
    from tree_training_amd.tree import TreeNode
    spec = load_golden("c1_tree.json")
    roots, nodes = forest_from_spec(spec["nodes"], TreeNode)
    for n in nodes:
        n.token_ids = [t % 64 for t in n.token_ids]
    leaves = [n for n in nodes if not n.children]
    g = torch.Generator().manual_seed(7)
    labels = {id(n): torch.randint(0, 64, (len(n.token_ids),), generator=g) for n in leaves}
    return roots, nodes, leaves, labels


def _compare_grads(model, ref_grads):
    gw = 0.0
    for name, p in model.named_parameters():
        if name not in ref_grads:
            assert p.grad is None or not p.grad.any(), name
            continue
        r = max_rel(ref_grads[name].numpy(), p.grad.double().cpu().numpy())
        gw = max(gw, r)
        if r > 5e-6:
            print(f"  {name}: {r:.3e}", flush=True)
        assert r < 1e-5, (name, r)
    print(f"  param grads max_rel {gw:.3e}", flush=True)


@pytest.mark.parametrize("fused_ce", [True, False])
def test_hybrid_model_sequential_grads_match_per_path_fp32(monkeypatch, fused_ce):
    """tree_grad_ckpt_sequential on the hybrid model (its GDN layers patched
    with the tree-aware conv + scan for the forward and every per-leaf
    backward): parameter gradients of sum_leaf CE / n_leaves against the
    float64 per-path runs of transformers' own modules, < 1e-5.
    fused_ce False is the reference's schedule, one retain_graph backward per
    leaf through the GDN layer's autograd node."""
    from tree_training_amd.ckpt import make_tree_loss_fn, tree_grad_ckpt_sequential
    roots, nodes, leaves, labels = _c1_forest()
    parent_of = {id(c): n for n in nodes for c in n.children}
    base = small_hybrid_model(3)
    ref = copy.deepcopy(base).double()
    model = base.to(DEV)
    print(f"hybrid model sequential (fused_ce={fused_ce}): {len(leaves)} leaves", flush=True)
    model.zero_grad(set_to_none=True)
    fn = make_tree_loss_fn([labels[id(n)] for n in leaves], leaves, len(leaves))
    tree_grad_ckpt_sequential(model, roots, fn, fused_leaf_ce=fused_ce)
    torch.cuda.synchronize()

    monkeypatch.setattr(qmod, "torch_chunk_gated_delta_rule", _gdn64)
    ref.zero_grad(set_to_none=True)
    for n in leaves:
        toks = _path_tokens(n, parent_of)
        out = ref(input_ids=torch.tensor([toks]), position_ids=torch.arange(len(toks))[None], use_cache=False)
        (F.cross_entropy(out.logits[0, len(toks) - len(n.token_ids):], labels[id(n)]) / len(leaves)).backward()
    _compare_grads(model, {k: p.grad for k, p in ref.named_parameters() if p.grad is not None})


def test_hybrid_model_reference_literal_matches_truncated_oracle():
    """reference_literal=True on the hybrid model — the reference's truncated
    GDN scan (I + R + R^2 per node), node-by-node projections, transformers'
    own q/k norm + rotary and logits + cross-entropy — against the float64
    restatement of the reference's own drivers with its GDN patch
    (oracle.model_path.tree_gdn_layers(reference_truncated=True) around
    dense_leaf_logits / sequential_param_grads): dfs_tree_forward leaf logits
    and tree_grad_ckpt_sequential parameter gradients, < 1e-5. The
    model's keys are nearly parallel and its decay slow
    (gdn_layer_util.strong_recurrence), so the truncation is visible: the
    default (exact-rule) engine run must differ from that oracle by > 1e-4."""
    from oracle.model_path import dense_leaf_logits, sequential_param_grads, tree_gdn_layers
    from tests.gdn_layer_util import strong_recurrence
    from tree_training_amd.ckpt import make_tree_loss_fn, tree_grad_ckpt_sequential
    from tree_training_amd.dfs_tree_forward import dfs_tree_forward
    roots, nodes, leaves, labels = _c1_forest()
    base = strong_recurrence(small_hybrid_model(3))
    ref = copy.deepcopy(base).double()
    model = base.to(DEV)
    print("hybrid model reference_literal vs truncated oracle", flush=True)
    with tree_gdn_layers(ref, roots, reference_truncated=True):
        with torch.no_grad():
            ref_logits, _ = dense_leaf_logits(ref, roots)
        ref_grads = sequential_param_grads(ref, roots, labels, len(leaves))
    with torch.no_grad():
        lit = dfs_tree_forward(model, roots, reference_literal=True)
        exact = dfs_tree_forward(model, roots)
    r_lit = max(max_rel(a[0].numpy(), b[0].double().cpu().numpy()) for a, b in zip(ref_logits, lit.leaf_logits))
    r_exact = max(max_rel(a[0].numpy(), b[0].double().cpu().numpy()) for a, b in zip(ref_logits, exact.leaf_logits))
    print(f"  leaf logits: literal {r_lit:.3e}, exact rule {r_exact:.3e}", flush=True)
    assert r_lit < 1e-5 and r_exact > 1e-4
    model.zero_grad(set_to_none=True)
    fn = make_tree_loss_fn([labels[id(n)] for n in leaves], leaves, len(leaves))
    tree_grad_ckpt_sequential(model, roots, fn, reference_literal=True)
    torch.cuda.synchronize()
    _compare_grads(model, ref_grads)
