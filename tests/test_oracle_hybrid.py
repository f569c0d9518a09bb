"""The oracle's restatement of the reference's hybrid run (partitions, gateway
KV, gateway-gradient chaining; oracle.model_path.hybrid_param_grads), pinned
on the CPU in float64 against the independent whole-tree oracle:
  * with the inherited gateway bias every partition sees exactly the
    whole-tree mask rows, so the hybrid gradients equal the sequential
    whole-tree run's (to float64 rounding) for every partitioning;
  * with the reference's literal bias (tree_grad_hybrid.py:207) they still do
    when no gateway is nested in another (the c1 tree), and differ on the
    two-level chain of tests/golden/q1_chain.json (the Q1 divergence).
A mistake in the gateway slices, the bias, the depth offsets, the per-leaf
schedule or the chaining breaks the first property. "Equal" is < 1e-6: the
transformers eager attention takes its softmax in float32 even in a float64
model (HF/models/qwen3/modeling_qwen3.py:202), and a gateway row (past keys
then own keys, non-ancestors masked) reduces in another order than the
whole-tree row (measured 2e-7); the Q1 divergence is > 1e-3."""
import copy

import pytest
import torch

from oracle.attention import max_rel
from oracle.model_path import hybrid_param_grads, sequential_param_grads
from tests.conftest import forest_from_spec, load_golden, make_qwen3


def _setup(tree):
    spec = load_golden({"c1": "c1_tree.json", "q1": "q1_chain.json"}[tree])
    roots, nodes = forest_from_spec(spec["nodes"])
    leaves = [n for n in nodes if not n.children]
    g = torch.Generator().manual_seed(99)
    labels = {id(n): torch.randint(1, 1000, (len(n.token_ids),), generator=g) for n in leaves}
    model = copy.deepcopy(make_qwen3("tiny", layers=2)).double()
    return model, roots, labels, len(leaves)


def _rel(a, b):
    assert set(a) == set(b)
    return max(max_rel(a[k].numpy(), b[k].numpy()) for k in a)


@pytest.mark.parametrize("tree,max_tokens", [("c1", 1000), ("c1", 20), ("c1", 10), ("q1", 6)])
def test_hybrid_oracle_inherited_bias_equals_whole_tree(tree, max_tokens):
    model, roots, labels, n = _setup(tree)
    whole = sequential_param_grads(model, roots, labels, n)
    hyb = hybrid_param_grads(model, roots, labels, n, max_tokens, legacy=False)
    assert _rel(whole, hyb) < 1e-6


@pytest.mark.parametrize("tree,max_tokens,equal", [("c1", 20, True), ("c1", 10, True), ("q1", 6, False)])
def test_hybrid_oracle_literal_bias(tree, max_tokens, equal):
    model, roots, labels, n = _setup(tree)
    whole = sequential_param_grads(model, roots, labels, n)
    lit = hybrid_param_grads(model, roots, labels, n, max_tokens, legacy=True)
    r = _rel(whole, lit)
    assert (r < 1e-6) if equal else (r > 1e-3), r
