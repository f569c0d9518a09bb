"""Host-side logic of the drop-in API (no GPU): DFS flattening, partitioning,
gateway metadata, GatewayCache semantics, transformers integration seams."""
import math
import random

import numpy as np
import pytest
import torch

from oracle.partition import hybrid_schedule, partition_tree_literal
from oracle.tree_meta import build_dfs_tree_info_literal
from tests.conftest import Node, forest_from_spec, make_qwen3
from tests.test_oracle_meta import random_forest
from tree_training_amd import hybrid as H
from tree_training_amd.gateway import GatewayCache
from tree_training_amd.tree import TreeNode, build_dfs_tree_info


def test_tree_node_api():
    r = TreeNode([1, 2, 3])
    c = r.add_child([4])
    assert c in r.children and not r.is_leaf and c.is_leaf
    assert TreeNode([5]).children == []


def test_host_fields_match_literal(c1_spec):
    for seed in range(30):
        rng = random.Random(seed)
        roots = random_forest(rng, n_roots=rng.randint(1, 3)) if seed else forest_from_spec(c1_spec["nodes"])[0]
        lit = build_dfs_tree_info_literal(roots)
        info = build_dfs_tree_info(roots)
        assert info.dfs_token_ids == lit["dfs_token_ids"]
        assert info.chunk_boundaries == lit["chunk_boundaries"]
        assert info.chunk_parent_map == lit["chunk_parent_map"]
        assert info.leaf_chunk_ids == lit["leaf_chunk_ids"]
        assert [id(n) for n in info.leaf_nodes] == [id(n) for n in lit["leaf_nodes"]]
        assert (info.N, info.n_chunks) == (lit["N"], lit["n_chunks"])
        # node depth offsets equal the first position of each chunk
        assert info.node_off == [lit["dfs_pos_ids"][s] for s, _ in lit["chunk_boundaries"]]


def test_deep_chain_is_iterative():
    root = TreeNode([1])
    n = root
    for _ in range(5000):
        n = n.add_child([2])
    info = build_dfs_tree_info([root])
    assert info.N == 5001 and info.leaf_chunk_ids == [5000]
    parts = H.partition_tree([root], 100)
    assert [p.token_count for p in parts] == [100] * 50 + [1]


def test_empty_node_rejected():
    r = TreeNode([1])
    r.add_child([])
    with pytest.raises(ValueError):
        build_dfs_tree_info([r])


def _is_preorder_brute(parent):
    """The indices are a DFS pre-order iff a DFS that visits children in
    increasing index order visits 0, 1, 2, ... in turn."""
    n = len(parent)
    if any(not (-1 <= p < i) for i, p in enumerate(parent)):
        return False
    kids = [[] for _ in range(n)]
    for i, p in enumerate(parent):
        if p >= 0:
            kids[p].append(i)
    order = []
    for r in [i for i, p in enumerate(parent) if p < 0]:
        stack = [r]
        while stack:
            x = stack.pop()
            order.append(x)
            stack.extend(reversed(kids[x]))
    return order == list(range(n))


def test_preorder_check():
    from tree_training_amd.tree import preorder_violation
    # parent < i holds, but node 3's parent (1) has closed: node 2 (its sibling) came between
    assert preorder_violation([-1, 0, 0, 1]) == 3
    assert preorder_violation([-1, 0, 1, 1, 0, -1, 5]) is None
    assert preorder_violation([-1, 1]) == 1 and preorder_violation([-1, -2]) == 1
    rng = random.Random(0)
    for _ in range(3000):
        n = rng.randint(1, 9)
        parent = [rng.randint(-1, i - 1) for i in range(n)]
        assert (preorder_violation(parent) is None) == _is_preorder_brute(parent), parent
    for seed in range(20):   # every flattened forest is pre-order
        roots = random_forest(random.Random(seed), n_roots=3)
        assert preorder_violation(build_dfs_tree_info(roots).chunk_parent_map) is None


def test_no_gpu_fails_loudly():
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    from tree_training_amd._lib import TreeAttnError
    info = build_dfs_tree_info([TreeNode([1, 2])])
    with pytest.raises(TreeAttnError):
        info.dfs_pos_ids


def test_partition_tree_matches_oracle(c1_spec):
    for mt, want in c1_spec["partitions"].items():
        roots, _ = forest_from_spec(c1_spec["nodes"], TreeNode)
        parts = H.partition_tree(roots, int(mt))
        assert [p.token_count for p in parts] == want["sizes"]
    rng = random.Random(5)
    for trial in range(80):
        roots = random_forest(rng, n_roots=rng.randint(1, 3), max_depth=6, max_len=7)
        budget = rng.randint(1, 30)
        a = H.partition_tree(roots, budget)
        b = partition_tree_literal(roots, budget)
        assert len(a) == len(b)
        for pa, pb in zip(a, b):
            assert [id(n) for n in pa.dfs_nodes] == [id(n) for n in pb.dfs_nodes]
            assert pa.cut_node_set == pb.cut_node_set
            assert pa.leaf_node_set == pb.leaf_node_set
            assert pa.token_count == pb.token_count
            assert (pa.parent is None) == (pb.parent is None)
            assert id(pa.parent_cut_node) == id(pb.parent_cut_node)


@pytest.mark.parametrize("legacy", [True, False])
def test_hybrid_plan_gateways_match_oracle(legacy, c1_spec, q1_spec):
    cases = [(forest_from_spec(c1_spec["nodes"], TreeNode)[0], mt) for mt in (1000, 20, 10)]
    cases.append((forest_from_spec(q1_spec["nodes"], TreeNode)[0], q1_spec["max_tokens"]))
    rng = random.Random(9)
    for _ in range(40):
        cases.append((random_forest(rng, n_roots=rng.randint(1, 2), max_depth=6, max_len=6), rng.randint(2, 16)))
    for roots, mt in cases:
        ours = H.hybrid_plan(roots, mt, legacy=legacy, pack_siblings=False)
        ref = hybrid_schedule(roots, mt, legacy=legacy)
        assert len(ours) == len(ref)
        for o, r in zip(ours, ref):
            assert o["pos_offset"] == r["pos_offset"]
            assert o["n_tokens"] == r["info"]["N"]
            if r["gateway"] is None:
                assert o["past_len"] == 0
                continue
            assert o["past_len"] == r["gateway"]["total"]
            assert [math.isfinite(x) for x in o["bias"].tolist()] == [math.isfinite(x) for x in r["gateway"]["bias"]]


def test_gateway_cache_reference_mode():
    gk = torch.randn(1, 2, 3, 4, requires_grad=True)
    gv = torch.randn(1, 2, 3, 4, requires_grad=True)
    c = GatewayCache([(gk, gv), (None, None)])
    k, v = torch.randn(1, 2, 5, 4), torch.randn(1, 2, 5, 4)
    fk, fv = c.update(k, v, 0)
    assert fk.shape == (1, 2, 8, 4) and torch.equal(fk[:, :, :3], gk.detach()) and torch.equal(fv[:, :, 3:], v)
    fk1, _ = c.update(k, v, 1)
    assert fk1 is k
    assert c.get_seq_length(0) == 3 and c.get_seq_length(1) == 0 and c.get_seq_length(7) == 0
    assert c.get_mask_sizes(torch.arange(5), 0) == (8, 0)
    assert c.get_mask_sizes(5, 0) == (8, 0)
    assert set(c._full_kv) == {0, 1}


def test_gateway_cache_segmented_mode():
    gk = torch.randn(1, 2, 3, 4)
    gv = torch.randn(1, 2, 3, 4)
    c = GatewayCache([(gk, gv)], segmented=True)
    k, v = torch.randn(1, 2, 5, 4), torch.randn(1, 2, 5, 4)
    rk, rv = c.update(k, v, 0)
    assert rk is k and rv is v                      # no concatenation on the hot path
    assert c.gate(0)[0] is gk
    fk, fv = c._full_kv[0]                          # still available on demand
    assert torch.equal(fk, torch.cat([gk, k], -2)) and 0 in c._full_kv


def test_transformers_passes_tree_ctx_to_attention():
    """The seam the engine relies on: a registered attention function gets the
    model kwargs and no dense mask is built for an unregistered-mask name."""
    from transformers import AttentionInterface
    seen = {}

    def fake_attention(module, q, k, v, mask, scaling=None, dropout=0.0, **kw):
        seen.setdefault("ctx", kw.get("tree_ctx"))
        seen.setdefault("mask", mask)
        seen["layers"] = seen.get("layers", 0) + 1
        out = torch.zeros(q.shape[0], q.shape[2], q.shape[1], q.shape[3], dtype=q.dtype)
        return out, None

    AttentionInterface.register("tree_probe", fake_attention)
    m = make_qwen3("tiny", layers=2)
    m.config._attn_implementation = "tree_probe"
    marker = object()
    m(input_ids=torch.tensor([[1, 2, 3]]), position_ids=torch.tensor([[0, 1, 1]]), tree_ctx=marker)
    assert seen["ctx"] is marker and seen["mask"] is None and seen["layers"] == 2


def test_run_tree_model_rejects_token_ids_outside_the_vocabulary():
    """The device embedding lookup does not check its indices; the driver
    refuses out-of-range ids on the host before any launch."""
    import types
    from tree_training_amd.dfs_tree_forward import run_tree_model
    from tree_training_amd.tree import TreeNode, build_dfs_tree_info
    info = build_dfs_tree_info([TreeNode([1, 2, 1000])])
    model = types.SimpleNamespace(config=types.SimpleNamespace(vocab_size=1000))
    with pytest.raises(ValueError, match="vocabulary"):
        run_tree_model(model, info, "cpu")


def test_reference_literal_sets_every_reference_option():
    """literal_options: reference_literal=True forces the options each driver
    takes to the reference's arithmetic and leaves them alone otherwise; the
    drivers take the switch (a missing name in any of them fails here on CPU)."""
    import inspect
    from tree_training_amd.ckpt import tree_grad_ckpt_sequential
    from tree_training_amd.dfs_tree_forward import dfs_tree_forward, literal_options
    from tree_training_amd.hybrid import tree_grad_hybrid
    opts = dict(legacy_gateway_bias=False, gdn_reference_truncated=False, gdn_per_node_projections=False,
                fused_prologue=True, fused_leaf_ce=True)
    assert literal_options(False, **opts) == opts
    assert literal_options(True, **opts) == dict(legacy_gateway_bias=True, gdn_reference_truncated=True,
                                                 gdn_per_node_projections=True, fused_prologue=False,
                                                 fused_leaf_ce=False)
    assert literal_options(True, fused_prologue=True) == dict(fused_prologue=False)
    assert literal_options(True, pack_siblings=True) == dict(pack_siblings=False)
    for fn, names in ((dfs_tree_forward, ("gdn_reference_truncated", "gdn_per_node_projections", "fused_prologue")),
                      (tree_grad_ckpt_sequential, ("fused_leaf_ce", "gdn_reference_truncated",
                                                   "gdn_per_node_projections", "fused_prologue")),
                      (tree_grad_hybrid, ("legacy_gateway_bias", "fused_leaf_ce", "fused_prologue",
                                          "pack_siblings"))):
        params = inspect.signature(fn).parameters
        assert "reference_literal" in params and params["reference_literal"].default is False
        for n in names:
            assert n in params, (fn.__name__, n)
    for mod in ("ckpt", "hybrid", "dfs_tree_forward"):     # every module-level name the drivers use resolves
        m = __import__(f"tree_training_amd.{mod}", fromlist=["x"])
        assert m.literal_options is literal_options


def test_packed_partitions_see_exactly_the_whole_tree(c1_spec):
    """pack_sibling_partitions merges only partitions of one cut node of one
    parent, within max_tokens, keeps every node in exactly one partition and
    parents before children; and with the inherited gateway bias every query
    of every packed partition sees (gateway keys with bias 0, plus its own
    partition's tree mask) exactly its ancestors-or-self in the whole forest,
    token by token — so packed and unpacked runs compute the same attention."""
    from oracle.tree_meta import mask_from_horizon, meta_closed_form
    cases = [(forest_from_spec(c1_spec["nodes"], TreeNode)[0], mt) for mt in (1000, 20, 10, 6)]
    rng = random.Random(11)
    for _ in range(30):
        cases.append((random_forest(rng, n_roots=rng.randint(1, 2), max_depth=5, max_len=6), rng.randint(3, 20)))
    merged_any = False
    for roots, mt in cases:
        parent_of, order = {}, []
        stack = list(reversed(roots))
        while stack:
            n = stack.pop()
            order.append(n)
            for c in reversed(n.children):
                parent_of[id(c)] = n
                stack.append(c)
        raw = H.partition_tree(roots, mt)
        parts = H.pack_sibling_partitions(H.partition_tree(roots, mt), mt)
        merged_any |= len(parts) < len(raw)
        assert sorted(id(n) for p in parts for n in p.dfs_nodes) == sorted(id(n) for n in order)
        pos = {id(p): i for i, p in enumerate(parts)}
        for i, p in enumerate(parts):
            if p.parent is not None:
                assert pos[id(p.parent)] < i
            if len(p.entry_nodes) > 1:
                assert p.token_count <= mt
                assert all(parent_of[id(e)] is p.parent_cut_node for e in p.entry_nodes)
        plans = H.hybrid_plan(roots, mt)
        assert len(plans) == len(parts)

        def ancestors_or_self(n):
            out = set()
            while n is not None:
                out.add(id(n))
                n = parent_of.get(id(n))
            return out

        gw_tokens = {}
        for p, pl in zip(parts, plans):
            node_len, par, nodes = H._flatten_partition(p)
            own = [(id(n), j) for n in nodes for j in range(len(n.token_ids))]
            gtok = gw_tokens.get(id(p), [])
            assert len(gtok) == pl["past_len"]
            vis_g = [t for t, b in zip(gtok, pl["bias"].tolist() if gtok else []) if b == 0.0]
            mask = mask_from_horizon(meta_closed_form(node_len, par)["horizon"])
            for qi, (nid, j) in enumerate(own):
                node = next(n for n in nodes if id(n) == nid)
                anc = ancestors_or_self(node)
                want = {(m, k) for m in anc for k in range(len(next(x for x in order if id(x) == m).token_ids))
                        if m != nid or k <= j}
                got = set(vis_g) | {own[kj] for kj in np.nonzero(mask[qi])[0]}
                assert got == want, (mt, qi)
            _, _, end, _, _, _ = H._dfs_info_for_partition(p)
            for child in parts:
                if child.parent is p:
                    gw_tokens[id(child)] = gtok + own[:end[id(child.parent_cut_node)]]
    assert merged_any
