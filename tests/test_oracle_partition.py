"""Pins the partition / gateway oracle against hand traces and invariants."""
import math
import random

from oracle.partition import hybrid_schedule, partition_tree_literal
from tests.conftest import forest_from_spec
from tests.test_oracle_meta import random_forest


def _names(part, objs_by_id):
    return [objs_by_id[id(n)].name for n in part.dfs_nodes]


def test_c1_partitions(c1_spec):
    for mt, want in c1_spec["partitions"].items():
        roots, objs = forest_from_spec(c1_spec["nodes"])
        parts = partition_tree_literal(roots, int(mt))
        assert [p.token_count for p in parts] == want["sizes"]
        assert [[n.name for n in p.dfs_nodes] for p in parts] == want["members"]


def test_c1_gateways(c1_spec):
    by_mt = {}
    for g in c1_spec["gateways"]:
        by_mt.setdefault(g["max_tokens"], []).append(g)
    for mt, gws in by_mt.items():
        roots, objs = forest_from_spec(c1_spec["nodes"])
        sched = hybrid_schedule(roots, mt, legacy=True)
        got = {}
        for ent in sched:
            gw = ent["gateway"]
            if gw is not None:
                got[gw["cut"].name] = gw
        for want in gws:
            gw = got[want["cut"]]
            assert gw["total"] == want["total"]
            assert gw["pos_off"] == want["pos_off"]
            assert [int(math.isfinite(b)) for b in gw["bias"]] == want["bias_visible"]
            # every partition fed by this cut got the same gateway object
            fed = [ent["partition"].entry_nodes[0].name for ent in sched
                   if ent["gateway"] is gw]
            assert fed == want["to"]


def test_q1_chain_legacy_vs_inherited(q1_spec):
    for legacy, key in ((True, "legacy_visible"), (False, "inherited_visible")):
        roots, objs = forest_from_spec(q1_spec["nodes"])
        sched = hybrid_schedule(roots, q1_spec["max_tokens"], legacy=legacy)
        assert [e["partition"].token_count for e in sched] == q1_spec["partitions"]["sizes"]
        gws = [e["gateway"] for e in sched if e["gateway"] is not None]
        for gw, want in zip(gws, q1_spec["gateways"]):
            assert gw["cut"].name == want["cut"]
            assert gw["total"] == want["total"]
            assert gw["pos_off"] == want["pos_off"]
            assert [int(math.isfinite(b)) for b in gw["bias"]] == want[key]
        # visible-key counts of E's tokens: gateway-visible + causal in-node
        last = sched[-1]
        vis = sum(int(math.isfinite(b)) for b in last["gateway"]["bias"])
        counts = [vis + j + 1 for j in range(3)]
        assert counts == q1_spec["E_visible_counts"]["legacy" if legacy else "inherited"]


def test_partition_invariants_random():
    rng = random.Random(3)
    for trial in range(60):
        roots = random_forest(rng, n_roots=rng.randint(1, 3), max_depth=5, max_len=6)
        budget = rng.randint(1, 25)
        parts = partition_tree_literal(roots, budget)
        seen = set()
        order = {id(p): i for i, p in enumerate(parts)}
        for p in parts:
            for n in p.dfs_nodes:
                assert id(n) not in seen
                seen.add(id(n))
            assert p.token_count <= max(budget, max(len(n.token_ids) for n in p.dfs_nodes))
            if p.parent is not None:
                assert order[id(p.parent)] < order[id(p)]
                assert id(p.parent_cut_node) in p.parent.cut_node_set

        def all_nodes(r):
            yield r
            for c in r.children:
                yield from all_nodes(c)
        assert seen == {id(n) for r in roots for n in all_nodes(r)}


def test_inherited_bias_gives_whole_tree_visibility():
    """With the inherited bias, every query of every partition sees exactly
    pos+1 keys (gateway + in-partition), i.e. the whole-tree mask row."""
    from oracle.tree_meta import flatten_forest, meta_closed_form, mask_from_horizon
    rng = random.Random(11)
    for trial in range(30):
        roots = random_forest(rng, n_roots=rng.randint(1, 2), max_depth=5, max_len=5)
        budget = rng.randint(2, 14)
        sched = hybrid_schedule(roots, budget, legacy=False)
        for ent in sched:
            info = ent["info"]
            own = info["attn_mask_bool"].sum(1)
            vis = 0 if ent["gateway"] is None else sum(
                int(math.isfinite(b)) for b in ent["gateway"]["bias"])
            pos = [p + ent["pos_offset"] for p in info["dfs_pos_ids"]]
            assert [int(vis + o) for o in own] == [p + 1 for p in pos]
