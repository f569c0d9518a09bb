"""Pins the metadata oracle: hand-traced fixture, brute force, closed form."""
import random

import numpy as np

from oracle.tree_meta import (brute_force_mask, build_dfs_tree_info_literal,
                              flatten_forest, mask_from_horizon, meta_closed_form)
from tests.conftest import Node, forest_from_spec


def random_forest(rng, n_roots=2, max_depth=4, max_branch=3, max_len=5):
    roots = []

    def grow(node, depth):
        if depth >= max_depth:
            return
        for _ in range(rng.randint(0, max_branch)):
            ch = node.add_child([0] * rng.randint(1, max_len))
            grow(ch, depth + 1)

    for _ in range(n_roots):
        r = Node([0] * rng.randint(1, max_len))
        grow(r, 1)
        roots.append(r)
    return roots


def test_literal_matches_hand_trace(c1_spec):
    roots, _ = forest_from_spec(c1_spec["nodes"])
    info = build_dfs_tree_info_literal(roots)
    assert info["N"] == c1_spec["N"]
    assert info["n_chunks"] == c1_spec["n_chunks"]
    assert [list(b) for b in info["chunk_boundaries"]] == c1_spec["chunk_boundaries"]
    assert info["chunk_parent_map"] == c1_spec["chunk_parent_map"]
    assert info["leaf_chunk_ids"] == c1_spec["leaf_chunk_ids"]
    assert info["dfs_pos_ids"] == c1_spec["dfs_pos_ids"]
    mask = info["attn_mask_bool"]
    assert int(mask.sum()) == c1_spec["nnz"]
    for i, cnt in c1_spec["visible_count_spot_checks"].items():
        assert int(mask[int(i)].sum()) == cnt
    # spot checks of the hand trace: q (token 20) does not see e (tokens 14..18)
    assert not mask[20, 14:19].any() and mask[20, 10:14].all()
    # g (token 26) sees f and c_left, not d_left/e/q
    assert not mask[26, 10:22].any() and mask[26, 22:26].all() and mask[26, 7:10].all()


def test_closed_form_matches_hand_trace(c1_spec):
    lens = [n["len"] for n in c1_spec["nodes"]]
    par = [n["parent"] for n in c1_spec["nodes"]]
    m = meta_closed_form(lens, par)
    assert m["pos"].tolist() == c1_spec["dfs_pos_ids"]
    assert m["node_hend"].tolist() == c1_spec["chunk_horizon"]
    assert int((m["pos"] + 1).sum()) == c1_spec["nnz"]
    roots, _ = forest_from_spec(c1_spec["nodes"])
    lit = build_dfs_tree_info_literal(roots)
    assert np.array_equal(mask_from_horizon(m["horizon"]), lit["attn_mask_bool"])


def test_random_forests_three_ways():
    rng = random.Random(7)
    for trial in range(40):
        roots = random_forest(rng, n_roots=rng.randint(1, 3))
        lens, par, _ = flatten_forest(roots)
        lit = build_dfs_tree_info_literal(roots)
        m = meta_closed_form(lens, par)
        bf = brute_force_mask(lens, par)
        assert np.array_equal(lit["attn_mask_bool"], bf)
        assert np.array_equal(mask_from_horizon(m["horizon"]), bf)
        assert m["pos"].tolist() == lit["dfs_pos_ids"]
        # every query sees exactly pos+1 keys, and the mask is lower-triangular
        assert np.array_equal(bf.sum(1), m["pos"] + 1)
        assert not np.triu(bf, 1).any()


def test_pos_offset_shifts_positions_only(c1_spec):
    lens = [n["len"] for n in c1_spec["nodes"]]
    par = [n["parent"] for n in c1_spec["nodes"]]
    a = meta_closed_form(lens, par)
    b = meta_closed_form(lens, par, pos_offset=37)
    assert np.array_equal(b["pos"], a["pos"] + 37)
    assert np.array_equal(b["horizon"], a["horizon"])


def test_single_chain_is_causal():
    lens, par = [3, 5, 2], [-1, 0, 1]
    m = meta_closed_form(lens, par)
    T = sum(lens)
    assert np.array_equal(mask_from_horizon(m["horizon"]), np.tril(np.ones((T, T), bool)))
    assert m["pos"].tolist() == list(range(T))
