"""GPU parity of the tree gated-delta-rule scan (tt_gdn_tree_fwd) against the
float64 oracle (oracle/gdn.py, exact mode), through the C ABI.

Bars: float32 outputs and node states max_rel < 1e-5; bf16 outputs < 2e-2
(max |error| over max |reference|). At the 16K-tree size the oracle is too
slow, so the check there is per-path equivalence: every root-to-leaf path run
as a plain chain of the same nodes gives bitwise the same outputs.
"""
import numpy as np
import pytest
import torch

from oracle import gdn as ogdn
from tree_training_amd.gdn import GdnTree, gdn_tree_forward
from tree_training_amd.workloads import agent_tree, random_forest

pytestmark = pytest.mark.gpu
D = 128


def _inputs(T, Hk, Hv, seed, realistic_gates=False):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((T, Hk, D)).astype(np.float32)
    k = rng.standard_normal((T, Hk, D)).astype(np.float32)
    v = rng.standard_normal((T, Hv, D)).astype(np.float32)
    if realistic_gates:
        a, b = rng.standard_normal((T, Hv)), rng.standard_normal((T, Hv))
        g, beta = ogdn.gdn_gates(a, b, np.log(rng.uniform(1e-3, 16, Hv)), np.ones(Hv))
    else:
        g = -np.abs(rng.standard_normal((T, Hv))) * 0.2
        beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((T, Hv))))
    return q, k, v, g.astype(np.float32), beta.astype(np.float32)


def _run(q, k, v, g, beta, lens, par, dtype):
    dev = torch.device("cuda", 0)
    t = lambda x: torch.from_numpy(x).to(dev)
    tree = GdnTree(lens, par, dev)
    o, st = gdn_tree_forward(t(q).to(dtype), t(k).to(dtype), t(v).to(dtype), t(g), t(beta), tree)
    torch.cuda.synchronize()
    return o.float().cpu().numpy(), st.cpu().numpy()


def _rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


CASES = {
    "forest_small_nodes": dict(topo=lambda: random_forest(3, node_len=(1, 12)), Hk=2, Hv=4),
    "forest_multi_chunk": dict(topo=lambda: random_forest(8, node_len=(20, 90)), Hk=2, Hv=2),
    "chain_ragged": dict(topo=lambda: ([33, 64, 95, 1], [-1, 0, 1, 2]), Hk=1, Hv=2),
    "single_tokens": dict(topo=lambda: ([1] * 9, [-1, 0, 1, 1, 3, -1, 5, 5, 0]), Hk=1, Hv=1),
    "c1_heads": dict(topo=lambda: ([3, 4, 3, 4, 5, 3, 3, 4, 4, 3, 4, 3, 4],
                                   [-1, 0, 1, 2, 3, 3, 2, 6, -1, 8, 9, 8, 11]), Hk=16, Hv=32),
}


@pytest.mark.parametrize("case", list(CASES))
def test_gdn_fp32_matches_oracle(case):
    c = CASES[case]
    lens, par = c["topo"]()
    T = sum(lens)
    q, k, v, g, beta = _inputs(T, c["Hk"], c["Hv"], sum(map(ord, case)))
    o, st = _run(q, k, v, g, beta, lens, par, torch.float32)
    o_ref, st_ref = ogdn.gdn_tree(q, k, v, g, beta, lens, par, mode="exact")
    assert _rel(o, o_ref) < 1e-5, case
    assert _rel(st, st_ref) < 1e-5, case


@pytest.mark.parametrize("case", ["forest_multi_chunk", "c1_heads"])
def test_gdn_bf16_matches_oracle(case):
    c = CASES[case]
    lens, par = c["topo"]()
    T = sum(lens)
    q, k, v, g, beta = _inputs(T, c["Hk"], c["Hv"], 7 + sum(map(ord, case)), realistic_gates=True)
    rb = lambda x: torch.from_numpy(x).bfloat16().float().numpy()
    q, k, v = rb(q), rb(k), rb(v)                 # the oracle sees the same bf16 inputs
    o, _ = _run(q, k, v, g, beta, lens, par, torch.bfloat16)
    o_ref, _ = ogdn.gdn_tree(q, k, v, g, beta, lens, par, mode="exact")
    assert _rel(o, o_ref) < 2e-2, case


def test_gdn_16k_tree_per_path_equivalence():
    """Full-size (agent tree, 16,318 tokens, 16 q/k heads, 32 v heads, bf16):
    the outputs on each sampled root-to-leaf path equal a run of that path
    alone as a chain of the same nodes, bit for bit."""
    lens, par = agent_tree(0)
    T = sum(lens)
    q, k, v, g, beta = _inputs(T, 16, 32, 5, realistic_gates=True)
    o, st = _run(q, k, v, g, beta, lens, par, torch.bfloat16)
    assert np.isfinite(o).all() and np.isfinite(st).all()
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]])
    leaves = [i for i in range(len(lens)) if i not in set(par)]
    for leaf in (leaves[0], leaves[len(leaves) // 2], leaves[-1]):
        path, j = [], leaf
        while j >= 0:
            path.append(j)
            j = par[j]
        path = path[::-1]
        idx = np.concatenate([np.arange(starts[i], starts[i] + lens[i]) for i in path])
        plens = [lens[i] for i in path]
        ppar = list(range(-1, len(path) - 1))
        o_p, st_p = _run(q[idx], k[idx], v[idx], g[idx], beta[idx], plens, ppar, torch.bfloat16)
        assert np.array_equal(o_p, o[idx])
        assert np.array_equal(st_p[-1], st[leaf])
