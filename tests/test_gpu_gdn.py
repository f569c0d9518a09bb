"""GPU parity of the tree gated-delta-rule scan (tt_gdn_tree_fwd,
tt_gdn_tree_bwd) against the float64 oracle (oracle/gdn.py: exact mode for the
forward, autograd through the token recurrence for the backward), through the
C ABI.

Bars: float32 outputs, node states and gradients (each of dq, dk, dv, dg,
dbeta) max_rel < 1e-5; bf16 outputs and gradients < 2e-2 (max |error| over
max |reference|). At the 16K-tree size the oracle is too slow, so the checks
there are per-path: every root-to-leaf path run as a plain chain of the same
nodes gives bitwise the same outputs, and with d_o supported on one path the
gradients equal that chain's, bitwise, and vanish off the path.
"""
import numpy as np
import pytest
import torch

from oracle import gdn as ogdn
from tree_training_amd.gdn import GdnTree, gdn_tree_backward, gdn_tree_forward
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
    # a level of 20 nodes x 32 v heads under a 40-token root
    "wide_level": dict(topo=lambda: ([40] + [7 + 3 * i for i in range(20)], [-1] + [0] * 20), Hk=16, Hv=32),
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


@pytest.mark.parametrize("seed", range(8))
def test_gdn_random_forests_match_oracle(seed):
    """Seeded random forests (1-3 roots, node lengths up to a drawn maximum of
    at most 150 tokens, at most 900 tokens), 1-4 q/k heads with one or two v
    heads each, simple or realistic gates, exact or reference semantics:
    float32 outputs and node states against the float64 oracle, < 1e-5."""
    rng = np.random.default_rng(2000 + seed)
    while True:
        lens, par = random_forest(int(rng.integers(0, 10**6)), n_roots=(1, int(rng.integers(1, 4))),
                                  max_depth=int(rng.integers(1, 6)), max_branch=int(rng.integers(1, 4)),
                                  node_len=(1, int(rng.integers(2, 150))))
        if sum(lens) <= 900:
            break
    T = sum(lens)
    Hk = int(rng.choice([1, 2, 4]))
    Hv = Hk * int(rng.choice([1, 2]))
    mode = "reference" if rng.random() < 0.4 else "exact"
    real = bool(rng.random() < 0.5)
    print(f"gdn random forest seed={seed}: T={T} nodes={len(lens)} Hk={Hk} Hv={Hv} {mode} realistic={real}",
          flush=True)
    q, k, v, g, beta = _inputs(T, Hk, Hv, 3000 + seed, realistic_gates=real)
    dev = torch.device("cuda", 0)
    t = lambda x: torch.from_numpy(x).to(dev)
    o, st = gdn_tree_forward(t(q), t(k), t(v), t(g), t(beta), GdnTree(lens, par, dev),
                             reference_truncated=mode == "reference")
    torch.cuda.synchronize()
    o_ref, st_ref = ogdn.gdn_tree(q, k, v, g, beta, lens, par, mode=mode)
    assert _rel(o.cpu().numpy(), o_ref) < 1e-5
    assert _rel(st.cpu().numpy(), st_ref) < 1e-5


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


def test_gdn_agent16k_two_heads_matches_oracle():
    """Full c5 topology (the agent tree: 16,318 tokens, 54 nodes of 64-512
    tokens, root-to-leaf paths of up to 76 chunks), realistic gates, fp32, one
    q/k head shared by two v heads, against the float64 exact-rule oracle
    (oracle.gdn.gdn_tree mode="exact": the token recurrence continued from the
    parent's final state). Outputs and node states: < 1e-5. Head 0's gates
    decay hard (the cumulative decay reaches -570 within one 32-token chunk),
    where a one-float prefix sum would put ~3e-5 relative error on the late
    tokens' decays and so on the states; the kernels carry it in two floats."""
    lens, par = agent_tree(0)
    T = sum(lens)
    q, k, v, g, beta = _inputs(T, 1, 2, 17, realistic_gates=True)
    print(f"gdn exact fwd 16k: T={T} nodes={len(lens)}", flush=True)
    o, st = _run(q, k, v, g, beta, lens, par, torch.float32)
    o_ref, st_ref = ogdn.gdn_tree(q, k, v, g, beta, lens, par, mode="exact")
    print(f"  o {_rel(o, o_ref):.2e}  states {_rel(st, st_ref):.2e}", flush=True)
    assert _rel(o, o_ref) < 1e-5, _rel(o, o_ref)
    assert _rel(st, st_ref) < 1e-5, _rel(st, st_ref)


def _run_bwd(q, k, v, g, beta, d_o, lens, par, dtype):
    dev = torch.device("cuda", 0)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    tree = GdnTree(lens, par, dev)
    outs = gdn_tree_backward(t(q).to(dtype), t(k).to(dtype), t(v).to(dtype), t(g), t(beta), t(d_o).to(dtype), tree)
    torch.cuda.synchronize()
    return [x.float().cpu().numpy() for x in outs]


def _oracle_grads(q, k, v, g, beta, d_o, lens, par):
    tt = [torch.from_numpy(np.asarray(x, np.float64)).requires_grad_(True) for x in (q, k, v, g, beta)]
    o = ogdn.gdn_tree_torch(*tt, lens, par)
    return [x.numpy() for x in torch.autograd.grad((o * torch.from_numpy(np.asarray(d_o, np.float64))).sum(), tt)]


BWD_NAMES = ("dq", "dk", "dv", "dg", "dbeta")


@pytest.mark.parametrize("case", list(CASES))
def test_gdn_bwd_fp32_matches_autograd_oracle(case):
    c = CASES[case]
    lens, par = c["topo"]()
    T = sum(lens)
    q, k, v, g, beta = _inputs(T, c["Hk"], c["Hv"], 3 + sum(map(ord, case)))
    d_o = np.random.default_rng(11).standard_normal((T, c["Hv"], D)).astype(np.float32)
    print(f"gdn bwd fp32 {case}: T={T} nodes={len(lens)}", flush=True)
    got = _run_bwd(q, k, v, g, beta, d_o, lens, par, torch.float32)
    ref = _oracle_grads(q, k, v, g, beta, d_o, lens, par)
    for name, a, b in zip(BWD_NAMES, got, ref):
        assert _rel(a, b) < 1e-5, (case, name, _rel(a, b))


@pytest.mark.parametrize("case", ["forest_multi_chunk", "c1_heads"])
def test_gdn_bwd_bf16_matches_autograd_oracle(case):
    c = CASES[case]
    lens, par = c["topo"]()
    T = sum(lens)
    q, k, v, g, beta = _inputs(T, c["Hk"], c["Hv"], 5 + sum(map(ord, case)), realistic_gates=True)
    rb = lambda x: torch.from_numpy(x).bfloat16().float().numpy()
    d_o = rb(np.random.default_rng(12).standard_normal((T, c["Hv"], D)).astype(np.float32))
    q, k, v = rb(q), rb(k), rb(v)
    print(f"gdn bwd bf16 {case}: T={T} nodes={len(lens)}", flush=True)
    got = _run_bwd(q, k, v, g, beta, d_o, lens, par, torch.bfloat16)
    ref = _oracle_grads(q, k, v, g, beta, d_o, lens, par)
    for name, a, b in zip(BWD_NAMES, got, ref):
        assert _rel(a, b) < 2e-2, (case, name, _rel(a, b))


def test_gdn_bwd_16k_tree_path_support():
    """Full size (agent tree, 16,318 tokens, 16/32 heads, bf16): with d_o
    non-zero only on one root-to-leaf path, the tree's gradients on that path
    equal the path run alone as a chain, bit for bit, and are exactly zero on
    every other token."""
    lens, par = agent_tree(0)
    T = sum(lens)
    q, k, v, g, beta = _inputs(T, 16, 32, 9, realistic_gates=True)
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]])
    leaves = [i for i in range(len(lens)) if i not in set(par)]
    leaf = leaves[len(leaves) // 2]
    path, j = [], leaf
    while j >= 0:
        path.append(j)
        j = par[j]
    path = path[::-1]
    idx = np.concatenate([np.arange(starts[i], starts[i] + lens[i]) for i in path])
    d_o = np.zeros((T, 32, D), np.float32)
    d_o[idx] = np.random.default_rng(4).standard_normal((len(idx), 32, D))
    print(f"gdn bwd 16k path support: leaf={leaf} path_tokens={len(idx)}", flush=True)
    full = _run_bwd(q, k, v, g, beta, d_o, lens, par, torch.bfloat16)
    chain = _run_bwd(q[idx], k[idx], v[idx], g[idx], beta[idx], d_o[idx], [lens[i] for i in path],
                     list(range(-1, len(path) - 1)), torch.bfloat16)
    off = np.setdiff1d(np.arange(T), idx)
    for name, a, b in zip(BWD_NAMES, full, chain):
        assert np.isfinite(a).all(), name
        assert np.array_equal(a[idx], b), name
        assert not np.any(a[off]), name


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("case", ["forest_multi_chunk", "c1_heads", "chain_ragged"])
def test_gdn_saved_forward_equals_recompute(case, dtype):
    """tt_gdn_tree_fwd_save + tt_gdn_tree_bwd_saved give bitwise the outputs,
    node states and gradients of tt_gdn_tree_fwd + the recomputing
    tt_gdn_tree_bwd (same kernels, same order of operations)."""
    from tree_training_amd import gdn as tgdn
    c = CASES[case]
    lens, par = c["topo"]()
    T = sum(lens)
    q, k, v, g, beta = _inputs(T, c["Hk"], c["Hv"], 21 + sum(map(ord, case)), realistic_gates=True)
    d_o = np.random.default_rng(13).standard_normal((T, c["Hv"], D)).astype(np.float32)
    dev = torch.device("cuda", 0)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    tree = GdnTree(lens, par, dev)
    args = (t(q).to(dtype), t(k).to(dtype), t(v).to(dtype), t(g), t(beta))
    print(f"gdn saved vs recompute {case} {dtype}: T={T}", flush=True)
    o0, st0 = gdn_tree_forward(*args, tree)
    o1, st1, saved = tgdn._gdn_forward(*args, tree, None, True, True)
    g0 = gdn_tree_backward(*args, t(d_o).to(dtype), tree)
    g1 = gdn_tree_backward(*args, t(d_o).to(dtype), tree, saved=saved)
    torch.cuda.synchronize()
    assert torch.equal(o0, o1) and torch.equal(st0, st1)
    for name, a, b in zip(BWD_NAMES, g0, g1):
        assert torch.equal(a, b), name


def test_gdn_autograd_keep_and_recompute_agree():
    """The autograd Function with and without kept forward states: bitwise
    the same gradients, and within the fp32 bar of the oracle."""
    from tree_training_amd import gdn as tgdn
    c = CASES["forest_multi_chunk"]
    lens, par = c["topo"]()
    T = sum(lens)
    q, k, v, g, beta = _inputs(T, c["Hk"], c["Hv"], 77)
    d_o = np.random.default_rng(14).standard_normal((T, c["Hv"], D)).astype(np.float32)
    dev = torch.device("cuda", 0)
    tree = GdnTree(lens, par, dev)
    grads = []
    for keep in (True, False):
        tgdn.KEEP_FORWARD_STATES = keep
        try:
            tt = [torch.from_numpy(x).to(dev).requires_grad_(True) for x in (q, k, v, g, beta)]
            o, _ = tgdn.gdn_tree(*tt, tree)
            grads.append(torch.autograd.grad((o * torch.from_numpy(d_o).to(dev)).sum(), tt))
        finally:
            tgdn.KEEP_FORWARD_STATES = True
    for name, a, b in zip(BWD_NAMES, *grads):
        assert torch.equal(a, b), name
    ref = _oracle_grads(q, k, v, g, beta, d_o, lens, par)
    for name, a, b in zip(BWD_NAMES, grads[0], ref):
        assert _rel(a.cpu().numpy(), b) < 1e-5, (name, _rel(a.cpu().numpy(), b))


def test_gdn_retain_graph_backwards_reuse_saved_forward(monkeypatch):
    """Under the reference's per-leaf schedule (several backward calls through
    one graph with retain_graph=True) every backward takes the kept forward
    terms (no recompute), and each gives the same gradients."""
    from tree_training_amd import gdn as tgdn
    c = CASES["forest_multi_chunk"]
    lens, par = c["topo"]()
    T = sum(lens)
    q, k, v, g, beta = _inputs(T, c["Hk"], c["Hv"], 78)
    d_o = np.random.default_rng(15).standard_normal((T, c["Hv"], D)).astype(np.float32)
    dev = torch.device("cuda", 0)
    tree = GdnTree(lens, par, dev)
    seen = []
    real = tgdn.gdn_tree_backward

    def spy(*a, **kw):
        seen.append(kw.get("saved") is not None)
        return real(*a, **kw)

    monkeypatch.setattr(tgdn, "gdn_tree_backward", spy)
    tt = [torch.from_numpy(x).to(dev).requires_grad_(True) for x in (q, k, v, g, beta)]
    o, _ = tgdn.gdn_tree(*tt, tree)
    loss = (o * torch.from_numpy(d_o).to(dev)).sum()
    grads = [torch.autograd.grad(loss, tt, retain_graph=True) for _ in range(3)]
    torch.cuda.synchronize()
    assert seen == [True, True, True]
    for gr in grads[1:]:
        for name, a, b in zip(BWD_NAMES, grads[0], gr):
            assert torch.equal(a, b), name


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("saved_fwd", [False, True], ids=["recompute", "saved"])
def test_gdn_packed_qkv_gradients(saved_fwd, dtype):
    """q, k, v as the column blocks of one packed [T, (2 Hk + Hv) 128] row
    buffer: dq, dk, dv come back as the same blocks of one new buffer
    (strided outputs through the C ABI), bitwise equal to the gradients of
    the same inputs held as separate contiguous tensors."""
    from tree_training_amd import gdn as tgdn
    c = CASES["c1_heads"]
    lens, par = c["topo"]()
    T, Hk, Hv = sum(lens), c["Hk"], c["Hv"]
    q, k, v, g, beta = _inputs(T, Hk, Hv, 91, realistic_gates=True)
    d_o = np.random.default_rng(16).standard_normal((T, Hv, D)).astype(np.float32)
    dev = torch.device("cuda", 0)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    tree = GdnTree(lens, par, dev)
    rows = t(np.concatenate([q.reshape(T, -1), k.reshape(T, -1), v.reshape(T, -1)], axis=1)).to(dtype)
    nk = Hk * D
    packed = (rows[:, :nk].view(T, Hk, D), rows[:, nk:2 * nk].view(T, Hk, D), rows[:, 2 * nk:].view(T, Hv, D))
    sep = tuple(x.contiguous() for x in packed)
    print(f"gdn packed qkv grads saved={saved_fwd} {dtype}: T={T}", flush=True)
    res = []
    for qkv in (packed, sep):
        saved = tgdn._gdn_forward(*qkv, t(g), t(beta), tree, None, True, True)[2] if saved_fwd else None
        res.append(gdn_tree_backward(*qkv, t(g), t(beta), t(d_o).to(dtype), tree, saved=saved))
    torch.cuda.synchronize()
    dq, dk, dv = res[0][:3]
    e = dq.element_size()
    assert dq.stride(0) == dk.stride(0) == dv.stride(0) == rows.shape[1]
    assert dk.data_ptr() == dq.data_ptr() + nk * e and dv.data_ptr() == dk.data_ptr() + nk * e
    assert res[1][0].is_contiguous()
    for name, a, b in zip(BWD_NAMES, *res):
        assert torch.equal(a, b), name


def test_gdn_conv_split_autograd_matches_torch_split():
    """tree_conv(split_sizes=...) feeding gdn_tree: the conv reads the q/k/v
    gradients in place (no concatenation) and gives bitwise the gradients of
    tree_conv + torch.split + gdn_tree."""
    from tree_training_amd import conv as tconv
    from tree_training_amd.gdn import gdn_tree
    c = CASES["c1_heads"]
    lens, par = c["topo"]()
    T, Hk, Hv = sum(lens), c["Hk"], c["Hv"]
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(5)
    C = (2 * Hk + Hv) * D
    bf = torch.bfloat16
    x0 = torch.randn(T, C, device=dev, generator=gen, dtype=bf)
    w0 = (torch.randn(C, 4, device=dev, generator=gen) * 0.5).to(bf)
    g0 = -torch.rand(T, Hv, device=dev, generator=gen) * 0.5
    b0 = torch.rand(T, Hv, device=dev, generator=gen)
    d_o = torch.randn(T, Hv, D, device=dev, generator=gen, dtype=bf)
    tree = GdnTree(lens, par, dev)
    sizes = (Hk * D, Hk * D, Hv * D)
    joined = []
    real_join = tconv._join_columns

    def spy(grads, sz, like):
        out = real_join(grads, sz, like)
        joined.append(out.data_ptr() == grads[0].data_ptr())
        return out

    print(f"conv split + gdn autograd: T={T} C={C}", flush=True)
    grads = []
    for split in (True, False):
        leaves = [z.clone().requires_grad_(True) for z in (x0, w0, g0, b0)]
        x, w, g, beta = leaves
        if split:
            q, k, v = tconv.tree_conv(x, w, None, tree, split_sizes=sizes)
        else:
            q, k, v = torch.split(tconv.tree_conv(x, w, None, tree), list(sizes), dim=-1)
        o, _ = gdn_tree(q.view(T, Hk, D), k.view(T, Hk, D), v.view(T, Hv, D), g, beta, tree, None, True)
        tconv._join_columns = spy
        try:
            grads.append(torch.autograd.grad((o.float() * d_o.float()).sum(), leaves))
        finally:
            tconv._join_columns = real_join
    torch.cuda.synchronize()
    assert joined == [True]
    for name, a, b in zip(("x", "weight", "g", "beta"), *grads):
        assert torch.equal(a, b), name
