"""GPU parity of the tree gated-delta-rule scan with a caller-given initial
state and gradients flowing into the node states (the reference's
``initial_state`` and differentiable ``last_state``, tree_dfs_ssm.py:84-86,
155), through the C ABI (tt_gdn_problem.initial_state; the d_node_states and
d_initial_state arguments of tt_gdn_tree_bwd / tt_gdn_tree_bwd_saved).

Oracles: autograd on float64 through ``oracle.gdn.gdn_tree_torch`` (exact
rule) and ``oracle.gdn.gdn_tree_reference_torch`` (the reference's I + R + R^2
per node), both pinned against transformers' recurrence from a given state
and against finite differences. Bars: float32 outputs, node states and every
gradient (dq, dk, dv, dg, dbeta, d_initial_state) max_rel < 1e-5; bf16 < 2e-2
(max |error| over max |reference|). At the 16K agent-tree size: the tree cut
below its trunk, with the subtrees run as a forest of their own from the
trunk's final state, gives bitwise the whole tree's outputs, node states and
gradients (those of the trunk's tokens through the forest's initial-state
gradient fed back into a run of the trunk alone).
"""
import numpy as np
import pytest
import torch

from oracle import gdn as ogdn
from tree_training_amd import gdn as tgdn
from tree_training_amd.gdn import GdnTree
from tree_training_amd.workloads import agent_tree

pytestmark = pytest.mark.gpu
D = 128
NAMES = ("dq", "dk", "dv", "dg", "dbeta", "d_initial_state")

# Two roots, nodes of 5 to 70 tokens (one to three chunks, ragged ends).
LENS, PAR = [45, 33, 70, 5, 38, 64], [-1, 0, 0, 2, -1, 4]


def _inputs(T, Hk, Hv, n_nodes, seed, g_scale):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((T, Hk, D)).astype(np.float32)
    k = rng.standard_normal((T, Hk, D)).astype(np.float32)
    v = rng.standard_normal((T, Hv, D)).astype(np.float32)
    g = (-np.abs(rng.standard_normal((T, Hv))) * g_scale).astype(np.float32)
    beta = (1.0 / (1.0 + np.exp(-rng.standard_normal((T, Hv))))).astype(np.float32)
    s0 = (0.5 * rng.standard_normal((Hv, D, D))).astype(np.float32)
    d_o = rng.standard_normal((T, Hv, D)).astype(np.float32)
    d_st = (0.1 * rng.standard_normal((n_nodes, Hv, D, D))).astype(np.float32)
    return q, k, v, g, beta, s0, d_o, d_st


def _rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def _dev(x, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x)).to(torch.device("cuda", 0))
    return t.to(dtype) if dtype is not None else t


@pytest.mark.parametrize("keep", [True, False], ids=["saved", "recompute"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("mode", ["exact", "reference"])
def test_gdn_initial_state_and_state_gradients_match_oracle(mode, dtype, keep, monkeypatch):
    monkeypatch.setattr(tgdn, "KEEP_FORWARD_STATES", keep)
    Hk, Hv, T = 2, 4, sum(LENS)
    q, k, v, g, beta, s0, d_o, d_st = _inputs(T, Hk, Hv, len(LENS), 40 + (mode == "reference"),
                                              0.2 if mode == "exact" else 0.05)
    if dtype == torch.bfloat16:   # the oracle sees the same bf16 inputs
        rb = lambda x: torch.from_numpy(x).bfloat16().float().numpy()
        q, k, v = rb(q), rb(k), rb(v)
    tree = GdnTree(LENS, PAR, torch.device("cuda", 0))
    ins = [_dev(q, dtype), _dev(k, dtype), _dev(v, dtype), _dev(g), _dev(beta), _dev(s0)]
    for t in ins:
        t.requires_grad_(True)
    o, st = tgdn.gdn_tree(*ins[:5], tree, reference_truncated=mode == "reference", initial_state=ins[5])
    loss = (o.float() * _dev(d_o)).sum() + (st * _dev(d_st)).sum()
    grads = torch.autograd.grad(loss, ins)
    torch.cuda.synchronize()

    fn = ogdn.gdn_tree_torch if mode == "exact" else ogdn.gdn_tree_reference_torch
    ref_in = [torch.from_numpy(np.asarray(x, np.float64)).requires_grad_(True) for x in (q, k, v, g, beta, s0)]
    o_ref, st_ref = fn(*ref_in[:5], LENS, PAR, initial_state=ref_in[5], return_states=True)
    ref_loss = (o_ref * torch.from_numpy(d_o.astype(np.float64))).sum() + \
        (st_ref * torch.from_numpy(d_st.astype(np.float64))).sum()
    ref_grads = torch.autograd.grad(ref_loss, ref_in)

    bar = 1e-5 if dtype == torch.float32 else 2e-2
    assert _rel(o.detach().float().cpu().numpy(), o_ref.detach().numpy()) < bar, "o"
    assert _rel(st.detach().cpu().numpy(), st_ref.detach().numpy()) < bar, "node states"
    for name, a, b in zip(NAMES, grads, ref_grads):
        assert _rel(a.float().cpu().numpy(), b.numpy()) < bar, name


def test_gdn_drop_in_initial_state_and_last_state_gradient():
    """``torch_chunk_gated_delta_rule_tree_varlen`` with the reference's
    ``initial_state`` [1, Hv, 128, 128] and ``output_final_state``: the last
    node's state is returned differentiable, and a loss on it alone (no
    gradient through the output) reaches q, k, v, g, beta and the initial
    state as autograd through the float64 oracle says (float32, < 1e-5)."""
    Hk, Hv, T = 2, 4, sum(LENS)
    q, k, v, g, beta, s0, _, d_st = _inputs(T, Hk, Hv, len(LENS), 44, 0.2)
    bounds, s = [], 0
    for L in LENS:
        bounds.append((s, s + L))
        s += L
    ins = [_dev(q)[None], _dev(k)[None], _dev(v)[None], _dev(g)[None], _dev(beta)[None], _dev(s0)[None]]
    for t in ins:
        t.requires_grad_(True)
    o, last = tgdn.torch_chunk_gated_delta_rule_tree_varlen(*ins[:5], bounds, PAR, initial_state=ins[5],
                                                            output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert o.shape == (1, T, Hv, D) and last.shape == (1, Hv, D, D)
    grads = torch.autograd.grad((last * _dev(d_st[-1])[None]).sum(), ins)
    torch.cuda.synchronize()

    ref_in = [torch.from_numpy(np.asarray(x, np.float64)).requires_grad_(True) for x in (q, k, v, g, beta, s0)]
    o_ref, st_ref = ogdn.gdn_tree_torch(*ref_in[:5], LENS, PAR, initial_state=ref_in[5], return_states=True)
    assert _rel(o[0].detach().cpu().numpy(), o_ref.detach().numpy()) < 1e-5
    assert _rel(last[0].detach().cpu().numpy(), st_ref[-1].detach().numpy()) < 1e-5
    # a node's state does not depend on q: autograd through the oracle has no dq
    ref_grads = torch.autograd.grad((st_ref[-1] * torch.from_numpy(d_st[-1].astype(np.float64))).sum(), ref_in,
                                    allow_unused=True)
    assert ref_grads[0] is None and not grads[0].any()
    for name, a, b in list(zip(NAMES, grads, ref_grads))[1:]:
        assert _rel(a[0].cpu().numpy(), b.numpy()) < 1e-5, name


def test_gdn_16k_tree_cut_below_its_trunk_continues_from_initial_state():
    """Full size (agent tree, 16,318 tokens, 16 q/k heads, 32 v heads, bf16),
    cut below its trunk (the chain of nodes from the root down to the first
    node with several children): the subtrees under the trunk, run as a
    forest of their own from the trunk's final state, give bitwise the whole
    tree's outputs and node states, and, with the same d_o, bitwise the
    gradients of their own tokens; the initial-state gradient of that forest
    (its roots' terms summed in node order, as a node's children's are), fed
    back as the incoming gradient of the trunk's last state in a run of the
    trunk alone, gives bitwise the trunk tokens' gradients of the whole
    tree."""
    lens, par = agent_tree(0)
    T, Hk, Hv = sum(lens), 16, 32
    c = 0                                         # the trunk: nodes 0 .. c, a chain
    while par.count(c) == 1 and par[c + 1] == c:
        c += 1
    assert par[:c + 1] == list(range(-1, c)) and par.count(c) >= 2 and min(par[c + 1:]) == c
    rng = np.random.default_rng(9)
    a, b = rng.standard_normal((T, Hv)), rng.standard_normal((T, Hv))
    g, beta = ogdn.gdn_gates(a, b, np.log(rng.uniform(1e-3, 16, Hv)), np.ones(Hv))
    bf = torch.bfloat16
    q = _dev(rng.standard_normal((T, Hk, D)).astype(np.float32), bf)
    k = _dev(rng.standard_normal((T, Hk, D)).astype(np.float32), bf)
    v = _dev(rng.standard_normal((T, Hv, D)).astype(np.float32), bf)
    d_o = _dev(rng.standard_normal((T, Hv, D)).astype(np.float32), bf)
    g, beta = _dev(g.astype(np.float32)), _dev(beta.astype(np.float32))
    dev = torch.device("cuda", 0)
    r = sum(lens[:c + 1])                         # tokens of the trunk

    whole = GdnTree(lens, par, dev)
    o, st = tgdn.gdn_tree_forward(q, k, v, g, beta, whole)
    gw = tgdn.gdn_tree_backward(q, k, v, g, beta, d_o, whole)

    trunk = GdnTree(lens[:c + 1], par[:c + 1], dev)
    top = [x[:r] for x in (q, k, v, g, beta)]
    o0, st0 = tgdn.gdn_tree_forward(*top, trunk)
    rest = GdnTree(lens[c + 1:], [-1 if p == c else p - c - 1 for p in par[c + 1:]], dev)
    sub = [x[r:] for x in (q, k, v, g, beta)]
    o1, st1 = tgdn.gdn_tree_forward(*sub, rest, initial_state=st0[c])
    g1 = tgdn.gdn_tree_backward(*sub, d_o[r:], rest, initial_state=st0[c], initial_state_grad=True)
    d_trunk = torch.zeros((c + 1, Hv, D, D), dtype=torch.float32, device=dev)
    d_trunk[c] = g1[5]
    g0 = tgdn.gdn_tree_backward(*top, d_o[:r], trunk, d_states=d_trunk)
    torch.cuda.synchronize()

    assert torch.isfinite(o.float()).all() and torch.isfinite(g1[5]).all() and g1[5].abs().max() > 0
    assert torch.equal(o[:r], o0) and torch.equal(o[r:], o1)
    assert torch.equal(st[:c + 1], st0) and torch.equal(st[c + 1:], st1)
    for name, a_w, b_r, b_0 in zip(NAMES, gw, g1, g0):
        assert torch.equal(a_w[r:], b_r), name
        assert torch.equal(a_w[:r], b_0), name


@pytest.mark.parametrize("mode", ["exact", "reference"])
def test_gdn_last_state_gradient_alone_equals_full_buffer(mode):
    """d_last_state (tt_gdn_problem.d_states_last_only) gives bitwise the
    gradients of a full d_states buffer that is zero except for the last
    node, with the saved forward and with the recomputing backward."""
    T = sum(LENS)
    q, k, v, g, beta, s0, d_o, d_st = _inputs(T, 2, 4, len(LENS), 21, 0.3)
    tree = GdnTree(LENS, PAR, torch.device("cuda", 0))
    ins = [_dev(x) for x in (q, k, v, g, beta)]
    full = torch.zeros(len(LENS), 4, D, D, device="cuda:0")
    full[-1] = _dev(d_st[-1])
    trunc = mode == "reference"
    _, _, saved = tgdn._gdn_forward(*ins, tree, None, True, True, trunc, None)
    for kept in (saved, None):
        a = tgdn.gdn_tree_backward(*ins, _dev(d_o), tree, saved=kept, reference_truncated=trunc, d_states=full)
        b = tgdn.gdn_tree_backward(*ins, _dev(d_o), tree, saved=kept, reference_truncated=trunc,
                                   d_last_state=_dev(d_st[-1]))
        torch.cuda.synchronize()
        for name, x, y in zip(NAMES, a, b):
            assert torch.equal(x, y), (mode, kept is None, name)
