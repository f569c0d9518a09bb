"""GPU parity of the tree-correct short convolution (tt_tree_conv_fwd,
tt_tree_conv_bwd) against the float64 oracle (oracle/gdn.py: ``tree_conv``,
pinned to torch's conv1d on every root-to-leaf path, and autograd through
``tree_conv_torch`` for the gradients), through the C ABI.

Bars: float32 max_rel < 1e-5 for y, dx, dweight, dbias; bf16 < 2e-2 (max
|error| over max |reference|). At full size (the 16K agent tree, 8192
channels) the checks are per-path: each root-to-leaf path run alone as a
chain gives bitwise the same y on its tokens, and with dy supported on one
path dx equals the chain's bitwise and vanishes elsewhere.
"""
import numpy as np
import pytest
import torch

from oracle import gdn as ogdn
from tree_training_amd.conv import _tree_correct_conv_varlen, tree_conv, tree_conv_backward, tree_conv_forward
from tree_training_amd.gdn import GdnTree
from tree_training_amd.workloads import agent_tree, random_forest

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)

CASES = {
    "short_nodes_k4": dict(topo=lambda: random_forest(3, node_len=(1, 3)), C=8, K=4, bias=True),
    "forest_k4_wide": dict(topo=lambda: random_forest(9, node_len=(1, 40)), C=1028, K=4, bias=False),
    "single_tokens_k3": dict(topo=lambda: ([1] * 9, [-1, 0, 1, 1, 3, -1, 5, 5, 0]), C=12, K=3, bias=True),
    "chain_k2": dict(topo=lambda: ([5, 1, 7], [-1, 0, 1]), C=16, K=2, bias=True),
    "chain_k1": dict(topo=lambda: ([3, 4], [-1, 0]), C=4, K=1, bias=False),
}


def _inputs(T, C, K, seed, bias):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, C)).astype(np.float32)
    w = (rng.standard_normal((C, K)) * 0.5).astype(np.float32)
    b = rng.standard_normal(C).astype(np.float32) if bias else None
    dy = rng.standard_normal((T, C)).astype(np.float32)
    return x, w, b, dy


def _rel(a, b):
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def _oracle(x, w, b, dy, lens, par):
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64)).requires_grad_(True)
    tx, tw = t(x), t(w)
    tb = t(b) if b is not None else None
    y = ogdn.tree_conv_torch(tx, tw, tb, lens, par)
    grads = torch.autograd.grad((y * torch.from_numpy(np.asarray(dy, np.float64))).sum(),
                                [tx, tw] + ([tb] if tb is not None else []))
    return [y.detach().numpy()] + [g.numpy() for g in grads]


def _gpu(x, w, b, dy, lens, par, dtype):
    tree = GdnTree(lens, par, DEV)
    t = lambda a: torch.from_numpy(a).to(DEV).to(dtype) if a is not None else None
    y = tree_conv_forward(t(x), t(w), t(b), tree)
    dx, dw, db = tree_conv_backward(t(x), t(w), t(b), t(dy), tree)
    torch.cuda.synchronize()
    out = [y.float().cpu().numpy(), dx.float().cpu().numpy(), dw.cpu().numpy()]
    return out + ([db.cpu().numpy()] if db is not None else [])


@pytest.mark.parametrize("case", list(CASES))
def test_conv_fp32_matches_oracle(case):
    c = CASES[case]
    lens, par = c["topo"]()
    x, w, b, dy = _inputs(sum(lens), c["C"], c["K"], sum(map(ord, case)), c["bias"])
    print(f"tree conv fp32 {case}: T={sum(lens)} C={c['C']} K={c['K']}", flush=True)
    got = _gpu(x, w, b, dy, lens, par, torch.float32)
    ref = _oracle(x, w, b, dy, lens, par)
    assert np.abs(ref[0] - ogdn.tree_conv(x, w, b, lens, par)).max() < 1e-12
    for name, a, r in zip(("y", "dx", "dw", "db"), got, ref):
        assert _rel(a, r) < 1e-5, (case, name, _rel(a, r))


@pytest.mark.parametrize("case", ["short_nodes_k4", "forest_k4_wide"])
def test_conv_bf16_matches_oracle(case):
    c = CASES[case]
    lens, par = c["topo"]()
    rb = lambda a: torch.from_numpy(a).bfloat16().float().numpy() if a is not None else None
    x, w, b, dy = map(rb, _inputs(sum(lens), c["C"], c["K"], 1 + sum(map(ord, case)), c["bias"]))
    got = _gpu(x, w, b, dy, lens, par, torch.bfloat16)
    ref = _oracle(x, w, b, dy, lens, par)
    for name, a, r in zip(("y", "dx", "dw", "db"), got, ref):
        assert _rel(a, r) < 2e-2, (case, name, _rel(a, r))


def test_conv_autograd_and_dropin():
    """The autograd Function's gradients equal tree_conv_backward's, and the
    reference-signature drop-in (channel-major input, a module with conv1d)
    gives the same y."""
    lens, par = random_forest(4, node_len=(1, 6))
    T, C, K = sum(lens), 64, 4
    x, w, b, dy = _inputs(T, C, K, 3, True)
    tree = GdnTree(lens, par, DEV)
    tx = torch.from_numpy(x).to(DEV).requires_grad_(True)
    tw = torch.from_numpy(w).to(DEV).reshape(C, 1, K).requires_grad_(True)
    tb = torch.from_numpy(b).to(DEV).requires_grad_(True)
    y = tree_conv(tx, tw, tb, tree)
    y.backward(torch.from_numpy(dy).to(DEV))
    dx, dw, db = tree_conv_backward(tx.detach(), tw.detach(), tb.detach(), torch.from_numpy(dy).to(DEV), tree)
    assert torch.equal(tx.grad, dx) and torch.equal(tw.grad.reshape(C, K), dw) and torch.equal(tb.grad, db)

    class _Ssm(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.conv1d = torch.nn.Conv1d(C, C, K, groups=C, padding=K - 1, bias=True)
            self.activation = "silu"
    ssm = _Ssm().to(DEV)
    with torch.no_grad():
        ssm.conv1d.weight.copy_(tw.detach())
        ssm.conv1d.bias.copy_(tb.detach())
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]])
    bounds = [(int(s), int(s + n)) for s, n in zip(starts, lens)]
    out = _tree_correct_conv_varlen(ssm, tx.detach().t().contiguous()[None], bounds, par)
    assert out.shape == (1, C, T)
    assert torch.equal(out[0].t(), y.detach())


def test_conv_16k_tree_per_path():
    lens, par = agent_tree(0)
    T, C, K = sum(lens), 8192, 4
    rng = np.random.default_rng(0)
    x = torch.from_numpy(rng.standard_normal((T, C), dtype=np.float32)).to(DEV).bfloat16()
    w = torch.from_numpy(rng.standard_normal((C, K), dtype=np.float32) * 0.5).to(DEV).bfloat16()
    tree = GdnTree(lens, par, DEV)
    y = tree_conv_forward(x, w, None, tree)
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]])
    leaves = [i for i in range(len(lens)) if i not in set(par)]
    leaf = leaves[len(leaves) // 3]
    path, j = [], leaf
    while j >= 0:
        path.append(j)
        j = par[j]
    path = path[::-1]
    idx = torch.from_numpy(np.concatenate([np.arange(starts[i], starts[i] + lens[i]) for i in path])).to(DEV)
    chain = GdnTree([lens[i] for i in path], list(range(-1, len(path) - 1)), DEV)
    print(f"tree conv 16k: leaf={leaf} path_tokens={len(idx)}", flush=True)
    y_p = tree_conv_forward(x[idx].contiguous(), w, None, chain)
    assert torch.equal(y[idx], y_p)
    dy = torch.zeros(T, C, device=DEV, dtype=torch.bfloat16)
    dy[idx] = torch.randn(len(idx), C, device=DEV).bfloat16()
    dx, dw, _ = tree_conv_backward(x, w, None, dy, tree)
    dx_p, dw_p, _ = tree_conv_backward(x[idx].contiguous(), w, None, dy[idx].contiguous(), chain)
    off = torch.ones(T, dtype=torch.bool, device=DEV)
    off[idx] = False
    assert torch.equal(dx[idx], dx_p)
    assert not dx[off].any()
    assert float((dw - dw_p).abs().max() / dw_p.abs().max()) < 1e-5
