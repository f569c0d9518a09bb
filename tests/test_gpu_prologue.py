"""GPU parity of the fused attention prologue (tt_qk_prologue_fwd / _bwd:
q/k RMSNorm + rotary embedding) against the float64 oracle
(oracle/prologue.py, pinned to transformers' Qwen3RMSNorm and
apply_rotary_pos_emb), through the C ABI: outputs, dq, dk and both norm-weight
gradients.

Bars: float32 max_rel < 1e-5 per tensor; bf16 < 2e-2. Full size (the 16K
agent tree, 32 q + 8 kv heads, bf16): a sample of rows against the oracle and
the weight gradients (full reductions over every row) against the oracle.
"""
import numpy as np
import pytest
import torch

from oracle.prologue import qk_prologue
from tree_training_amd.prologue import qk_prologue_backward, qk_prologue_forward
from tree_training_amd.workloads import agent_tree

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
D = 128


def _rope(pos, theta=1e6):
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    f = torch.as_tensor(pos, dtype=torch.float64)[:, None] * inv[None]
    emb = torch.cat([f, f], dim=-1)
    return emb.cos(), emb.sin()


def _case(T, Hq, Hkv, seed, pos):
    g = torch.Generator().manual_seed(seed)
    proj_q = torch.randn(T, Hq * D, dtype=torch.float64, generator=g) * 2.0
    proj_k = torch.randn(T, Hkv * D, dtype=torch.float64, generator=g) * 0.5
    qw = torch.rand(D, dtype=torch.float64, generator=g) + 0.5
    kw = torch.rand(D, dtype=torch.float64, generator=g) + 0.5
    cos, sin = _rope(pos)
    dq = torch.randn(T, Hq, D, dtype=torch.float64, generator=g)
    dk = torch.randn(T, Hkv, D, dtype=torch.float64, generator=g)
    return proj_q, proj_k, qw, kw, cos, sin, dq, dk


def _oracle(proj_q, proj_k, qw, kw, cos, sin, dq, dk, Hq, Hkv, eps=1e-6):
    T = proj_q.shape[0]
    x = proj_q.view(T, Hq, D).clone().requires_grad_(True)
    y = proj_k.view(T, Hkv, D).clone().requires_grad_(True)
    w1, w2 = qw.clone().requires_grad_(True), kw.clone().requires_grad_(True)
    qo, ko = qk_prologue(x, w1, eps, cos, sin), qk_prologue(y, w2, eps, cos, sin)
    grads = torch.autograd.grad((qo * dq).sum() + (ko * dk).sum(), (x, y, w1, w2))
    return [qo.detach(), ko.detach()] + list(grads)


def _gpu(proj_q, proj_k, qw, kw, cos, sin, dq, dk, Hq, Hkv, dtype, eps=1e-6):
    T = proj_q.shape[0]
    t = lambda a: a.to(DEV, dtype)
    pq, pk = t(proj_q), t(proj_k)
    q_raw, k_raw = pq.view(T, Hq, D), pk.view(T, Hkv, D)        # strided like the projection outputs
    qo, ko = qk_prologue_forward(q_raw, k_raw, t(qw), t(kw), eps, eps, t(cos), t(sin))
    gq, gk, gqw, gkw = qk_prologue_backward(q_raw, k_raw, t(qw), t(kw), eps, eps, t(cos), t(sin), t(dq), t(dk))
    torch.cuda.synchronize()
    return [x.double().cpu() for x in (qo, ko, gq, gk, gqw, gkw)]


def _rel(a, b):
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


NAMES = ("q", "k", "dq", "dk", "dq_weight", "dk_weight")


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("T,Hq,Hkv", [(47, 32, 8), (5, 4, 1), (130, 8, 2)])
def test_prologue_matches_oracle(dtype, tol, T, Hq, Hkv):
    pos = np.random.default_rng(T).integers(0, 3000, T)
    args = _case(T, Hq, Hkv, T + Hq, pos)
    if dtype == torch.bfloat16:           # the oracle sees the same rounded inputs
        args = tuple(a.bfloat16().double() for a in args)
    print(f"prologue {dtype} T={T} Hq={Hq} Hkv={Hkv}", flush=True)
    got = _gpu(*args, Hq, Hkv, dtype)
    ref = _oracle(*args, Hq, Hkv)
    for n, a, b in zip(NAMES, got, ref):
        assert _rel(a, b) < tol, (n, _rel(a, b))


def test_prologue_full_size_bf16():
    lens, par = agent_tree(0)
    T, Hq, Hkv = sum(lens), 32, 8
    from oracle.tree_meta import meta_closed_form
    pos = np.asarray(meta_closed_form(lens, par)["pos"])
    args = tuple(a.bfloat16().double() for a in _case(T, Hq, Hkv, 1, pos))
    print(f"prologue full size T={T}", flush=True)
    got = _gpu(*args, Hq, Hkv, torch.bfloat16)
    rows = torch.from_numpy(np.random.default_rng(2).choice(T, 512, replace=False))
    sub = [args[0][rows], args[1][rows], args[2], args[3], args[4][rows], args[5][rows], args[6][rows], args[7][rows]]
    ref = _oracle(*sub, Hq, Hkv)
    for n, a, b in zip(NAMES[:4], got[:4], ref[:4]):
        assert _rel(a[rows], b) < 2e-2, n
    full = _oracle(*args, Hq, Hkv)
    assert _rel(got[4], full[4]) < 2e-2 and _rel(got[5], full[5]) < 2e-2
