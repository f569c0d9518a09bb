"""Pins the fp64 attention oracle against library routines and invariants."""
import numpy as np
import torch

from oracle.attention import attn_bwd, attn_fwd, gateway_mask, key_interval_mask, max_rel
from oracle.dense_path import additive_mask, dense_fwd_bwd
from oracle.tree_meta import mask_from_horizon, meta_closed_form

C1_LENS = [3, 4, 3, 4, 5, 3, 3, 4, 4, 3, 4, 3, 4]
C1_PAR = [-1, 0, 1, 2, 3, 3, 2, 6, -1, 8, 9, 8, 11]


def _inputs(N, Lk, Hq=4, Hkv=2, D=16, seed=0):
    g = np.random.default_rng(seed)
    q = g.standard_normal((N, Hq, D))
    k = g.standard_normal((Lk, Hkv, D))
    v = g.standard_normal((Lk, Hkv, D))
    do = g.standard_normal((N, Hq, D))
    return q, k, v, do


def test_fwd_bwd_match_torch_sdpa_autograd():
    m = meta_closed_form(C1_LENS, C1_PAR)
    mask = mask_from_horizon(m["horizon"])
    N = m["T"]
    q, k, v, do = _inputs(N, N, seed=1)
    scale = 16 ** -0.5
    o, lse = attn_fwd(q, k, v, mask, scale)
    dq, dk, dv = attn_bwd(q, k, v, mask, scale, do)
    # torch SDPA (float64) + autograd on the dense additive mask, HF layout
    tq = torch.tensor(q).permute(1, 0, 2)[None]
    tk = torch.tensor(k).permute(1, 0, 2)[None]
    tv = torch.tensor(v).permute(1, 0, 2)[None]
    tdo = torch.tensor(do)[None]
    am = additive_mask(torch.tensor(mask), torch.float64)
    to, tdq, tdk, tdv = dense_fwd_bwd(tq, tk, tv, am, scale, tdo)
    assert max_rel(to[0].numpy(), o) < 1e-12
    assert max_rel(tdq[0].permute(1, 0, 2).numpy(), dq) < 1e-12
    assert max_rel(tdk[0].permute(1, 0, 2).numpy(), dk) < 1e-12
    assert max_rel(tdv[0].permute(1, 0, 2).numpy(), dv) < 1e-12
    # lse: log of the softmax denominator
    s = np.einsum("nhd,mhd->hnm", q, np.repeat(k, 2, axis=1)) * scale
    s[:, ~mask] = -np.inf
    ref_lse = np.log(np.exp(s).sum(-1))
    assert np.abs(ref_lse - lse).max() < 1e-12


def test_finite_difference_gradients():
    m = meta_closed_form([2, 3, 2], [-1, 0, 0])
    mask = mask_from_horizon(m["horizon"])
    N = m["T"]
    q, k, v, do = _inputs(N, N, Hq=2, Hkv=1, D=4, seed=2)
    scale = 0.7
    dq, dk, dv = attn_bwd(q, k, v, mask, scale, do)

    def f(qq, kk, vv):
        return float((attn_fwd(qq, kk, vv, mask, scale)[0] * do).sum())

    eps = 1e-6
    for arr, grad, which in ((q, dq, 0), (k, dk, 1), (v, dv, 2)):
        it = np.nditer(arr, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            args_p = [q.copy(), k.copy(), v.copy()]
            args_m = [q.copy(), k.copy(), v.copy()]
            args_p[which][idx] += eps
            args_m[which][idx] -= eps
            fd = (f(*args_p) - f(*args_m)) / (2 * eps)
            assert abs(fd - grad[idx]) < 1e-6 * max(1.0, abs(fd))


def test_per_path_equivalence():
    """Tree rows of each root-to-leaf path equal plain causal attention over
    that path's concatenated tokens (the tree-training claim)."""
    m = meta_closed_form(C1_LENS, C1_PAR)
    mask = mask_from_horizon(m["horizon"])
    N = m["T"]
    q, k, v, do = _inputs(N, N, seed=3)
    scale = 0.25
    o, _ = attn_fwd(q, k, v, mask, scale)
    start = m["node_start"]
    lens = np.asarray(C1_LENS)
    for leaf in [4, 5, 7, 10, 12]:
        chain = []
        c = leaf
        while c >= 0:
            chain.append(c)
            c = C1_PAR[c]
        chain.reverse()
        toks = np.concatenate([np.arange(start[c], start[c] + lens[c]) for c in chain])
        L = len(toks)
        causal = np.tril(np.ones((L, L), bool))
        op, _ = attn_fwd(q[toks], k[toks], v[toks], causal, scale)
        assert np.abs(op - o[toks]).max() < 1e-12


def test_gateway_mask_and_key_intervals():
    own = mask_from_horizon(meta_closed_form([2, 2], [-1, 0])["horizon"])
    bias = [0.0, -np.inf, 0.0]
    gm = gateway_mask(own, bias)
    assert gm.shape == (4, 7)
    assert gm[:, 0].all() and not gm[:, 1].any() and gm[:, 2].all()
    lo = [0, 0, 0] + list(range(4))
    hi = [4, 0, 4] + list(meta_closed_form([2, 2], [-1, 0])["horizon"])
    assert np.array_equal(key_interval_mask(lo, hi, 4), gm)
