"""GPU parity of the HIP kernels against the CPU oracle (through the C ABI)."""
import ctypes
import math
import sys

import numpy as np
import pytest
import torch

from oracle.attention import attn_bwd, attn_fwd, key_interval_mask, max_rel
from oracle.tree_meta import mask_from_horizon, meta_closed_form
from tests.conftest import load_golden
from tree_training_amd import workloads

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
HQ, HKV, D = 32, 8, 128


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _meta(lens, par, pos_offset=0):
    from tree_training_amd.meta import TreeMetaDevice
    return TreeMetaDevice(lens, par, pos_offset=pos_offset, device=DEV, validate=True)


# --------------------------------------------------------------------------- MFMA layout
def test_mfma_layout_selftest():
    import ctypes
    from tree_training_amd._lib import lib
    from tree_training_amd.meta import _ptr, _stream
    say("selftest mfma32")
    g = torch.Generator().manual_seed(0)
    a = torch.randn(32, 16, generator=g).bfloat16()
    b = torch.randn(16, 32, generator=g).bfloat16()
    da, db = a.to(DEV), b.to(DEV)
    d = torch.empty(32, 32, device=DEV)
    assert lib().tt_selftest_mfma32(_ptr(da), _ptr(db), _ptr(d), _stream(torch.device(DEV))) == 0
    torch.cuda.synchronize()
    ref = a.float() @ b.float()
    assert torch.allclose(d.cpu(), ref, atol=1e-4, rtol=1e-4), (d.cpu() - ref).abs().max()


# --------------------------------------------------------------------------- metadata
def test_meta_c1_fixture():
    spec = load_golden("c1_tree.json")
    lens = [n["len"] for n in spec["nodes"]]
    par = [n["parent"] for n in spec["nodes"]]
    m = _meta(lens, par)
    assert m.pos.cpu().tolist() == spec["dfs_pos_ids"]
    assert m.node_hend.cpu().tolist() == spec["chunk_horizon"]
    assert m.node_start.cpu().tolist() == [b[0] for b in spec["chunk_boundaries"]]
    from tree_training_amd.meta import KeyPlan
    kp = KeyPlan(m.horizon, validate=True)
    assert kp.visible_pairs() == spec["nnz"]
    cf = meta_closed_form(lens, par)
    assert np.array_equal(kp.dense_mask().cpu().numpy(), mask_from_horizon(cf["horizon"]))


@pytest.mark.parametrize("seed", range(12))
def test_meta_random_forests(seed):
    lens, par = workloads.random_forest(seed, node_len=(1, 70))
    say(f"meta random forest seed={seed} n={len(lens)} T={sum(lens)}")
    off = (seed * 37) % 100
    m = _meta(lens, par, pos_offset=off)
    ref = meta_closed_form(lens, par, pos_offset=off)
    assert np.array_equal(m.pos.cpu().numpy(), ref["pos"])
    assert np.array_equal(m.horizon.cpu().numpy(), ref["horizon"])
    assert np.array_equal(m.node_of.cpu().numpy(), ref["node_of"])
    assert np.array_equal(m.node_off.cpu().numpy(), ref["node_off"])


def _branchy(n):
    """n nodes, parents drawn below each node (pre-order), lengths 1..9."""
    rng = np.random.default_rng(n)
    par = [-1]
    for i in range(1, n):
        par.append(int(rng.integers(max(0, i - 6), i)))
    # pre-order: regroup children after their parent (depth-first walk)
    kids = [[] for _ in range(n)]
    for i in range(1, n):
        kids[par[i]].append(i)
    order, stack = [], [0]
    while stack:
        v = stack.pop()
        order.append(v)
        stack.extend(reversed(kids[v]))
    new = {v: k for k, v in enumerate(order)}
    lens = [int(rng.integers(1, 10)) for _ in range(n)]
    return [lens[v] for v in order], [-1 if par[v] < 0 else new[par[v]] for v in order]


# 512 and 513 nodes: the largest tree whose node arrays sit in LDS, and the smallest in the workspace
@pytest.mark.parametrize("name", ["agent16k", "rollout48k", "chain", "star", "branchy512", "branchy513"])
def test_meta_large(name):
    topo = {
        "agent16k": lambda: workloads.agent_tree(0),
        "rollout48k": lambda: workloads.rollout_tree(0),
        "chain": lambda: ([3] * 3000, [-1] + list(range(2999))),
        "star": lambda: ([5] + [2] * 5000, [-1] + [0] * 5000),
        "branchy512": lambda: _branchy(512),
        "branchy513": lambda: _branchy(513),
    }[name]()
    lens, par = topo
    say(f"meta large {name} n={len(lens)} T={sum(lens)}")
    m = _meta(lens, par)
    ref = meta_closed_form(lens, par)
    assert np.array_equal(m.pos.cpu().numpy(), ref["pos"])
    assert np.array_equal(m.horizon.cpu().numpy(), ref["horizon"])
    assert np.array_equal(m.node_off.cpu().numpy(), ref["node_off"])
    from tree_training_amd.meta import KeyPlan
    kp = KeyPlan(m.horizon)
    assert kp.visible_pairs() == workloads.visible_pairs(topo) == int((ref["pos"] + 1).sum())


def test_meta_rejects_bad_input():
    from tree_training_amd.meta import TreeMetaDevice
    with pytest.raises(ValueError):
        TreeMetaDevice([2, 3], [-1, 1], device=DEV, validate=True)   # parent not before child
    with pytest.raises(ValueError):
        TreeMetaDevice([2, 0, 1], [-1, 0, 0], device=DEV, validate=True)  # empty node
    with pytest.raises(ValueError):
        TreeMetaDevice([1, 1, 1, 1], [-1, 0, 0, 1], device=DEV, validate=True)   # not pre-order


def test_meta_status_flags_non_preorder():
    """The device check alone (host check skipped): parent < i holds for
    parents [-1, 0, 0, 1] but node 3 follows its parent's closed subtree."""
    from tree_training_amd._lib import TT_STATUS_BAD_PARENT
    from tree_training_amd.meta import TreeMetaDevice
    m = TreeMetaDevice([1, 1, 1, 1], [-1, 0, 0, 1], device=DEV, validate=False)
    assert int(m.status.item()) & TT_STATUS_BAD_PARENT
    for lens, par in [([3, 4, 3, 4, 5, 3, 3, 4, 4, 3, 4, 3, 4], [-1, 0, 1, 2, 3, 3, 2, 6, -1, 8, 9, 8, 11]),
                      ([1, 1, 1, 1, 1], [-1, 0, 1, 1, 0])]:
        assert int(TreeMetaDevice(lens, par, device=DEV, validate=False).status.item()) == 0


# --------------------------------------------------------------------------- tile plan
def _plan_expected(lo, hi, n_q):
    """The tile plan restated in numpy from the key intervals [lo, hi): header,
    per 128-query block the ascending non-empty 64-key tiles tagged full, the
    heaviest-first block order, per 128-key tile the visible query range, its
    heaviest-first order and the dK/dV work-item offsets."""
    lo, hi = np.asarray(lo, np.int64), np.asarray(hi, np.int64)
    n_keys = len(lo)
    n_qb, n_kt, n_kb = -(-n_q // 128), -(-n_keys // 64), -(-n_keys // 128)
    a, b = np.maximum(lo, 0), np.minimum(hi, n_q)
    P = int(np.clip(b - a, 0, None).sum())
    rows = []
    for qb in range(n_qb):
        i0, i1 = 128 * qb, min(128 * qb + 128, n_q)
        lst = []
        for kt in range(n_kt):
            j = np.arange(64 * kt, min(64 * kt + 64, n_keys))
            some = (np.maximum(lo[j], i0) < np.minimum(hi[j], i1)).any()
            every = len(j) == 64 and ((lo[j] <= i0) & (hi[j] >= i1)).all()
            if some:
                lst.append((kt << 1) | int(every))
        rows.append(lst)
    cnt = np.array([len(r) for r in rows])
    row_order = sorted(range(n_qb), key=lambda i: (-cnt[i], i))
    qlo, qhi = np.zeros(n_kb, np.int64), np.zeros(n_kb, np.int64)
    for kb in range(n_kb):
        j = np.arange(128 * kb, min(128 * kb + 128, n_keys))
        vis = a[j] < b[j]
        if vis.any():
            qlo[kb], qhi[kb] = a[j][vis].min(), b[j][vis].max()
    kb_order = sorted(range(n_kb), key=lambda i: (-(qhi[i] - qlo[i]), i))
    half = (1 << (n_q.bit_length() - 1)) // 2 if n_q >= 2 else 0
    qch = 4096 if half > 4096 else max(half, 256)
    items = [1 if qhi[k] - qlo[k] <= qch else (qhi[k] - 1) // qch - qlo[k] // qch + 1 for k in kb_order]
    kb_base = np.concatenate([[0], np.cumsum(items)])
    return dict(P=P, n_qb=n_qb, n_kt=n_kt, n_kb=n_kb, rows=rows, row_order=row_order, qlo=qlo, qhi=qhi,
                kb_order=kb_order, kb_base=kb_base)


def _plan_expected_fast(lo, hi, n_q):
    """_plan_expected vectorised over the query blocks (one numpy pass per
    64-key tile), for trees too large for the per-pair loop."""
    lo, hi = np.asarray(lo, np.int64), np.asarray(hi, np.int64)
    n_keys = len(lo)
    n_qb, n_kt, n_kb = -(-n_q // 128), -(-n_keys // 64), -(-n_keys // 128)
    a, b = np.maximum(lo, 0), np.minimum(hi, n_q)
    i0 = 128 * np.arange(n_qb)
    i1 = np.minimum(i0 + 128, n_q)
    cls = np.zeros((n_qb, n_kt), np.int64)
    for kt in range(n_kt):
        j = np.arange(64 * kt, min(64 * kt + 64, n_keys))
        some = (np.maximum(lo[j][:, None], i0[None]) < np.minimum(hi[j][:, None], i1[None])).any(0)
        every = ((lo[j][:, None] <= i0[None]) & (hi[j][:, None] >= i1[None])).all(0) & (len(j) == 64)
        cls[:, kt] = np.where(some, np.where(every, 2, 1), 0)
    rows = [[(int(kt) << 1) | int(cls[q, kt] == 2) for kt in np.nonzero(cls[q])[0]] for q in range(n_qb)]
    cnt = (cls != 0).sum(1)
    row_order = sorted(range(n_qb), key=lambda i: (-cnt[i], i))
    qlo, qhi = np.zeros(n_kb, np.int64), np.zeros(n_kb, np.int64)
    for kb in range(n_kb):
        j = np.arange(128 * kb, min(128 * kb + 128, n_keys))
        vis = a[j] < b[j]
        if vis.any():
            qlo[kb], qhi[kb] = a[j][vis].min(), b[j][vis].max()
    kb_order = sorted(range(n_kb), key=lambda i: (-(qhi[i] - qlo[i]), i))
    half = (1 << (n_q.bit_length() - 1)) // 2 if n_q >= 2 else 0
    qch = 4096 if half > 4096 else max(half, 256)
    n_items = lambda k: 1 if qhi[k] - qlo[k] <= qch else (qhi[k] - 1) // qch - qlo[k] // qch + 1
    kb_base = np.concatenate([[0], np.cumsum([n_items(k) for k in kb_order])])
    # split tiles (more than one work item) ranked in key order
    split = np.array([n_items(k) > 1 for k in range(n_kb)], bool)
    srank = np.where(split, np.cumsum(split) - 1, -1)
    # work items as (tile rank, chunk): up to 4096 items sorted by length
    # (descending), then query window (descending), rank, chunk; above that
    # window-major (top query window first; a window's items in tile order)
    total = int(kb_base[-1])
    wm = total > 4096
    if not wm:
        keyed = []
        for r, k in enumerate(kb_order):
            m = n_items(k)
            for c in range(m):
                if qhi[k] <= qlo[k]:
                    q0 = q1 = 0
                elif m == 1:
                    q0, q1 = (qlo[k] // 32) * 32, qhi[k]
                else:
                    w = qlo[k] // qch + c
                    q0, q1 = max((qlo[k] // 32) * 32, w * qch), min(qhi[k], (w + 1) * qch)
                w = qlo[k] // qch + c if m > 1 else ((qhi[k] - 1) // qch if qhi[k] > qlo[k] else 0)
                keyed.append((-min(max(q1 - q0, 0), 4096), -w, r, c))
        items = [(r, c) for _, _, r, c in sorted(keyed)]
    else:
        items = []
        for w in range((n_q - 1) // qch, -1, -1):
            for r, k in enumerate(kb_order):
                if n_items(k) > 1:
                    if qlo[k] // qch <= w <= (qhi[k] - 1) // qch:
                        items.append((r, w - qlo[k] // qch))
                elif ((qhi[k] - 1) // qch if qhi[k] > qlo[k] else 0) == w:
                    items.append((r, 0))
    assert len(items) == total
    return dict(P=int(np.clip(b - a, 0, None).sum()), n_qb=n_qb, n_kt=n_kt, n_kb=n_kb, rows=rows,
                row_order=row_order, qlo=qlo, qhi=qhi, kb_order=kb_order, kb_base=kb_base, kb_srank=srank,
                n_split=int(split.sum()), kb_item=np.array(items, np.int32).reshape(-1, 2), item_order=2 if wm else 1)


def _plan_decode(buf, n_q, n_keys):
    """The device plan buffer split at PlanLayout's offsets (64-byte header)."""
    n_qb, n_kt, n_kb = -(-n_q // 128), -(-n_keys // 64), -(-n_keys // 128)
    i32 = lambda off, n: np.frombuffer(buf, np.int32, n, off)
    o = 64
    row_cnt = i32(o, n_qb); o += 4 * n_qb
    row_order = i32(o, n_qb); o += 4 * n_qb
    row_list = i32(o, n_qb * n_kt).reshape(n_qb, n_kt); o += 4 * n_qb * n_kt
    qlo = i32(o, n_kb); o += 4 * n_kb
    qhi = i32(o, n_kb); o += 4 * n_kb
    kb_order = i32(o, n_kb); o += 4 * n_kb
    kb_base = i32(o, n_kb + 1); o += 4 * (n_kb + 1)
    kb_srank = i32(o, n_kb); o += 4 * n_kb
    o = (o + 7) & ~7
    hdr = i32(8, 6)
    kb_item = i32(o, 2 * int(hdr[3])).reshape(-1, 2)
    return dict(P=int(np.frombuffer(buf, np.uint64, 1, 0)[0]), n_qb=int(hdr[0]), n_kt=int(hdr[1]),
                n_kb=int(hdr[2]), n_items=int(hdr[3]), n_split=int(hdr[4]), item_order=int(hdr[5]),
                rows=[list(row_list[q, :row_cnt[q]]) for q in range(n_qb)], row_order=list(row_order),
                qlo=qlo, qhi=qhi, kb_order=list(kb_order), kb_base=kb_base, kb_srank=kb_srank, kb_item=kb_item)


def test_build_trees_matches_separate_calls():
    """meta.build_trees (tt_trees_build, three launches per 16 trees) gives
    bit-for-bit the metadata, key intervals and plan of the separate calls
    (tt_meta_build + tt_keys_build + tt_plan_build): 21 trees (two batches),
    the 16K tree's hybrid partitions with their gateway biases, a bias with a
    bad value (status bit), and a 70K-token tree beyond the batched limit."""
    from tree_training_amd._lib import TT_STATUS_BAD_BIAS
    from tree_training_amd.hybrid import hybrid_plan
    from tree_training_amd.meta import KeyPlan, TreeMetaDevice, build_trees
    from tree_training_amd.tree import TreeNode
    specs = [(*workloads.random_forest(s, node_len=(1, 200)), 0, None) for s in range(12)]
    roots, _ = workloads.forest_from_topology(workloads.agent_tree(0), TreeNode)
    for pl in hybrid_plan(roots, 4096):
        specs.append((pl["node_len"], pl["parent"], pl["pos_offset"],
                      None if pl["bias"] is None else pl["bias"].to(DEV)))
    bad = torch.zeros(40)
    bad[3] = 1.0
    specs.append(([30, 20], [-1, 0], 7, bad))
    specs.append(([70000], [-1], 0, None))
    say(f"build_trees: {len(specs)} trees")
    built = build_trees(specs, DEV)
    for i, ((nl, pa, po, pb), (meta, plan)) in enumerate(zip(specs, built)):
        m2 = TreeMetaDevice(nl, pa, pos_offset=po, device=DEV)
        p2 = KeyPlan(m2.horizon, pb)
        for f in ("node_start", "node_off", "node_hend", "pos", "node_of", "horizon"):
            assert torch.equal(getattr(meta, f), getattr(m2, f)), (i, f)
        assert torch.equal(plan.key_lo, p2.key_lo) and torch.equal(plan.key_hi, p2.key_hi), i
        n_q, n_keys = plan.n_q, plan.n_keys
        a = _plan_decode(plan.plan.cpu().numpy().tobytes(), n_q, n_keys)
        b = _plan_decode(p2.plan.cpu().numpy().tobytes(), n_q, n_keys)
        for k in ("P", "n_qb", "n_kt", "n_kb", "n_items", "n_split", "item_order", "rows", "row_order",
                  "kb_order"):
            assert a[k] == b[k], (i, k)
        for k in ("qlo", "qhi", "kb_base", "kb_srank", "kb_item"):
            assert np.array_equal(a[k], b[k]), (i, k)
        st = int(meta.status.item())
        want = int(m2.status.item()) | int(p2.status.item())
        assert st == want, (i, st, want)
        assert (st == TT_STATUS_BAD_BIAS) == (i == len(specs) - 2), (i, st)


@pytest.mark.parametrize("case", ["forest", "agent16k", "gateway", "rollout48k", "rollout270k"])
def test_plan_matches_numpy(case):
    """Every field of the device tile plan equals the numpy restatement
    (bit-exact: it is index work). Up to 2048 query blocks and key tiles the
    plan's last passes run as one workgroup; the 270K-token rollout (2112 of
    each, and more than 65536 tokens for the metadata) takes the multi-launch
    paths. The dK/dV work items are sorted by length, then query window, up
    to 4096 of them (the 270K tree's are listed window-major)."""
    from tree_training_amd.meta import KeyPlan
    bias = None
    if case == "forest":
        lens, par = workloads.random_forest(4, node_len=(1, 300))
    elif case == "agent16k":
        lens, par = workloads.agent_tree(0)
    elif case == "rollout270k":
        lens, par = [8192] + [1024] * 256, [-1] + [0] * 256
    elif case == "rollout48k":
        lens, par = workloads.rollout_tree(0)
    else:
        lens, par = [700, 500, 300], [-1, 0, 0]
        vis = np.random.default_rng(3).random(1300) < 0.7
        bias = torch.tensor(np.where(vis, 0.0, -np.inf), dtype=torch.float32, device=DEV)
    say(f"plan case={case} T={sum(lens)}")
    m = _meta(lens, par)
    plan = KeyPlan(m.horizon, bias, validate=True)
    n_q, n_keys = plan.n_q, plan.n_keys
    got = _plan_decode(plan.plan.cpu().numpy().tobytes(), n_q, n_keys)
    lo, hi = plan.key_lo.cpu().numpy(), plan.key_hi.cpu().numpy()
    exp = _plan_expected_fast(lo, hi, n_q)
    if n_q < 20000:   # the vectorised restatement against the per-pair loop
        ref = _plan_expected(lo, hi, n_q)
        for k in ("P", "rows", "row_order", "kb_order"):
            assert exp[k] == ref[k], k
        for k in ("qlo", "qhi", "kb_base"):
            assert np.array_equal(exp[k], ref[k]), k
    if case == "rollout270k":
        ref = meta_closed_form(lens, par)
        assert np.array_equal(m.pos.cpu().numpy(), ref["pos"])
        assert np.array_equal(m.horizon.cpu().numpy(), ref["horizon"])
        assert exp["n_qb"] > 2048 and exp["n_kb"] > 2048 and n_q > 65536
    for k in ("P", "n_qb", "n_kt", "n_kb", "n_split", "item_order", "rows", "row_order", "kb_order"):
        assert got[k] == exp[k], k
    for k in ("qlo", "qhi", "kb_base", "kb_srank", "kb_item"):
        assert np.array_equal(got[k], exp[k]), k
    assert got["n_items"] == exp["kb_base"][-1]
    assert exp["item_order"] == (2 if case == "rollout270k" else 1)
    if bias is None:   # the host count (tt_attn_split_tiles) is the plan's
        assert KeyPlan(m.horizon, topo=(lens, par)).split_tiles() == max(exp["n_split"], 1)


# --------------------------------------------------------------------------- attention
def _qkv(T, Lp, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    # transformers layout: [1, H, T, D] views of token-major storage
    q = torch.randn(1, T, HQ, D, generator=g).to(dtype)
    k = torch.randn(1, T, HKV, D, generator=g).to(dtype)
    v = torch.randn(1, T, HKV, D, generator=g).to(dtype)
    do = torch.randn(1, T, HQ, D, generator=g).to(dtype)
    kp = torch.randn(1, Lp, HKV, D, generator=g).to(dtype) if Lp else None
    vp = torch.randn(1, Lp, HKV, D, generator=g).to(dtype) if Lp else None
    return q, k, v, do, kp, vp


def _run(lens, par, dtype, seed=0, past_vis=None, parts=(0,), deterministic=None):
    from tree_training_amd.attention import attn_backward, attn_forward
    from tree_training_amd.meta import KeyPlan
    T = sum(lens)
    Lp = 0 if past_vis is None else len(past_vis)
    q, k, v, do, kp, vp = _qkv(T, Lp, dtype, seed)
    m = _meta(lens, par)
    bias = None
    if Lp:
        bias = torch.tensor([0.0 if b else -math.inf for b in past_vis], device=DEV)
    plan = KeyPlan(m.horizon, bias, validate=True)
    tr = lambda x: None if x is None else x.to(DEV).transpose(1, 2)
    scale = D ** -0.5
    acc = None
    if Lp:
        acc = (torch.zeros(Lp, HKV, D, device=DEV), torch.zeros(Lp, HKV, D, device=DEV))
    o, lse = attn_forward(tr(q), tr(k), tr(v), plan, scale, tr(kp), tr(vp))
    dq, dk, dv = attn_backward(tr(q), tr(k), tr(v), plan, scale, o, lse, do.to(DEV), tr(kp), tr(vp), acc,
                               parts=parts, deterministic=deterministic)
    torch.cuda.synchronize()
    # oracle on the same (rounded) inputs, fp64
    cf = meta_closed_form(lens, par)
    lo = ([0] * Lp) + list(range(T))
    hi = ([T if b else 0 for b in (past_vis or [])]) + list(cf["horizon"])
    mask = key_interval_mask(lo, hi, T)
    f64 = lambda x: x[0].double().numpy()
    kk = f64(k) if not Lp else np.concatenate([f64(kp), f64(k)], axis=0)
    vv = f64(v) if not Lp else np.concatenate([f64(vp), f64(v)], axis=0)
    ro, rlse = attn_fwd(f64(q), kk, vv, mask, scale)
    rdq, rdk, rdv = attn_bwd(f64(q), kk, vv, mask, scale, f64(do))
    out = dict(o=(ro, o.float().cpu().numpy()), lse=(rlse, lse.cpu().numpy()),
               dq=(rdq, dq.float().cpu().numpy()), dk=(rdk[Lp:], dk.float().cpu().numpy()),
               dv=(rdv[Lp:], dv.float().cpu().numpy()))
    if Lp:
        out["dk_past"] = (rdk[:Lp], acc[0].cpu().numpy())
        out["dv_past"] = (rdv[:Lp], acc[1].cpu().numpy())
    return out


TOL = {torch.bfloat16: 2e-2, torch.float32: 1e-5}


def check_close(name, ref, got, tol):
    """max_rel (verify_hybrid.py:129-132) against the tolerance; a reference
    that is exactly zero up to rounding (e.g. dQ of a query with one visible
    key) is compared in absolute terms instead."""
    if np.abs(ref).max() < 1e-9:
        assert np.abs(got).max() < tol, f"{name}: |got| {np.abs(got).max():.3e} for a zero reference"
        return
    r = max_rel(ref, got)
    assert r < tol, f"{name}: max_rel {r:.3e} >= {tol}"

CASES = {
    "c1": ([3, 4, 3, 4, 5, 3, 3, 4, 4, 3, 4, 3, 4], [-1, 0, 1, 2, 3, 3, 2, 6, -1, 8, 9, 8, 11]),
    "single_token": ([1], [-1]),
    "chain_ragged": ([37, 100, 5, 211], [-1, 0, 1, 2]),
    "wide": ([130] + [67] * 9, [-1] + [0] * 9),
    "forest7": workloads.random_forest(7, node_len=(1, 90)),
    "agent_small": workloads.agent_tree(3, max_tokens=1500),
    # key tiles whose visible query range exceeds one dK/dV work item (split + fp32 sums)
    "long_prompt": ([4400, 300, 250, 410], [-1, 0, 0, 0]),
}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("case", list(CASES))
def test_attention_parity(case, dtype):
    lens, par = CASES[case]
    say(f"attention parity case={case} dtype={dtype} T={sum(lens)}")
    res = _run(lens, par, dtype, seed=sum(map(ord, case)))
    tol = TOL[dtype]
    for name, (ref, got) in res.items():
        if name == "lse":
            assert np.abs(ref - got).max() < (2e-2 if dtype == torch.bfloat16 else 1e-5), name
            continue
        check_close(name, ref, got, tol)


@pytest.mark.parametrize("seed", range(16))
def test_attention_random_forests(seed):
    """Seeded random cases against the fp64 oracle: irregular forests (1-3
    roots, depth up to 6, node lengths up to a drawn maximum, at most 2,500
    tokens), half of them under a gateway of up to 600 keys with a drawn
    visible share, either dtype, the backward in one call or in parts, with
    and without TT_BWD_DETERMINISTIC."""
    rng = np.random.default_rng(1000 + seed)
    while True:
        lens, par = workloads.random_forest(int(rng.integers(0, 10**6)), n_roots=(1, int(rng.integers(1, 4))),
                                            max_depth=int(rng.integers(1, 7)), max_branch=int(rng.integers(1, 5)),
                                            node_len=(1, int(rng.integers(2, 400))))
        if sum(lens) <= 2500:
            break
    dtype = torch.bfloat16 if rng.random() < 0.6 else torch.float32
    Lp = int(rng.integers(1, 600)) if rng.random() < 0.5 else 0
    past_vis = [bool(x) for x in (rng.random(Lp) < rng.random())] if Lp else None
    det = bool(rng.random() < 0.3)
    parts = [(0,), (3, 4), (1, 2, 4)][int(rng.integers(0, 3))]
    say(f"attention random forest seed={seed}: T={sum(lens)} nodes={len(lens)} Lp={Lp} dtype={dtype} det={det} "
        f"parts={parts}")
    res = _run(lens, par, dtype, seed=seed, past_vis=past_vis, parts=parts, deterministic=det)
    for name, (ref, got) in res.items():
        if name != "lse":
            check_close(name, ref, got, TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("shape", ["short", "split"])
def test_attention_gateway(dtype, shape):
    # "split": the gateway keys are seen by more queries than one dK/dV work item covers
    lens, par, n_past = {"short": ([40, 70, 33], [-1, 0, 0], 150),
                         "split": ([2400, 1500, 1400], [-1, 0, 0], 300)}[shape]
    rng = np.random.default_rng(5)
    past_vis = [bool(x) for x in (rng.random(n_past) < 0.6)]
    say(f"attention gateway dtype={dtype} Lp={len(past_vis)}")
    res = _run(lens, par, dtype, seed=11, past_vis=past_vis)
    tol = TOL[dtype]
    for name, (ref, got) in res.items():
        if name == "lse":
            continue
        check_close(name, ref, got, tol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("parts", [(1, 2, 4), (3, 4), (1, 6)], ids=["delta,dq,dkdv", "delta+dq,dkdv", "delta,dq+dkdv"])
def test_attention_backward_parts(parts, dtype):
    """The backward run as separate tt_attn_bwd calls (bwd_parts in order):
    delta by its own kernel or fused into the dQ pass, with a gateway whose
    keys split into several dK/dV work items; against the fp64 oracle."""
    lens, par, n_past = [2400, 1500, 1400], [-1, 0, 0], 300
    rng = np.random.default_rng(6)
    past_vis = [bool(x) for x in (rng.random(n_past) < 0.6)]
    say(f"attention backward parts={parts} dtype={dtype}")
    res = _run(lens, par, dtype, seed=12, past_vis=past_vis, parts=parts)
    tol = TOL[dtype]
    for name, (ref, got) in res.items():
        if name == "lse":
            continue
        check_close(name, ref, got, tol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("case", ["long_prompt", "gateway_split", "gateway_split_parts"])
def test_attention_deterministic(case, dtype):
    """TT_BWD_DETERMINISTIC, both dtypes: keys whose query range is split over
    several dK/dV work items (own keys of the long prompt; gateway keys seen
    by every query, added into the fp32 gateway sums) sum their partials in
    work-item order, so two backwards of the same inputs are bitwise equal,
    and both match the fp64 oracle (< 2e-2 bf16, < 1e-5 fp32)."""
    past_vis, parts = None, (0,)
    if case == "long_prompt":
        lens, par = CASES["long_prompt"]
    else:
        lens, par = [2400, 1500, 1400], [-1, 0, 0]
        past_vis = [bool(x) for x in (np.random.default_rng(8).random(300) < 0.6)]
        if case == "gateway_split_parts":
            parts = (3, 4)
    say(f"attention deterministic case={case} dtype={dtype} T={sum(lens)}")
    runs = [_run(lens, par, dtype, seed=21, past_vis=past_vis, parts=parts, deterministic=True)
            for _ in range(2)]
    for name, (ref, got) in runs[0].items():
        assert np.array_equal(got, runs[1][name][1]), f"{name}: two deterministic runs differ"
        if name != "lse":
            check_close(name, ref, got, TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("hq,hkv", [(16, 16), (32, 4), (12, 4), (2, 1)])
def test_attention_head_layouts(hq, hkv, dtype):
    """Other GQA layouts than Qwen3-4B's 32/8: MHA (16/16), 8 q heads per kv
    head (32/4), a q-head count that is not a multiple of 8 (12/4: the
    workgroup -> head mapping without the per-XCD grouping) and a single kv
    head (2/1), with a gateway prefix, against the fp64 oracle."""
    from tree_training_amd.attention import attn_backward, attn_forward
    from tree_training_amd.meta import KeyPlan
    lens, par = workloads.random_forest(21, node_len=(1, 70))
    T, Lp = sum(lens), 45
    say(f"attention head layout hq={hq} hkv={hkv} dtype={dtype} T={T}")
    g = torch.Generator().manual_seed(hq * 100 + hkv)
    q = torch.randn(1, T, hq, D, generator=g).to(dtype)
    k = torch.randn(1, T, hkv, D, generator=g).to(dtype)
    v = torch.randn(1, T, hkv, D, generator=g).to(dtype)
    do = torch.randn(1, T, hq, D, generator=g).to(dtype)
    kp = torch.randn(1, Lp, hkv, D, generator=g).to(dtype)
    vp = torch.randn(1, Lp, hkv, D, generator=g).to(dtype)
    vis = [(i % 4) != 2 for i in range(Lp)]
    bias = torch.tensor([0.0 if b else -math.inf for b in vis], device=DEV)
    m = _meta(lens, par)
    plan = KeyPlan(m.horizon, bias, validate=True)
    tr = lambda x: x.to(DEV).transpose(1, 2)
    acc = (torch.zeros(Lp, hkv, D, device=DEV), torch.zeros(Lp, hkv, D, device=DEV))
    scale = D ** -0.5
    o, lse = attn_forward(tr(q), tr(k), tr(v), plan, scale, tr(kp), tr(vp))
    dq, dk, dv = attn_backward(tr(q), tr(k), tr(v), plan, scale, o, lse, do.to(DEV), tr(kp), tr(vp), acc)
    torch.cuda.synchronize()
    cf = meta_closed_form(lens, par)
    mask = key_interval_mask([0] * Lp + list(range(T)), [T if b else 0 for b in vis] + list(cf["horizon"]), T)
    f64 = lambda x: x[0].double().numpy()
    kk = np.concatenate([f64(kp), f64(k)], axis=0)
    vv = np.concatenate([f64(vp), f64(v)], axis=0)
    ro, _ = attn_fwd(f64(q), kk, vv, mask, scale)
    rdq, rdk, rdv = attn_bwd(f64(q), kk, vv, mask, scale, f64(do))
    tol = TOL[dtype]
    for name, ref, got in (("o", ro, o), ("dq", rdq, dq), ("dk", rdk[Lp:], dk), ("dv", rdv[Lp:], dv),
                           ("dk_past", rdk[:Lp], acc[0]), ("dv_past", rdv[:Lp], acc[1])):
        check_close(name, ref, got.float().cpu().numpy(), tol)


@pytest.mark.parametrize("parts", [(0,), (3, 4)], ids=["one_call", "delta+dq,dkdv"])
def test_attention_key_split_gateway_partition(parts):
    """A gateway partition with few queries (473 tokens in two nodes, 4 query
    blocks x 32 heads = 128 pairs) under 3,760 gateway keys of which two runs
    are visible: the bf16 forward and dQ passes split each pair's keys four
    ways and merge the fp32 partials (tt_attn_fwd_workspace_bytes > 0). The
    result matches the fp64 oracle, and two runs are bitwise equal (the
    merge adds the ranges in a fixed order)."""
    from tree_training_amd import _lib
    from tree_training_amd.attention import _Problem
    from tree_training_amd.meta import KeyPlan
    lens, par, n_past = [300, 173], [-1, 0], 3760
    past_vis = [i < 1357 or i >= 3648 for i in range(n_past)]
    T = sum(lens)
    m = _meta(lens, par)
    plan = KeyPlan(m.horizon, torch.tensor([0.0 if b else -math.inf for b in past_vis], device=DEV))
    x = torch.zeros(1, HQ, T, D, dtype=torch.bfloat16, device=DEV)
    kv = torch.zeros(1, HKV, T, D, dtype=torch.bfloat16, device=DEV)
    kvp = torch.zeros(1, HKV, n_past, D, dtype=torch.bfloat16, device=DEV)
    pb = _Problem(x, kv, kv, kvp, kvp, plan, D ** -0.5)
    assert _lib.lib().tt_attn_fwd_workspace_bytes(ctypes.byref(pb.s)) > 0
    say(f"attention key split gateway partition T={T} Lp={n_past} parts={parts}")
    runs = [_run(lens, par, torch.bfloat16, seed=31, past_vis=past_vis, parts=parts) for _ in range(2)]
    for name, (ref, got) in runs[0].items():
        if name in ("o", "lse", "dq"):
            assert np.array_equal(got, runs[1][name][1]), f"{name}: two runs differ"
        if name == "lse":
            assert np.abs(ref - got).max() < 2e-2, name
            continue
        check_close(name, ref, got, TOL[torch.bfloat16])
