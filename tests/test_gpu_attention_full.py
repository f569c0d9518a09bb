"""Full-size parity of the bf16 tree attention (the 16K agent tree and the 48K
rollout tree, 32 q / 8 kv heads, d 128), through size-independent properties.

A DFS-packed tree attention restricted to one root-to-leaf path is plain
causal attention over that path's tokens. So for sampled leaves:
  * the tree forward's outputs and log-sum-exps on the path's tokens equal
    causal GQA attention over the path (torch, float32, on the same
    bf16-rounded inputs);
  * with dO non-zero only on the path, the tree backward's dq, dk, dv on the
    path equal that attention's gradients, and every other token's dq, dk, dv
    is exactly zero (no other query carries a gradient, and no other key is
    seen by a path query).
With a full dO (every token), the whole 16K tree's outputs and gradients equal
a float64 dense-mask attention (the reference's additive mask, from the
oracle's closed form j <= i < h[j], one q head at a time on the GPU).
And the 16K tree cut into tree_grad_hybrid's 4096-token partitions, each
attending to its gateway prefix, gives the whole tree's outputs and gradients
(gateway gradients accumulated in fp32 and scattered back to their tokens).
Bars: max_rel (max |error| over max |reference|) < 2e-2 for bf16, 1e-5 for
fp32, for o, dq, dk, dv; |lse error| < 2e-2 (bf16), 1e-4
(fp32, natural-log units of values near 8).
"""
import numpy as np
import pytest
import torch

from tree_training_amd import workloads

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
HQ, HKV, D = 32, 8, 128
REP = HQ // HKV


def _path_tokens(lens, par, leaf):
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]])
    path, j = [], leaf
    while j >= 0:
        path.append(j)
        j = par[j]
    return np.concatenate([np.arange(starts[i], starts[i] + lens[i]) for i in path[::-1]])


def _causal_reference(q, k, v, do, scale):
    """Causal GQA attention over one sequence and its gradients, float32:
    q, do [L, HQ, D]; k, v [L, HKV, D]. Returns o, lse [HQ, L], dq, dk, dv."""
    L = q.shape[0]
    causal = torch.ones(L, L, dtype=torch.bool, device=q.device).tril()
    o = torch.empty_like(q)
    lse = torch.empty(HQ, L, device=q.device)
    dq = torch.empty_like(q)
    dk = torch.zeros_like(k)
    dv = torch.zeros_like(v)
    for h in range(HQ):
        g = h // REP
        qh, kh, vh, doh = (q[:, h].contiguous(), k[:, g].contiguous(), v[:, g].contiguous(),
                           do[:, h].contiguous())
        s = (qh @ kh.t().contiguous()) * scale
        s = s.masked_fill(~causal, float("-inf"))
        m = s.max(dim=1, keepdim=True).values
        e = torch.exp(s - m)
        z = e.sum(dim=1, keepdim=True)
        p = e / z
        oh = p @ vh
        o[:, h] = oh
        lse[h] = (m + torch.log(z))[:, 0]
        dp = doh @ vh.t().contiguous()
        ds = p * (dp - (doh * oh).sum(dim=1, keepdim=True))
        dq[:, h] = (ds @ kh) * scale
        dk[:, g] += (ds.t().contiguous() @ qh) * scale
        dv[:, g] += p.t().contiguous() @ doh
    return o, lse, dq, dk, dv


def _max_rel(ref, got):
    return float((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30))


@pytest.mark.parametrize("workload,n_paths,dt", [("agent16k", 3, "bf16"), ("rollout48k", 2, "bf16"),
                                                 ("agent16k", 3, "fp32"), ("rollout48k", 2, "fp32")])
def test_attention_full_size_per_path(workload, n_paths, dt):
    from tree_training_amd.attention import attn_backward, attn_forward
    from tree_training_amd.meta import KeyPlan, TreeMetaDevice
    lens, par = workloads.agent_tree(0) if workload == "agent16k" else workloads.rollout_tree(0)
    T = sum(lens)
    g = torch.Generator(device=DEV).manual_seed(3)
    bf = torch.bfloat16 if dt == "bf16" else torch.float32
    bar = 2e-2 if dt == "bf16" else 1e-5
    q = torch.randn(T, HQ, D, device=DEV, generator=g, dtype=bf)
    k = torch.randn(T, HKV, D, device=DEV, generator=g, dtype=bf)
    v = torch.randn(T, HKV, D, device=DEV, generator=g, dtype=bf)
    scale = D ** -0.5
    meta = TreeMetaDevice(lens, par, device=DEV)
    plan = KeyPlan(meta.horizon, None)
    view = lambda x: x[None].transpose(1, 2)   # [1, H, T, D] views of token-major storage
    o, lse = attn_forward(view(q), view(k), view(v), plan, scale)
    leaves = [i for i in range(len(lens)) if i not in set(par)]
    rng = np.random.default_rng(7)
    for leaf in rng.choice(leaves, size=n_paths, replace=False):
        idx = _path_tokens(lens, par, int(leaf))
        print(f"{workload}: leaf {leaf}, path of {len(idx)} tokens", flush=True)
        ti = torch.from_numpy(idx).to(DEV)
        do = torch.zeros(T, HQ, D, device=DEV, dtype=bf)
        do[ti] = torch.randn(len(idx), HQ, D, device=DEV, generator=g, dtype=bf)
        dq, dk, dv = attn_backward(view(q), view(k), view(v), plan, scale, o, lse, do[None])
        ro, rlse, rdq, rdk, rdv = _causal_reference(q[ti].float(), k[ti].float(), v[ti].float(),
                                                    do[ti].float(), scale)
        torch.cuda.synchronize()
        r = _max_rel(ro, o[ti].float())
        print(f"  o max_rel {r:.2e}", flush=True)
        assert r < bar
        assert float((lse[:, ti] - rlse).abs().max()) < (2e-2 if dt == "bf16" else 1e-4)
        for name, ref, got in (("dq", rdq, dq), ("dk", rdk, dk), ("dv", rdv, dv)):
            gf = got.float()
            assert torch.isfinite(gf).all(), name
            r = _max_rel(ref, gf[ti])
            print(f"  {name} max_rel {r:.2e}", flush=True)
            assert r < bar, (workload, int(leaf), name, r)
            off = torch.ones(T, dtype=torch.bool, device=DEV)
            off[ti] = False
            assert not gf[off].any(), (workload, int(leaf), name, "non-zero off the path")


def _dense_tree_reference(q, k, v, do, horizon, scale):
    """Float64 attention over the packed tree with the dense visibility mask
    (query i sees key j iff j <= i < horizon[j]) and its gradients, one q head
    at a time: q, do [T, HQ, D]; k, v [T, HKV, D]. Returns o, lse, dq, dk, dv."""
    T = q.shape[0]
    idx = torch.arange(T, device=q.device)
    hz = torch.as_tensor(horizon, device=q.device)
    visible = (idx[None, :] <= idx[:, None]) & (idx[:, None] < hz[None, :])   # [query, key]
    f64 = torch.float64
    o = torch.empty(T, HQ, D, dtype=f64, device=q.device)
    lse = torch.empty(HQ, T, dtype=f64, device=q.device)
    dq = torch.empty(T, HQ, D, dtype=f64, device=q.device)
    dk = torch.zeros(T, HKV, D, dtype=f64, device=q.device)
    dv = torch.zeros(T, HKV, D, dtype=f64, device=q.device)
    for h in range(HQ):
        g = h // REP
        qh, kh, vh, doh = (q[:, h].to(f64).contiguous(), k[:, g].to(f64).contiguous(),
                           v[:, g].to(f64).contiguous(), do[:, h].to(f64).contiguous())
        p = (qh @ kh.t().contiguous()) * scale
        p.masked_fill_(~visible, float("-inf"))
        m = p.amax(dim=1, keepdim=True)
        p.sub_(m).exp_()
        z = p.sum(dim=1, keepdim=True)
        p.div_(z)
        oh = p @ vh
        o[:, h] = oh
        lse[h] = (m + torch.log(z))[:, 0]
        ds = doh @ vh.t().contiguous()
        ds.sub_((doh * oh).sum(dim=1, keepdim=True)).mul_(p)
        dq[:, h] = (ds @ kh) * scale
        dk[:, g] += (ds.t().contiguous() @ qh) * scale
        dv[:, g] += p.t().contiguous() @ doh
        del p, ds
    return o, lse, dq, dk, dv


@pytest.mark.parametrize("dt", ["bf16", "fp32"])
def test_attention_full_size_full_do_dense_reference(dt):
    """The 16K agent tree (16,318 tokens, 32 q / 8 kv heads) with dO on every
    token: o, lse, dq, dk, dv of the tree kernels against the float64 dense-mask
    reference on the same (rounded) inputs. Shared-prefix keys (the root's are
    seen by every query) sum their dK/dV over many work items here, which the
    per-path tests (dO on one path) never exercise. Bars: max_rel < 2e-2
    (bf16), 1e-5 (fp32); |lse error| < 2e-2 (bf16), 1e-4 (fp32)."""
    from oracle.tree_meta import meta_closed_form
    from tree_training_amd.attention import attn_backward, attn_forward
    from tree_training_amd.meta import KeyPlan, TreeMetaDevice
    lens, par = workloads.agent_tree(0)
    T = sum(lens)
    g = torch.Generator(device=DEV).manual_seed(11)
    bf = torch.bfloat16 if dt == "bf16" else torch.float32
    bar = 2e-2 if dt == "bf16" else 1e-5
    q = torch.randn(T, HQ, D, device=DEV, generator=g, dtype=bf)
    k = torch.randn(T, HKV, D, device=DEV, generator=g, dtype=bf)
    v = torch.randn(T, HKV, D, device=DEV, generator=g, dtype=bf)
    do = torch.randn(T, HQ, D, device=DEV, generator=g, dtype=bf)
    scale = D ** -0.5
    view = lambda x: x[None].transpose(1, 2)
    plan = KeyPlan(TreeMetaDevice(lens, par, device=DEV).horizon, None)
    o, lse = attn_forward(view(q), view(k), view(v), plan, scale)
    dq, dk, dv = attn_backward(view(q), view(k), view(v), plan, scale, o, lse, do[None])
    print(f"agent16k {dt}: full-dO backward done, dense float64 reference", flush=True)
    ro, rlse, rdq, rdk, rdv = _dense_tree_reference(q, k, v, do, meta_closed_form(lens, par)["horizon"], scale)
    torch.cuda.synchronize()
    lerr = float((lse.double() - rlse).abs().max())
    print(f"  lse max abs err {lerr:.2e}", flush=True)
    assert lerr < (2e-2 if dt == "bf16" else 1e-4)
    for name, ref, got in (("o", ro, o), ("dq", rdq, dq), ("dk", rdk, dk), ("dv", rdv, dv)):
        gf = got.double()
        assert torch.isfinite(gf).all(), name
        r = float((gf - ref).abs().max() / ref.abs().max())
        print(f"  {name} max_rel {r:.2e}", flush=True)
        assert r < bar, (dt, name, r)


def test_attention_gateway_partitions_full_size():
    """The 16K agent tree split with max_tokens=4096 (tree_grad_hybrid's
    partitions; each child partition attends to its gateway: the parent's
    gateway plus the parent's tokens up to the cut node, with the inherited
    ancestor-aware bias) gives the whole tree's attention: per partition, o and
    dq on its tokens equal the whole-tree run's, and each token's dk, dv —
    its own partition's plus what every descendant partition accumulated into
    its gateway entry (fp32) — equal the whole-tree run's."""
    from tree_training_amd.attention import attn_backward, attn_forward
    from tree_training_amd.hybrid import _flatten_partition, hybrid_plan, partition_tree
    from tree_training_amd.meta import KeyPlan, TreeMetaDevice
    from tree_training_amd.tree import TreeNode
    topo = workloads.agent_tree(0)
    lens, par = topo
    T = sum(lens)
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]])
    roots, nodes = workloads.forest_from_topology(topo, TreeNode)
    gidx = {id(n): i for i, n in enumerate(nodes)}
    parts = partition_tree(roots, 4096)
    plans = hybrid_plan(roots, 4096, pack_siblings=False)
    assert len(parts) == len(plans) > 1
    g = torch.Generator(device=DEV).manual_seed(5)
    bf = torch.bfloat16
    q = torch.randn(T, HQ, D, device=DEV, generator=g, dtype=bf)
    k = torch.randn(T, HKV, D, device=DEV, generator=g, dtype=bf)
    v = torch.randn(T, HKV, D, device=DEV, generator=g, dtype=bf)
    do = torch.randn(T, HQ, D, device=DEV, generator=g, dtype=bf)
    scale = D ** -0.5
    view = lambda x: x[None].transpose(1, 2)
    plan = KeyPlan(TreeMetaDevice(lens, par, device=DEV).horizon, None)
    o, lse = attn_forward(view(q), view(k), view(v), plan, scale)
    dq, dk, dv = attn_backward(view(q), view(k), view(v), plan, scale, o, lse, do[None])

    own_tokens, prefix_tokens = {}, {}
    sum_dk = torch.zeros(T, HKV, D, device=DEV)
    sum_dv = torch.zeros(T, HKV, D, device=DEV)
    for p, pl in zip(parts, plans):
        node_len, parent, pnodes = _flatten_partition(p)
        assert node_len == pl["node_len"] and parent == pl["parent"]
        tok = np.concatenate([np.arange(starts[gidx[id(n)]], starts[gidx[id(n)]] + len(n.token_ids))
                              for n in pnodes])
        own_tokens[id(p)] = tok
        if p.parent is None:
            pre = np.zeros(0, np.int64)
        else:
            pp = p.parent
            pn = _flatten_partition(pp)[2]
            cut_pos = [i for i, n in enumerate(pn) if n is p.parent_cut_node][0]
            # the gateway ends with the cut node's own tokens (its end in the parent's DFS order)
            cut_end = int(sum(len(n.token_ids) for n in pn[:cut_pos + 1]))
            pre = np.concatenate([prefix_tokens[id(pp)], own_tokens[id(pp)][:cut_end]])
        prefix_tokens[id(p)] = pre
        assert len(pre) == pl["past_len"]
        ti = torch.from_numpy(tok).to(DEV)
        kp = vp = bias = acc = None
        if len(pre):
            tp = torch.from_numpy(pre).to(DEV)
            kp, vp = view(k[tp].contiguous()), view(v[tp].contiguous())
            bias = pl["bias"].to(DEV)
            acc = (torch.zeros(len(pre), HKV, D, device=DEV), torch.zeros(len(pre), HKV, D, device=DEV))
        pplan = KeyPlan(TreeMetaDevice(node_len, parent, device=DEV).horizon, bias)
        qi, ki, vi = view(q[ti].contiguous()), view(k[ti].contiguous()), view(v[ti].contiguous())
        po, plse = attn_forward(qi, ki, vi, pplan, scale, kp, vp)
        pdq, pdk, pdv = attn_backward(qi, ki, vi, pplan, scale, po, plse, do[ti][None].contiguous(), kp, vp, acc)
        print(f"partition: {len(tok)} tokens, gateway {len(pre)}", flush=True)
        assert _max_rel(o[ti].float(), po.float()) < 2e-2
        assert _max_rel(dq[ti].float(), pdq.float()) < 2e-2
        sum_dk.index_add_(0, ti, pdk.float())
        sum_dv.index_add_(0, ti, pdv.float())
        if acc is not None:
            sum_dk.index_add_(0, tp, acc[0])
            sum_dv.index_add_(0, tp, acc[1])
    assert sorted(np.concatenate(list(own_tokens.values())).tolist()) == list(range(T))
    torch.cuda.synchronize()
    assert _max_rel(dk.float(), sum_dk) < 2e-2
    assert _max_rel(dv.float(), sum_dv) < 2e-2


@pytest.mark.parametrize("workload,dt", [("agent16k", "bf16"), ("agent16k", "fp32"), ("rollout48k", "bf16")])
def test_attention_deterministic_full_size(workload, dt):
    """With TT_BWD_DETERMINISTIC and the workspace sized from the tree
    (tt_attn_det_slots), two backwards are bitwise equal (dq, dk, dv and the
    fp32 gateway sums), and they agree with the default (atomic) backward to
    rounding (max_rel < 1e-2 bf16, < 1e-5 fp32). agent16k runs under a
    4096-key gateway that every query sees (its tiles and the root's split
    into several dK/dV work items); rollout48k is the 48K tree, whose 8192
    prompt keys are seen by all 49,152 queries."""
    from tree_training_amd.attention import attn_backward, attn_forward
    from tree_training_amd.meta import KeyPlan, TreeMetaDevice
    lens, par = workloads.agent_tree(0) if workload == "agent16k" else workloads.rollout_tree(0)
    T, Lp = sum(lens), (4096 if workload == "agent16k" else 0)
    g = torch.Generator(device=DEV).manual_seed(9)
    bf = torch.bfloat16 if dt == "bf16" else torch.float32
    q = torch.randn(T, HQ, D, device=DEV, generator=g, dtype=bf)
    k = torch.randn(T, HKV, D, device=DEV, generator=g, dtype=bf)
    v = torch.randn(T, HKV, D, device=DEV, generator=g, dtype=bf)
    kp = vp = None
    if Lp:
        kp = torch.randn(Lp, HKV, D, device=DEV, generator=g, dtype=bf)
        vp = torch.randn(Lp, HKV, D, device=DEV, generator=g, dtype=bf)
    do = torch.randn(T, HQ, D, device=DEV, generator=g, dtype=bf)
    scale = D ** -0.5
    view = lambda x: None if x is None else x[None].transpose(1, 2)
    plan = KeyPlan(TreeMetaDevice(lens, par, device=DEV).horizon, torch.zeros(Lp, device=DEV) if Lp else None,
                   topo=(lens, par))
    assert plan.det_slots() == _plan_extra_items(plan) > 0
    o, lse = attn_forward(view(q), view(k), view(v), plan, scale, view(kp), view(vp))
    outs = []
    for det in (True, True, False):
        acc = (torch.zeros(Lp, HKV, D, device=DEV), torch.zeros(Lp, HKV, D, device=DEV)) if Lp else None
        dq, dk, dv = attn_backward(view(q), view(k), view(v), plan, scale, o, lse, do[None], view(kp), view(vp),
                                   acc, deterministic=det)
        outs.append((dq, dk, dv) + (tuple(acc) if acc else ()))
        print(f"{workload} + gateway {Lp} {dt}: backward deterministic={det} done", flush=True)
    torch.cuda.synchronize()
    names = ("dq", "dk", "dv", "dk_past", "dv_past")
    for name, a, b, c in zip(names, *outs):
        assert torch.equal(a, b), f"{name}: two deterministic runs differ"
        assert torch.isfinite(a.float()).all(), name
        assert _max_rel(c.float(), a.float()) < (1e-2 if dt == "bf16" else 1e-5), name


def _plan_extra_items(plan):
    """dK/dV work items beyond the first of each key tile, read back from the
    device plan (header: int32 n_kb at byte 16, n_items at byte 20)."""
    hdr = plan.plan[:24].view(torch.int32).cpu()
    return int(hdr[5]) - int(hdr[4])


def test_attention_deterministic_workspace_from_tree():
    """tt_attn_det_slots (host arithmetic on the topology) equals the extra
    work items of the device-built plan on the workloads' trees, with and
    without gateways; with it the deterministic backward's workspace at the
    16K agent tree (32/8 heads, bf16) is at most 1.5x the default one, where
    the topology-free bound is about 4x."""
    from tree_training_amd._lib import TT_BWD_DETERMINISTIC, lib
    from tree_training_amd.attention import _Problem
    from tree_training_amd.meta import KeyPlan, TreeMetaDevice
    import ctypes
    cases = [("agent16k", workloads.agent_tree(0), 0), ("agent16k+gw", workloads.agent_tree(0), 4096),
             ("rollout48k", workloads.rollout_tree(0), 0), ("agent_s3", workloads.agent_tree(3), 777)]
    for name, (lens, par), Lp in cases:
        bias = None
        if Lp:
            bias = torch.zeros(Lp)
            bias[Lp // 3: Lp // 2] = float("-inf")
        plan = KeyPlan(TreeMetaDevice(lens, par, device=DEV).horizon, bias, topo=(lens, par))
        print(f"{name}: det_slots {plan.det_slots()} plan {_plan_extra_items(plan)}", flush=True)
        assert plan.det_slots() == _plan_extra_items(plan), name
    lens, par = workloads.agent_tree(0)
    T = sum(lens)
    plan = KeyPlan(TreeMetaDevice(lens, par, device=DEV).horizon, None, topo=(lens, par))
    q = torch.empty(1, HQ, T, D, device=DEV, dtype=torch.bfloat16)
    k = torch.empty(1, HKV, T, D, device=DEV, dtype=torch.bfloat16)
    pb = _Problem(q, k, k, None, None, plan, D ** -0.5)
    default = lib().tt_attn_bwd_workspace_bytes(ctypes.byref(pb.s))
    pb.s.bwd_parts = TT_BWD_DETERMINISTIC
    bound = lib().tt_attn_bwd_workspace_bytes(ctypes.byref(pb.s))
    pb.s.det_slots = plan.det_slots()
    exact = lib().tt_attn_bwd_workspace_bytes(ctypes.byref(pb.s))
    print(f"agent16k workspace: default {default} deterministic {exact} (bound {bound})", flush=True)
    assert exact <= 1.5 * default < bound


def test_attention_deterministic_undersized_slots_poison_not_overrun():
    """A det_slots below the tree's count writes nothing past the workspace:
    the tiles whose later items lack a slot get NaN dk/dv, every other key's
    gradients equal those of the exactly sized run bitwise."""
    from tree_training_amd._lib import TT_BWD_DETERMINISTIC
    from tree_training_amd.attention import attn_backward, attn_forward
    from tree_training_amd.meta import KeyPlan, TreeMetaDevice
    lens, par = [2048, 300, 900, 700], [-1, 0, 0, 2]
    T = sum(lens)
    g = torch.Generator(device=DEV).manual_seed(4)
    q = torch.randn(T, HQ, D, device=DEV, generator=g, dtype=torch.bfloat16)
    k = torch.randn(T, HKV, D, device=DEV, generator=g, dtype=torch.bfloat16)
    v = torch.randn(T, HKV, D, device=DEV, generator=g, dtype=torch.bfloat16)
    do = torch.randn(T, HQ, D, device=DEV, generator=g, dtype=torch.bfloat16)
    view = lambda x: x[None].transpose(1, 2)
    plan = KeyPlan(TreeMetaDevice(lens, par, device=DEV).horizon, None, topo=(lens, par))
    need = plan.det_slots()
    assert need >= 2
    o, lse = attn_forward(view(q), view(k), view(v), plan, D ** -0.5)
    full = attn_backward(view(q), view(k), view(v), plan, D ** -0.5, o, lse, do[None], deterministic=True)
    plan._det = need - 1
    short = attn_backward(view(q), view(k), view(v), plan, D ** -0.5, o, lse, do[None], deterministic=True)
    torch.cuda.synchronize()
    assert torch.equal(full[0], short[0])
    for a, b in zip(full[1:], short[1:]):
        bad = torch.isnan(b.float()).any(dim=2).any(dim=1)
        assert bad.any() and not bad.all()
        assert torch.equal(a[~bad], b[~bad])


def _last_split_tile(lens, par, n_q):
    """Highest-numbered 128-key tile with more than one dK/dV work item (own
    key j is seen by queries [j, subtree end of its node); numpy restatement
    of the work-item window rule)."""
    start = np.concatenate([[0], np.cumsum(lens)[:-1]])
    end = start + np.asarray(lens)
    for u in range(len(lens) - 1, 0, -1):
        if par[u] >= 0:
            end[par[u]] = max(end[par[u]], end[u])
    hi_key = np.repeat(end, lens)
    half = (1 << (n_q.bit_length() - 1)) // 2
    qch = min(max(half, 256), 4096)
    last = -1
    for kb in range(-(-n_q // 128)):
        lo, hi = 128 * kb, int(hi_key[128 * kb:128 * kb + 128].max())
        if hi - lo > qch and (hi - 1) // qch - lo // qch + 1 > 1:
            last = kb
    return last


@pytest.mark.parametrize("dt", ["bf16", "fp32"])
def test_attention_split_tiles_exact_and_undersized(dt):
    """The fp32 split sums sized from the tree (tt_attn_split_tiles, one
    128-key block per split key tile, compacted by the plan's split ranks)
    against the default workspace (a block for every key tile): the
    deterministic backward is bitwise equal, the default one equal to its
    atomics' rounding. A split_tiles one below the tree's count writes nothing
    past the workspace: exactly the keys of the last split tile (in key order)
    get NaN dk/dv, every other key's gradients are unchanged."""
    from tree_training_amd.attention import attn_backward, attn_forward
    from tree_training_amd.meta import KeyPlan, TreeMetaDevice
    lens, par = [2048, 300, 900, 700], [-1, 0, 0, 2]
    T = sum(lens)
    bf = torch.bfloat16 if dt == "bf16" else torch.float32
    g = torch.Generator(device=DEV).manual_seed(5)
    q, k, v, do = (torch.randn(T, h, D, device=DEV, generator=g, dtype=bf) for h in (HQ, HKV, HKV, HQ))
    view = lambda x: x[None].transpose(1, 2)
    plan = KeyPlan(TreeMetaDevice(lens, par, device=DEV).horizon, None, topo=(lens, par))
    need = plan.split_tiles()
    assert need == int(plan.plan[:28].view(torch.int32)[6].item()) >= 2
    kb_last = _last_split_tile(lens, par, T)
    print(f"split_tiles {need}, last split tile {kb_last}, {dt}", flush=True)
    o, lse = attn_forward(view(q), view(k), view(v), plan, D ** -0.5)
    run = lambda det: attn_backward(view(q), view(k), view(v), plan, D ** -0.5, o, lse, do[None],
                                    deterministic=det)
    exact = {det: run(det) for det in (True, False)}
    plan._split = 0                       # a block for every key tile
    full = {det: run(det) for det in (True, False)}
    plan._split = need - 1
    short = {det: run(det) for det in (True, False)}
    torch.cuda.synchronize()
    bar = 2e-2 if dt == "bf16" else 1e-5
    want_bad = torch.zeros(T, dtype=torch.bool, device=DEV)
    want_bad[128 * kb_last:128 * kb_last + 128] = True
    for det in (True, False):
        for name, a, b, c in zip(("dq", "dk", "dv"), exact[det], full[det], short[det]):
            assert torch.isfinite(a.float()).all(), (det, name)
            if det:
                assert torch.equal(a, b), (det, name)
            else:
                assert _max_rel(a.float(), b.float()) < bar, (det, name)
            if name == "dq":
                assert torch.equal(a, c) if det else _max_rel(a.float(), c.float()) < bar, (det, name)
                continue
            bad = torch.isnan(c.float()).any(dim=2).any(dim=1)
            assert torch.equal(bad, want_bad), (det, name)
            if det:
                assert torch.equal(a[~bad], c[~bad]), (det, name)
            else:
                assert _max_rel(a[~bad].float(), c[~bad].float()) < bar, (det, name)
