#!/usr/bin/env python3
"""Tree-attention forward + backward benchmark on one MI355X.

Workload (default ``agent16k``): the synthetic agent-trajectory tree (depth 6,
branching U{2,3,4}, node lengths U{64..512}, DFS-packed, capped at 16,384
tokens; seed 0) through one Qwen3-4B-shaped GQA attention layer (32 q heads,
8 kv heads, head_dim 128), bf16, q/k/v/dO ~ N(0,1) seeded, resident in HBM.
One step = DFS metadata + tile plan + tree-attention forward + full backward
(dQ, dK, dV) over the whole packed tree, each through the C ABI.

Metric: useful TFLOP/s = 12 * d * Hq * P / t_step, with P the number of
ancestor-visible (query, key) pairs per head (flash recompute not counted),
plus packed tokens/s. The dominant kernel's roofline figure is measured live
with HIP events on the launch stream; the CPU baseline times the dense-mask
restatement of the reference path (additive mask + repeat_kv + SDPA + autograd)
on a bounded sample on the host cores.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--workload agent16k|gateway16k|rollout48k|gdn16k|prologue16k|leafce16k]

Other workloads, each on the same 16K tree unless named:
  gateway16k   the tree cut into 4096-token partitions (tree_grad_hybrid, with
               the partitions of one cut node packed while they fit: 6), every
               partition's metadata and plan in one batched build, then each
               partition's attention fwd+bwd over its gateway prefix;
  rollout48k   one 8K prompt with 64 leaves (50,109 tokens);
  gdn16k       one GDN layer core (tree conv + gated-delta-rule scan) fwd+bwd,
               16 q/k heads, 32 v heads, fp32 state; packed tokens/s against
               the fp32 peak;
  prologue16k  the fused q/k RMSNorm + rotary fwd+bwd (HBM roofline);
  leafce16k    the fused leaf loss (chunked lm_head + row-wise CE) fwd+bwd.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

HQ, HKV, D = 32, 8, 128
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_FP32_TFS = 157.3        # MI355X fp32 (dense) TFLOP/s
PEAK_HBM_GBS = 8000.0
TRAFFIC_PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "tree_attn_agent16k_hbm_traffic.md")


def profiled_traffic(kernel, workload):
    """HBM bytes per launch of `kernel`, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (copy-calibrated), for the agent16k
    workload it was measured on; None otherwise."""
    if workload != "agent16k":
        return None
    try:
        with open(TRAFFIC_PROFILE) as f:
            lines = f.read().splitlines()
    except OSError:
        return None
    for ln in lines:
        cells = [c.strip() for c in ln.strip().strip("|").split("|")]
        if len(cells) >= 4 and cells[0] == kernel and cells[3].isdigit():
            return int(cells[3])
    return None


def profiled_step_traffic(profile):
    """HBM bytes per step of the library's kernels, from a committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (its "**N bytes**" total);
    None when the summary is absent."""
    import re
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", profile)
    try:
        with open(path) as f:
            m = re.search(r"\*\*(\d+) bytes\*\*", f.read())
    except OSError:
        return None
    return int(m.group(1)) if m else None


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="agent16k",
                    choices=["agent16k", "gateway16k", "rollout48k", "gdn16k", "prologue16k", "leafce16k"])
    ap.add_argument("--dtype", default="bf16", choices=["bf16", "fp32"],
                    help="attention workloads: element type of q/k/v/dO and the kernels' operands")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-runs", type=int, default=3)
    ap.add_argument("--calibrate-copy-mb", type=int, default=0,
                    help="before timing, run a plain device copy of this many MB (a known-size kernel for "
                         "scaling HBM byte counters)")
    return ap.parse_args()


def build_workload(name):
    from tree_training_amd import workloads
    if name == "rollout48k":
        return workloads.rollout_tree(0)
    return workloads.agent_tree(0)


def gateway_split(topo, max_tokens=4096):
    """Partitions of the tree (tree_grad_hybrid.partition_tree) with their
    inherited gateway visibility, as (node_len, parent, past_visible, pos_off)."""
    from tree_training_amd.tree import TreeNode
    from tree_training_amd.hybrid import hybrid_plan
    from tree_training_amd.workloads import forest_from_topology
    roots, _ = forest_from_topology(topo, TreeNode)
    return hybrid_plan(roots, max_tokens)


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the tree-attention path has no multi-GPU mode (a tree's "
              "key tiles would shard by kv-head group or by subtree across GPUs); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    if args.workload == "gdn16k":
        return run_gdn(args)
    if args.workload == "prologue16k":
        return run_prologue(args)
    if args.workload == "leafce16k":
        return run_leafce(args)
    import torch
    from tree_training_amd import _lib
    from tree_training_amd.attention import _Problem, attn_forward, fwd_workspace
    from tree_training_amd.meta import KeyPlan, TreeMetaDevice, _ptr, _stream, build_trees
    from tree_training_amd.workloads import visible_pairs
    import ctypes

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    topo = build_workload(args.workload)
    lens, par = topo
    T = sum(lens)
    P = visible_pairs(topo)
    g = torch.Generator(device=dev).manual_seed(0)
    bf = torch.bfloat16 if args.dtype == "bf16" else torch.float32
    # token-major storage viewed as [1, H, T, D] (transformers layout)
    q = torch.randn(1, T, HQ, D, device=dev, generator=g, dtype=bf).transpose(1, 2)
    k = torch.randn(1, T, HKV, D, device=dev, generator=g, dtype=bf).transpose(1, 2)
    v = torch.randn(1, T, HKV, D, device=dev, generator=g, dtype=bf).transpose(1, 2)
    do = torch.randn(1, T, HQ, D, device=dev, generator=g, dtype=bf)
    scale = D ** -0.5
    lib = _lib.lib()
    stream = torch.cuda.current_stream(dev)

    segments = None
    if args.workload == "gateway16k":
        segments = []
        for part in gateway_split(topo):
            n, lp = part["n_tokens"], part["past_len"]
            seg = dict(part)
            seg["q"] = torch.randn(1, n, HQ, D, device=dev, generator=g, dtype=bf).transpose(1, 2)
            seg["k"] = torch.randn(1, n, HKV, D, device=dev, generator=g, dtype=bf).transpose(1, 2)
            seg["v"] = torch.randn(1, n, HKV, D, device=dev, generator=g, dtype=bf).transpose(1, 2)
            seg["do"] = torch.randn(1, n, HQ, D, device=dev, generator=g, dtype=bf)
            if lp:
                seg["kp"] = torch.randn(1, HKV, lp, D, device=dev, generator=g, dtype=bf)
                seg["vp"] = torch.randn(1, HKV, lp, D, device=dev, generator=g, dtype=bf)
                seg["acc"] = (torch.zeros(lp, HKV, D, device=dev), torch.zeros(lp, HKV, D, device=dev))
                seg["bias_dev"] = seg["bias"].to(dev)
            segments.append(seg)

    def run_problem(lens_, par_, qq, kk, vv, dd, kp=None, vp=None, bias=None, acc=None, ev=None, pos_off=0,
                    plan=None):
        if plan is None:
            meta = TreeMetaDevice(lens_, par_, pos_offset=pos_off, device=dev)
            plan = KeyPlan(meta.horizon, bias)
        pb = _Problem(qq, kk, vv, kp, vp, plan, scale)
        N = pb.N
        o = torch.empty((N, HQ, D), dtype=bf, device=dev)
        lse = torch.empty((HQ, N), dtype=torch.float32, device=dev)
        dq = torch.empty((N, HQ, D), dtype=bf, device=dev)
        dk = torch.empty((N, HKV, D), dtype=bf, device=dev)
        dv = torch.empty((N, HKV, D), dtype=bf, device=dev)
        ws_bytes = lib.tt_attn_bwd_workspace_bytes(ctypes.byref(pb.s))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        st = _stream(dev)
        from tree_training_amd.attention import _tok_view
        dd, dst, dsh = _tok_view(dd)
        dt = _lib.TTTensor(dd.data_ptr(), dst, dsh)
        ak, av = (acc if acc is not None else (None, None))

        def rec(i):
            if ev is not None:
                ev[i].record(stream)
        rec(0)
        fws = fwd_workspace(pb, dev)
        _lib.check(lib.tt_attn_fwd(ctypes.byref(pb.s), _ptr(o), _ptr(lse), _ptr(fws) if fws is not None else None,
                                   fws.numel() if fws is not None else 0, st), "fwd")
        rec(1)
        if ev is None:   # one call, as the autograd backward makes it
            pb.s.bwd_parts = 0
            _lib.check(lib.tt_attn_bwd(ctypes.byref(pb.s), _ptr(o), _ptr(lse), dt, _ptr(dq), _ptr(dk), _ptr(dv),
                                       _ptr(ak), _ptr(av), _ptr(ws), ws_bytes, st), "bwd")
            return o, dq, dk, dv
        # delta and dQ in one call (the dQ kernel computes delta), then dK/dV:
        # the same work as bwd_parts=0, split only to time the passes
        pb.s.bwd_parts = _lib.TT_BWD_DELTA | _lib.TT_BWD_DQ
        _lib.check(lib.tt_attn_bwd(ctypes.byref(pb.s), _ptr(o), _ptr(lse), dt, _ptr(dq), _ptr(dk), _ptr(dv),
                                   _ptr(ak), _ptr(av), _ptr(ws), ws_bytes, st), "bwd delta+dq")
        rec(2)
        pb.s.bwd_parts = _lib.TT_BWD_DKDV
        _lib.check(lib.tt_attn_bwd(ctypes.byref(pb.s), _ptr(o), _ptr(lse), dt, _ptr(dq), _ptr(dk), _ptr(dv),
                                   _ptr(ak), _ptr(av), _ptr(ws), ws_bytes, st), "bwd dkdv")
        rec(3)
        return o, dq, dk, dv

    def step(ev=None):
        if segments is None:
            run_problem(lens, par, q, k, v, do, ev=ev)
            return
        # every partition's metadata and plan in one batched build (topology only),
        # as tree_grad_hybrid does, then the partitions in creation order
        built = build_trees([(seg["node_len"], seg["parent"], seg["pos_offset"], seg.get("bias_dev"))
                             for seg in segments], dev)
        for seg, (_, plan) in zip(segments, built):
            run_problem(seg["node_len"], seg["parent"], seg["q"], seg["k"], seg["v"], seg["do"],
                        seg.get("kp"), seg.get("vp"), seg.get("bias_dev"), seg.get("acc"),
                        ev=None, pos_off=seg["pos_offset"], plan=plan)

    if args.calibrate_copy_mb:
        src = torch.empty(args.calibrate_copy_mb << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    t0 = time.perf_counter()
    start_ev = torch.cuda.Event(enable_timing=True)
    end_ev = torch.cuda.Event(enable_timing=True)
    start_ev.record(stream)
    for i in range(args.steps):
        step(evs[i] if segments is None else None)
    end_ev.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = start_ev.elapsed_time(end_ev) / args.steps

    flops = 12.0 * D * HQ * P
    tflops = flops / (ms_step * 1e-3) / 1e12
    tokens_s = T / (ms_step * 1e-3)
    kernels = {}
    roofline = None
    if segments is None:
        sfx = "bf16" if args.dtype == "bf16" else "f32"
        names = [f"fwd_{sfx}_kernel", f"bwd_dq_{sfx}_kernel", f"bwd_dkdv_{sfx}_kernel"]
        peak = PEAK_BF16_TFLOPS if args.dtype == "bf16" else PEAK_FP32_TFS
        useful = [4.0 * D * HQ * P, 4.0 * D * HQ * P, 4.0 * D * HQ * P]
        for j, name in enumerate(names):
            ms = statistics.mean(e[j].elapsed_time(e[j + 1]) for e in evs)
            kernels[name] = {"ms": round(ms, 4),
                             "useful_tflops": round(useful[j] / (ms * 1e-3) / 1e12, 2) if useful[j] else None}
        dom = max((n for n in names if kernels[n]["useful_tflops"]), key=lambda n: kernels[n]["ms"])
        ach = kernels[dom]["useful_tflops"]
        roofline = {"bound": "mfma", "kernel": dom, "achieved": ach, "peak": peak,
                    "unit": "TFLOP/s", "frac": round(ach / peak, 4),
                    "traffic": profiled_traffic(dom, args.workload) if args.dtype == "bf16" else None,
                    "flops_per_launch": useful[names.index(dom)]}
        if dom == "bwd_dkdv_bf16_kernel":
            roofline["timed"] = "dK/dV pass: split-sum zero + bwd_dkdv_bf16_kernel + split-sum finalize"
        if dom == "bwd_dq_f32_kernel":
            roofline["timed"] = "dQ pass: bwd_delta_f32_kernel + bwd_dq_f32_kernel"

    cpu = None
    if not args.no_cpu_baseline and args.dtype == "bf16":
        cpu = cpu_baseline(topo, args.cpu_runs, args.workload)

    line = {
        "metric": f"tree-attn fwd+bwd useful TFLOP/s (16K-token DFS tree, {args.dtype})",
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic (seeded topology and N(0,1) q/k/v/dO)",
        "config": {"workload": args.workload, "packed_tokens": T, "visible_pairs_per_head": P,
                   "n_nodes": len(lens), "heads_q": HQ, "heads_kv": HKV, "head_dim": D,
                   "layer": "one Qwen3-4B-shaped GQA attention layer", "parallelism": "single GPU",
                   **({"max_tokens": 4096, "partitions": len(segments)} if segments is not None else {})},
        "tokens_per_s": round(tokens_s, 1),
        "frac_of_peak": round(tflops / (PEAK_BF16_TFLOPS if args.dtype == "bf16" else PEAK_FP32_TFS), 4),
        "wall_s_timed": round(wall, 3),
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def run_leafce(args):
    """Leaf loss head on the 16K agent tree: lm_head (V = 151,936, hidden 2560,
    bf16) + cross-entropy on every leaf's tokens, forward + backward, through
    the fused chunked path (``loss.TreeCELoss.fused``: tt_ce_rows between
    hipBLASLt GEMMs, no [T, V] logits). The reference's path (logits for every
    token, then F.cross_entropy per leaf) is timed beside it on the same GPU,
    with both paths' peak memory."""
    import torch
    import torch.nn.functional as F
    from tree_training_amd.loss import TreeCELoss
    from tree_training_amd.workloads import agent_tree
    V, H = 151936, 2560
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    lens, par = agent_tree(0)
    T = sum(lens)
    starts = [0]
    for L in lens[:-1]:
        starts.append(starts[-1] + L)
    kids = set(p for p in par if p >= 0)
    spans = [(starts[i], starts[i] + lens[i]) for i in range(len(lens)) if i not in kids]
    n_leaf_tok = sum(e - s for s, e in spans)
    gen = torch.Generator(device=dev).manual_seed(0)
    bf = torch.bfloat16
    hidden = torch.randn(T, H, device=dev, generator=gen, dtype=bf).requires_grad_(True)
    weight = (torch.randn(V, H, device=dev, generator=gen, dtype=bf) * 0.02).requires_grad_(True)
    nodes = [object() for _ in spans]
    labels = [torch.randint(0, V, (e - s,), device=dev, generator=gen) for s, e in spans]
    fn = TreeCELoss(labels, nodes, len(spans))

    # Both paths start each step with unset gradients (zero_grad(set_to_none=True)).
    def fused_step():
        hidden.grad = weight.grad = None
        fn.fused_spans(hidden, [(s, e, n) for (s, e), n in zip(spans, nodes)], weight).backward()

    def torch_step():
        hidden.grad = weight.grad = None
        logits = (hidden @ weight.t())[None]
        loss = sum(fn(logits[:, s:e, :], n) for (s, e), n in zip(spans, nodes))
        loss.backward()

    def timed(step, steps):
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(dev)
        base = torch.cuda.memory_allocated(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st = torch.cuda.current_stream(dev)
        t0 = time.perf_counter()
        e0.record(st)
        for _ in range(steps):
            step()
        e1.record(st)
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated(dev) - base
        return e0.elapsed_time(e1) / steps, time.perf_counter() - t0, peak

    ms, wall, peak = timed(fused_step, args.steps)
    ms_t, _, peak_t = timed(torch_step, max(2, args.steps // 4))
    flops = 3 * 2.0 * n_leaf_tok * V * H          # logits, d_hidden, d_weight GEMMs (leaf tokens only)
    tfs = flops / (ms * 1e-3) / 1e12
    cpu = None if args.no_cpu_baseline else leafce_cpu_baseline(args.cpu_runs)
    line = {
        "metric": "leaf loss head (lm_head + CE) fwd+bwd leaf tokens/s (16K-token DFS tree, V=151936)",
        "value": round(n_leaf_tok / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 GEMMs, f32 softmax",
        "data": "synthetic (seeded N(0,1) hidden states, 0.02 N(0,1) lm_head, uniform labels)",
        "config": {"workload": "leafce16k", "packed_tokens": T, "leaf_tokens": n_leaf_tok, "leaves": len(spans),
                   "vocab": V, "hidden": H, "chunk": 4096, "parallelism": "single GPU"},
        "wall_s_timed": round(wall, 3),
        "peak_extra_bytes": int(peak),
        "reference_path": {"ms_per_step": round(ms_t, 4), "peak_extra_bytes": int(peak_t),
                           "what": "logits for every token (hidden @ W^T) + F.cross_entropy per leaf + autograd"},
        "roofline": {"bound": "mfma", "kernel": "whole step (3 GEMMs per chunk + tt_ce_rows)", "achieved": round(tfs, 1),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(tfs / PEAK_BF16_TFLOPS, 5),
                     "traffic": None, "flops_per_step": flops},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def leafce_cpu_baseline(runs):
    """torch cross-entropy (forward + autograd backward) on 64 rows of the
    full vocabulary in float32 on the host, 16 threads, median of ``runs``,
    in rows/s (the GEMMs are not included)."""
    import torch
    import torch.nn.functional as F
    cores = cpu_threads()
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 151936, generator=g).requires_grad_(True)
    y = torch.randint(0, 151936, (64,), generator=g)
    times = []
    for i in range(runs + 1):
        t0 = time.perf_counter()
        F.cross_entropy(x, y).backward()
        if i:
            times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"value": round(64 / t, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"64 rows x 151936 classes, torch float32 cross-entropy forward + backward on the host "
                      f"(the softmax part only), median of {runs} after 1 warm-up", "seconds_per_sample": round(t, 4)}


def run_prologue(args):
    """Fused attention prologue (q/k RMSNorm + rotary embedding) forward +
    backward on the 16K agent tree at its depth positions, Qwen3-4B shapes (32
    q / 8 kv heads, d 128), bf16, through the C ABI. Also times transformers'
    own prologue (q_norm / k_norm + apply_rotary_pos_emb, forward + autograd
    backward) on the same GPU for comparison."""
    import torch
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm, apply_rotary_pos_emb
    from tree_training_amd.meta import TreeMetaDevice
    from tree_training_amd.prologue import qk_prologue_backward, qk_prologue_forward
    from tree_training_amd.workloads import agent_tree
    Hq, Hkv = HQ, HKV
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    lens, par = agent_tree(0)
    T = sum(lens)
    pos = TreeMetaDevice(lens, par, pos_offset=0, device=dev).pos       # depth positions (metadata kernel)
    gen = torch.Generator(device=dev).manual_seed(0)
    bf = torch.bfloat16
    pq = torch.randn(T, Hq * D, device=dev, generator=gen, dtype=bf)
    pk = torch.randn(T, Hkv * D, device=dev, generator=gen, dtype=bf)
    qw = (torch.rand(D, device=dev, generator=gen) + 0.5).to(bf)
    kw = (torch.rand(D, device=dev, generator=gen) + 0.5).to(bf)
    inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, device=dev, dtype=torch.float32) / D))
    emb = torch.cat([pos[:, None].float() * inv[None]] * 2, dim=-1)
    cos, sin = emb.cos().to(bf), emb.sin().to(bf)
    dq = torch.randn(T, Hq, D, device=dev, generator=gen, dtype=bf)
    dk = torch.randn(T, Hkv, D, device=dev, generator=gen, dtype=bf)
    q_raw, k_raw = pq.view(T, Hq, D), pk.view(T, Hkv, D)

    def step():
        qk_prologue_forward(q_raw, k_raw, qw, kw, 1e-6, 1e-6, cos, sin)
        qk_prologue_backward(q_raw, k_raw, qw, kw, 1e-6, 1e-6, cos, sin, dq, dk)

    qn, kn = Qwen3RMSNorm(D).to(dev, bf), Qwen3RMSNorm(D).to(dev, bf)
    with torch.no_grad():
        qn.weight.copy_(qw)
        kn.weight.copy_(kw)
    xq = q_raw.detach().requires_grad_(True)
    xk = k_raw.detach().requires_grad_(True)

    def torch_step():
        a = qn(xq[None]).transpose(1, 2)
        b = kn(xk[None]).transpose(1, 2)
        qe, ke = apply_rotary_pos_emb(a, b, cos[None], sin[None])
        torch.autograd.backward((qe, ke), (dq[None].transpose(1, 2), dk[None].transpose(1, 2)))

    def timed(fn, steps):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st = torch.cuda.current_stream(dev)
        t0 = time.perf_counter()
        e0.record(st)
        for _ in range(steps):
            fn()
        e1.record(st)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps, time.perf_counter() - t0

    ms, wall = timed(step, args.steps)
    ms_torch, _ = timed(torch_step, args.steps)
    row = (Hq + Hkv) * D * 2
    alg = T * (row + 2 * D * 2) + T * (3 * row + 2 * D * 2)     # fwd: x, cos/sin, out; bwd: x, dout, cos/sin, dx
    gbs = alg / (ms * 1e-3) / 1e9
    cpu = None if args.no_cpu_baseline else prologue_cpu_baseline(args.cpu_runs)
    line = {
        "metric": "attention prologue (q/k RMSNorm + RoPE) fwd+bwd packed tokens/s (16K-token DFS tree)",
        "value": round(T / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 in/out, f32 arithmetic",
        "data": "synthetic (seeded N(0,1) projections and gradients; rotary table at the tree's depth positions)",
        "config": {"workload": "prologue16k", "packed_tokens": T, "heads_q": Hq, "heads_kv": Hkv, "head_dim": D,
                   "rope_theta": 1e6, "parallelism": "single GPU"},
        "wall_s_timed": round(wall, 3),
        "torch_prologue_ms": round(ms_torch, 4),
        "roofline": {"bound": "hbm", "kernel": "prologue_fwd_kernel + prologue_bwd_kernel (+ dw reduce)",
                     "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 5), "traffic": None, "bytes_per_step": alg},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def prologue_cpu_baseline(runs):
    """The float64 oracle (torch, autograd backward) on 512 tokens x 40 heads,
    16 host threads, median of ``runs`` after a warm-up, in tokens/s."""
    import torch
    from oracle.prologue import qk_prologue
    cores = cpu_threads()
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(0)
    n = 512
    x = torch.randn(n, HQ + HKV, D, dtype=torch.float64, generator=g).requires_grad_(True)
    w = torch.rand(D, dtype=torch.float64, generator=g).requires_grad_(True)
    cos, sin = torch.rand(n, D, dtype=torch.float64), torch.rand(n, D, dtype=torch.float64)
    dy = torch.randn(n, HQ + HKV, D, dtype=torch.float64, generator=g)
    times = []
    for i in range(runs + 1):
        t0 = time.perf_counter()
        out = qk_prologue(x, w, 1e-6, cos, sin)
        torch.autograd.grad((out * dy).sum(), (x, w))
        if i:
            times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"value": round(n / t, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{n} tokens x 40 heads, float64 oracle forward + autograd backward (torch CPU), "
                      f"median of {runs} after 1 warm-up", "seconds_per_sample": round(t, 4)}


def gdn_useful_flops(n_chunk_heads, C=32, Dh=128):
    """fp32 FLOPs of the chunked tree gated delta rule, forward + backward,
    counted once (the backward's forward recompute excluded), per (chunk, v
    head) pair, as multiply-adds x 2:
      forward   3 C D^2 (W S, q S, the state update) + 5 C^2 D (q k^T, k k^T,
                T (beta v), T (beta k), A V') + C^3 / 3 (the triangular inverse)
      backward  6 C D^2 (A^T dO and K~ dS aside, the products with the states:
                K~ dS, (e^G q)^T dO, W^T dV', dO S^T, dV' S^T, V' dS^T)
                + 11 C^2 D + 2 C^3 (the chunk's 32 x 32 algebra)."""
    fwd = 3 * C * Dh * Dh + 5 * C * C * Dh + C ** 3 / 3
    bwd = 6 * C * Dh * Dh + 11 * C * C * Dh + 2 * C ** 3
    return 2.0 * (fwd + bwd) * n_chunk_heads


def run_gdn(args):
    """One tree-aware GDN layer core on the 16K agent tree, forward + backward:
    tree conv (8192 channels, width 4) + tree gated-delta-rule scan, through
    the autograd Functions (the projections and the norm stay torch GEMMs and
    are not timed)."""
    import torch
    from tree_training_amd.conv import tree_conv
    from tree_training_amd.gdn import GdnTree, gdn_tree
    from tree_training_amd.workloads import agent_tree
    HK, HV, K = 16, 32, 4
    C = 2 * HK * D + HV * D
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    lens, par = agent_tree(0)
    T = sum(lens)
    gen = torch.Generator(device=dev).manual_seed(0)
    bf = torch.bfloat16
    x = torch.randn(T, C, device=dev, generator=gen, dtype=bf).requires_grad_(True)   # raw qkv projections
    w = (torch.randn(C, K, device=dev, generator=gen) * 0.5).to(bf).requires_grad_(True)
    a = torch.randn(T, HV, device=dev, generator=gen)
    b = torch.randn(T, HV, device=dev, generator=gen)
    A_log = torch.log(torch.rand(HV, device=dev, generator=gen) * 16.0 + 1e-3)
    g = (-A_log.exp() * torch.nn.functional.softplus(a + 1.0)).requires_grad_(True)   # dt_bias = 1
    beta = b.sigmoid().requires_grad_(True)
    d_o = torch.randn(T, HV, D, device=dev, generator=gen, dtype=bf)
    tree = GdnTree(lens, par, dev)

    def step():
        # Gradients start unset each step (an optimizer's zero_grad(set_to_none=True)),
        # so backward writes them rather than adding into the last step's.
        for t in (x, w, g, beta):
            t.grad = None
        q, k, v = tree_conv(x, w, None, tree, split_sizes=(HK * D, HK * D, HV * D))
        o, _ = gdn_tree(q.view(T, HK, D), k.view(T, HK, D), v.view(T, HV, D), g, beta, tree, None, True)
        o.backward(d_o)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    flops = gdn_useful_flops(tree.n_chunks * HV)
    tfs = flops / (ms * 1e-3) / 1e12
    cpu = None if args.no_cpu_baseline else gdn_cpu_baseline(lens, par, args.cpu_runs)
    line = {
        "metric": "tree GDN layer core (conv + scan) fwd+bwd packed tokens/s (16K-token DFS tree)",
        "value": round(T / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 in/out, f32 arithmetic and state",
        "data": "synthetic (seeded topology; qkv rows and dO N(0,1); conv weight 0.5 N(0,1); gates from N(0,1) "
                "logits, A_log = log U(0,16), dt_bias = 1)",
        "config": {"workload": "gdn16k", "packed_tokens": T, "n_nodes": len(lens), "tree_levels": tree.n_levels,
                   "chunks": tree.n_chunks, "heads_qk": HK, "heads_v": HV, "head_dim": D, "conv_channels": C,
                   "conv_width": K, "chunk": 32, "layer": "one GDN layer core (conv + scan), fwd+bwd",
                   "parallelism": "single GPU"},
        "wall_s_timed": round(wall, 3),
        "roofline": {"bound": "mfma", "kernel": "whole step (conv, prep, level scans, reverse scans, gradient "
                                                 "kernels); fp32 products (scans and state products on fp32 MFMA, "
                                                 "the rest on the vector ALUs), ceiling = fp32 peak",
                     "achieved": round(tfs, 2), "peak": PEAK_FP32_TFS, "unit": "TFLOP/s",
                     "frac": round(tfs / PEAK_FP32_TFS, 5),
                     "traffic": profiled_step_traffic("gdn16k_counters.md"),
                     "traffic_unit": "HBM bytes per step, library kernels (rocprofv3 FETCH_SIZE / WRITE_SIZE, "
                                     "copy-calibrated)", "flops_per_step": flops},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def gdn_cpu_baseline(lens, par, runs):
    """The float64 torch oracle (token recurrence, autograd backward) on one
    root-to-leaf path of the tree and one v head, forward + backward, one host
    thread; median of ``runs`` after a warm-up, in tokens/s scaled to the 32
    v heads of the workload."""
    import numpy as np
    import torch
    from oracle.gdn import gdn_tree_torch
    torch.set_num_threads(1)
    leaf = next(i for i in range(len(lens)) if i not in set(par))
    path, j = [], leaf
    while j >= 0:
        path.append(j)
        j = par[j]
    plens = [lens[i] for i in path[::-1]]
    T = sum(plens)
    rng = np.random.default_rng(0)
    mk = lambda *s: torch.from_numpy(rng.standard_normal(s)).requires_grad_(True)
    q, k, v = mk(T, 1, D), mk(T, 1, D), mk(T, 1, D)
    g = torch.from_numpy(-np.abs(rng.standard_normal((T, 1))) * 0.5).requires_grad_(True)
    beta = torch.from_numpy(rng.uniform(0, 1, (T, 1))).requires_grad_(True)
    d_o = torch.from_numpy(rng.standard_normal((T, 1, D)))
    times = []
    for i in range(runs + 1):
        t0 = time.perf_counter()
        o = gdn_tree_torch(q, k, v, g, beta, plens, list(range(-1, len(plens) - 1)))
        o.backward(d_o)
        if i:
            times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"value": round(T / (t * 32), 1), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"one root-to-leaf path ({T} tokens, {len(plens)} nodes) of the tree, 1 of 32 v heads: "
                      f"float64 token recurrence with autograd backward (oracle), median of {runs} after 1 "
                      f"warm-up, scaled by 1/32",
            "seconds_per_sample": round(t, 3)}


def cpu_threads():
    """Host threads for the CPU baselines: the job's CPU share when the
    launcher states it (OMP_NUM_THREADS, set to the cores granted to this
    process on a shared host), else os.cpu_count()."""
    n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    return min(n, int(env)) if env.isdigit() and int(env) > 0 else n


C1_TOPOLOGY = ([3, 4, 3, 4, 5, 3, 3, 4, 4, 3, 4, 3, 4], [-1, 0, 1, 2, 3, 3, 2, 6, -1, 8, 9, 8, 11])


def literal_metadata_seconds(workload, topo):
    """Host time of the reference's metadata as its literal loops (the
    restatement of build_dfs_tree_info's per-pair mask loop; for the gateway
    workload the whole partition schedule: partitions, per-partition DFS info
    and gateway biases), on the 47-token two-root tree and on the workload's
    tree. The 48K rollout tree (3.9e8 mask writes) is not timed."""
    from oracle.partition import hybrid_schedule
    from oracle.tree_meta import build_dfs_tree_info_literal
    from tree_training_amd.tree import TreeNode
    from tree_training_amd.workloads import forest_from_topology
    out = {}
    for name, tp in (("c1_47_tokens", C1_TOPOLOGY), (workload, topo)):
        if name == "rollout48k":
            out[name] = None
            continue
        roots, _ = forest_from_topology(tp, TreeNode)
        t0 = time.perf_counter()
        if name == "gateway16k":
            hybrid_schedule(roots, 4096)
        else:
            build_dfs_tree_info_literal(roots)
        out[name] = round(time.perf_counter() - t0, 4)
    return out


def cpu_baseline(topo, runs, workload="agent16k"):
    """Dense-mask restatement of the reference path on the host cores, on one
    kv-head group (4 q heads + 1 kv head) of the same tree: median of ``runs``
    fwd+bwd after one warm-up. Reported in the metric's unit (useful TFLOP/s
    for the sampled heads)."""
    import torch
    from oracle.dense_path import additive_mask, dense_fwd_bwd
    from oracle.tree_meta import mask_from_horizon, meta_closed_form
    from tree_training_amd.workloads import visible_pairs
    cores = cpu_threads()
    torch.set_num_threads(cores)
    lens, par = topo
    m = meta_closed_form(lens, par)
    T = m["T"]
    P = visible_pairs(topo)
    t0 = time.perf_counter()
    am = additive_mask(torch.from_numpy(mask_from_horizon(m["horizon"])), torch.bfloat16)
    t_mask = time.perf_counter() - t0
    g = torch.Generator().manual_seed(0)
    hq = HQ // HKV
    q = torch.randn(1, hq, T, D, generator=g).bfloat16()
    k = torch.randn(1, 1, T, D, generator=g).bfloat16()
    v = torch.randn(1, 1, T, D, generator=g).bfloat16()
    do = torch.randn(1, T, hq, D, generator=g).bfloat16()
    times = []
    for i in range(runs + 1):
        t0 = time.perf_counter()
        dense_fwd_bwd(q, k, v, am, D ** -0.5, do)
        dt = time.perf_counter() - t0
        if i:
            times.append(dt)
    t = statistics.median(times)
    useful = 12.0 * D * hq * P
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(useful / t / 1e12, 5), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"1 of 8 kv-head groups (4 q heads) of the full {T}-token tree, dense additive mask + "
                      f"repeat_kv + SDPA fwd+bwd in bf16 (torch CPU), median of {runs} after 1 warm-up",
            "seconds_per_sample": round(t, 3), "mask_build_s": round(t_mask, 3),
            "metadata_literal_s": literal_metadata_seconds(workload, topo),
            "tokens_per_s_full_layer": round(T / (t * HKV), 1), "cpu_model": model,
            "os_cpu_count": os.cpu_count()}


if __name__ == "__main__":
    main()
