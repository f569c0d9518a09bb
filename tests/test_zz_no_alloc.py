"""tt_attn_bwd_noalloc (the backward without a workspace argument, for callers
that cannot allocate) against tt_attn_bwd on the same inputs, through the C
ABI: two calls in a row on one GPU, the second with a smaller problem, so the
shared scratch array is reused with stale contents from the first.

Bars: dq bitwise equal (one writer per element); dk / dv / gateway
accumulators within the dtype's bar (max_rel < 1e-5 for float32, 2e-2 for
bf16: fp32 atomics of split key tiles may round differently between runs)."""
import ctypes
import math
import sys

import numpy as np
import pytest
import torch

from tree_training_amd import _lib, workloads

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
HQ, HKV, D = 32, 8, 128


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).abs().max() / max(float(b.abs().max()), 1e-30))


def _case(lens, par, n_past, dtype, seed):
    from tree_training_amd.attention import _Problem, fwd_workspace
    from tree_training_amd.meta import KeyPlan, TreeMetaDevice
    T = sum(lens)
    g = torch.Generator().manual_seed(seed)
    mk = lambda *s: torch.randn(*s, generator=g).to(dtype).to(DEV)
    q, k, v, do = mk(1, T, HQ, D), mk(1, T, HKV, D), mk(1, T, HKV, D), mk(1, T, HQ, D)
    kp = vp = bias = None
    if n_past:
        kp, vp = mk(1, n_past, HKV, D), mk(1, n_past, HKV, D)
        bias = torch.tensor([0.0 if (i % 5) != 2 else -math.inf for i in range(n_past)])
    meta = TreeMetaDevice(lens, par, device=DEV, validate=True)
    plan = KeyPlan(meta.horizon, bias, validate=True)
    tr = lambda x: None if x is None else x.transpose(1, 2)
    pb = _Problem(tr(q), tr(k), tr(v), tr(kp), tr(vp), plan, D ** -0.5)
    o = torch.empty((T, HQ, D), dtype=dtype, device=DEV)
    lse = torch.empty((HQ, T), dtype=torch.float32, device=DEV)
    st = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    fws = fwd_workspace(pb, DEV)
    _lib.check(_lib.lib().tt_attn_fwd(ctypes.byref(pb.s), ctypes.c_void_p(o.data_ptr()),
                                      ctypes.c_void_p(lse.data_ptr()),
                                      ctypes.c_void_p(fws.data_ptr()) if fws is not None else None,
                                      fws.numel() if fws is not None else 0, st), "tt_attn_fwd")
    return dict(pb=pb, o=o, lse=lse, do=do, T=T, n_past=n_past, dtype=dtype, keep=(meta, plan))


def _bwd(c, noalloc):
    lib = _lib.lib()
    T, n_past, dtype = c["T"], c["n_past"], c["dtype"]
    dq = torch.full((T, HQ, D), float("nan"), dtype=dtype, device=DEV)
    dk = torch.full((T, HKV, D), float("nan"), dtype=dtype, device=DEV)
    dv = torch.full((T, HKV, D), float("nan"), dtype=dtype, device=DEV)
    acc = [torch.zeros(max(n_past, 1), HKV, D, device=DEV) for _ in range(2)]
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    d_o = _lib.TTTensor(c["do"].data_ptr(), HQ * D, D)
    st = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    accp = [P(a) if n_past else None for a in acc]
    if noalloc:
        rc = lib.tt_attn_bwd_noalloc(ctypes.byref(c["pb"].s), P(c["o"]), P(c["lse"]), d_o, P(dq), P(dk), P(dv),
                                     accp[0], accp[1], st)
        what = "tt_attn_bwd_noalloc"
    else:
        ws_bytes = lib.tt_attn_bwd_workspace_bytes(ctypes.byref(c["pb"].s))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
        rc = lib.tt_attn_bwd(ctypes.byref(c["pb"].s), P(c["o"]), P(c["lse"]), d_o, P(dq), P(dk), P(dv),
                             accp[0], accp[1], P(ws), ws_bytes, st)
        what = "tt_attn_bwd"
    _lib.check(rc, what)
    torch.cuda.synchronize()
    return dq, dk, dv, acc[0][:n_past], acc[1][:n_past]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_noalloc_backward_matches_workspace_backward(dtype):
    big = (workloads.random_forest(14, node_len=(40, 300)), 700)       # ragged forest + gateway
    small = (([70, 45, 90, 33], [-1, 0, 0, 2]), 0)                      # smaller, no gateway
    for step, ((lens, par), n_past) in enumerate((big, small)):
        print(f"noalloc {dtype} call {step}: T={sum(lens)} n_past={n_past}", flush=True)
        sys.stdout.flush()
        c = _case(lens, par, n_past, dtype, seed=40 + step)
        need = _lib.lib().tt_attn_bwd_workspace_bytes(ctypes.byref(c["pb"].s))
        assert 0 < need <= _lib.lib().tt_noalloc_scratch_bytes()
        ref = _bwd(c, noalloc=False)
        got = _bwd(c, noalloc=True)
        names = ("dq", "dk", "dv", "dk_gateway", "dv_gateway")
        for name, a, b in zip(names, got, ref):
            assert a.shape == b.shape, name
            if a.numel() == 0:      # gateway slices of the call without a gateway
                continue
            assert torch.isfinite(a).all(), name
            if name == "dq":
                assert torch.equal(a, b), name
            else:
                bar = 1e-5 if dtype == torch.float32 else 2e-2
                assert _rel(a, b) < bar, (name, _rel(a, b))


def test_noalloc_agent_tree_with_exact_split_tiles():
    """The 16K agent tree (16,318 tokens, bf16, 32/8 heads) fits the scratch
    once its split sums are sized from the tree (tt_attn_split_tiles): the
    no-allocation backward against tt_attn_bwd with the same problem."""
    lens, par = workloads.agent_tree(0)
    print(f"noalloc agent tree T={sum(lens)}", flush=True)
    c = _case(lens, par, 0, torch.bfloat16, seed=44)
    from tree_training_amd.meta import KeyPlan
    plan = KeyPlan(c["keep"][0].horizon, topo=(lens, par))
    c["pb"].s.split_tiles = plan.split_tiles()
    lib = _lib.lib()
    need = lib.tt_attn_bwd_workspace_bytes(ctypes.byref(c["pb"].s))
    assert c["pb"].s.split_tiles >= 1 and 0 < need <= lib.tt_noalloc_scratch_bytes()
    c["pb"].s.split_tiles = 0
    assert lib.tt_attn_bwd_workspace_bytes(ctypes.byref(c["pb"].s)) > lib.tt_noalloc_scratch_bytes()
    c["pb"].s.split_tiles = plan.split_tiles()
    ref = _bwd(c, noalloc=False)
    got = _bwd(c, noalloc=True)
    for name, a, b in zip(("dq", "dk", "dv"), got, ref):
        assert torch.isfinite(a.float()).all(), name
        if name == "dq":
            assert torch.equal(a, b), name
        else:
            assert _rel(a, b) < 2e-2, (name, _rel(a, b))


_FIRST_CALL_PROBE = r"""
import ctypes, torch
from tree_training_amd import _lib
from tree_training_amd.attention import _Problem, attn_forward
from tree_training_amd.meta import KeyPlan, TreeMetaDevice
dev = torch.device("cuda", 0)
lens, par, HQ, HKV, D = [300, 200, 100], [-1, 0, 0], 32, 8, 128
T = sum(lens)
g = torch.Generator(device=dev).manual_seed(0)
q = torch.randn(1, HQ, T, D, device=dev, generator=g, dtype=torch.bfloat16)
k = torch.randn(1, HKV, T, D, device=dev, generator=g, dtype=torch.bfloat16)
plan = KeyPlan(TreeMetaDevice(lens, par, device=dev).horizon)
o, lse = attn_forward(q, k, k, plan, D ** -0.5)
pb = _Problem(q, k, k, None, None, plan, D ** -0.5)
do = torch.randn(T, HQ, D, device=dev, generator=g, dtype=torch.bfloat16)
out = [torch.empty(T, h, D, device=dev, dtype=torch.bfloat16) for h in (HQ, HKV, HKV)]
torch.cuda.synchronize()
lib = _lib.lib()
P = lambda t: ctypes.c_void_p(t.data_ptr())
st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
free = [torch.cuda.mem_get_info(dev)[0]]
lib.tt_noalloc_scratch_bytes()
free.append(torch.cuda.mem_get_info(dev)[0])
for _ in range(2):
    _lib.check(lib.tt_attn_bwd_noalloc(ctypes.byref(pb.s), P(o), P(lse), _lib.TTTensor(do.data_ptr(), HQ * D, D),
                                       *map(P, out), None, None, st), "tt_attn_bwd_noalloc")
    torch.cuda.synchronize()
    free.append(torch.cuda.mem_get_info(dev)[0])
print("FREE", *free)
"""


def test_noalloc_scratch_reserved_on_first_call():
    """The scratch array lives in a translation unit of its own, whose code
    object HIP loads on first use: in a fresh process that has run the
    library's other kernels, device memory is taken only by the first
    tt_attn_bwd_noalloc call (>= the scratch size), and not again by the
    second (a process that never calls it never holds the scratch)."""
    import os
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("noalloc first-call probe (subprocess)", flush=True)
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_PROBE], cwd=root, capture_output=True, text=True,
                       timeout=240, env=dict(os.environ, PYTHONPATH=root))
    assert r.returncode == 0, r.stderr[-2000:]
    line = [ln for ln in r.stdout.splitlines() if ln.startswith("FREE")][-1]
    f0, f1, f2, f3 = map(int, line.split()[1:])
    MiB = 1 << 20
    print(f"taken: host query {(f0 - f1) / MiB:.1f} MiB, first call {(f1 - f2) / MiB:.1f} MiB, "
          f"second call {(f2 - f3) / MiB:.1f} MiB", flush=True)
    assert f0 - f1 < 4 * MiB
    assert f1 - f2 >= _lib.lib().tt_noalloc_scratch_bytes()
    assert abs(f2 - f3) < 4 * MiB


def test_noalloc_rejects_problems_beyond_the_scratch():
    """A problem whose workspace exceeds the scratch array returns
    TT_E_WORKSPACE and launches nothing (outputs untouched)."""
    from tree_training_amd.attention import _Problem
    from tree_training_amd.meta import KeyPlan, TreeMetaDevice
    lib = _lib.lib()
    T = 40000
    meta = TreeMetaDevice([T], [-1], device=DEV, validate=True)
    plan = KeyPlan(meta.horizon)
    x = torch.zeros(1, HQ, T, D, dtype=torch.bfloat16, device=DEV)
    kv = torch.zeros(1, HKV, T, D, dtype=torch.bfloat16, device=DEV)
    pb = _Problem(x, kv, kv, None, None, plan, D ** -0.5)
    assert lib.tt_attn_bwd_workspace_bytes(ctypes.byref(pb.s)) > lib.tt_noalloc_scratch_bytes()
    out = torch.full((T, HQ, D), 7.0, dtype=torch.bfloat16, device=DEV)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = lib.tt_attn_bwd_noalloc(ctypes.byref(pb.s), P(out), P(out), _lib.TTTensor(out.data_ptr(), HQ * D, D),
                                 P(out), P(out), P(out), None, None,
                                 ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream))
    assert rc == _lib.TT_E_WORKSPACE
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
