"""Device-side tree metadata and tile plans (thin wrappers over the C ABI).

``TreeMetaDevice`` replaces the positions / dense mask of ``build_dfs_tree_info``
(dfs_tree_forward.py:91-184) with int32 device arrays produced by the HIP
metadata kernel: ``pos`` (depth-based positions, plus the partition offset of
tree_grad_hybrid.py:307-310), ``node_of`` and ``horizon`` (exclusive subtree
end per token; key j is visible to query i iff j <= i < horizon[j]).

``KeyPlan`` turns a horizon (and an optional gateway bias, the ``attn_bias`` of
tree_grad_hybrid.py:160-209) into per-key visible query intervals and the
block-sparsity plan the attention kernels walk. One plan serves every layer of
a forward pass.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import check, lib
from .tree import preorder_violation


def _ptr(t: Optional[torch.Tensor]):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def upload_i32(rows, device) -> torch.Tensor:
    """Host integers (a sequence, or equal-length rows) as a device int32 tensor,
    without synchronising the stream.

    ``torch.tensor(..., device=cuda)`` copies from pageable memory and then waits
    for the whole stream, so every upload would drain the launch queue. Staged
    through pinned memory, the copy is queued like a kernel; torch's caching
    host allocator keeps the pinned block until the copy has run."""
    return to_device(torch.from_numpy(np.ascontiguousarray(np.asarray(rows, dtype=np.int32))), device,
                     torch.int32)


def to_device(t: torch.Tensor, device, dtype: torch.dtype) -> torch.Tensor:
    """``t`` as a contiguous ``dtype`` tensor on ``device``; a host tensor goes
    through pinned memory with a non-blocking copy (no stream synchronisation)."""
    if t.device.type == "cpu":
        h = t.to(dtype).contiguous()
        # a fresh pinned copy: the caller may reuse its own (pinned) tensor at once
        h = h.clone().pin_memory() if h.is_pinned() else h.pin_memory()
        return h.to(device, non_blocking=True)
    return t.to(device=device, dtype=dtype).contiguous()


def require_device(device=None) -> torch.device:
    """The product path runs on a ROCm GPU only; fail loudly otherwise."""
    if not torch.cuda.is_available():
        raise _lib.TreeAttnError("tree attention needs a ROCm GPU (torch.cuda.is_available() is False)")
    if device is None:
        return torch.device("cuda", torch.cuda.current_device())
    device = torch.device(device)
    if device.type != "cuda":
        raise _lib.TreeAttnError(f"tree attention runs on the GPU, got device {device}")
    return device


class TreeMetaDevice:
    """Positions and subtree horizons of a DFS pre-order forest, on the GPU."""

    def __init__(self, node_len: Sequence[int], parent: Sequence[int], pos_offset: int = 0,
                 device=None, validate: bool = False):
        n = len(node_len)
        if n < 1:
            raise ValueError("empty forest")
        if validate:
            bad = preorder_violation(parent)
            if bad is not None:
                raise ValueError(f"node {bad}: parent {parent[bad]} breaks DFS pre-order")
        dev = require_device(device)
        T = int(sum(node_len))
        self.device, self.n_nodes, self.T, self.pos_offset = dev, n, T, int(pos_offset)
        i32 = dict(dtype=torch.int32, device=dev)
        lp = upload_i32([list(node_len), list(parent)], dev)
        self.node_len, self.parent = lp[0], lp[1]
        nodes = torch.empty((3, n), **i32)
        self.node_start, self.node_off, self.node_hend = nodes[0], nodes[1], nodes[2]
        toks = torch.empty((3, T), **i32)
        self.pos, self.node_of, self.horizon = toks[0], toks[1], toks[2]
        self.status = torch.zeros(1, **i32)
        ws_bytes = lib().tt_meta_workspace_bytes(n)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        rc = lib().tt_meta_build(_ptr(self.node_len), _ptr(self.parent), n, T, self.pos_offset,
                                 _ptr(self.node_start), _ptr(self.node_off), _ptr(self.node_hend),
                                 _ptr(self.pos), _ptr(self.node_of), _ptr(self.horizon), _ptr(self.status),
                                 _ptr(ws), ws_bytes, _stream(dev))
        check(rc, "tt_meta_build")
        self._ws = ws  # keep alive until the stream has consumed it
        if validate:
            self.check_status()

    def check_status(self):
        st = int(self.status.item())
        if st:
            raise ValueError(f"invalid tree metadata input (status bits {st:#x}): "
                             "node lengths must be >= 1, lengths must sum to the token count and the "
                             "parents must form a DFS pre-order (each node inside its parent's subtree range)")


def build_trees(specs, device=None, validate: bool = False):
    """Device metadata and tile plans of several trees — the partitions of a
    hybrid step — through ``tt_trees_build``: three launches per 16 trees
    instead of four per tree, one upload of all topologies, and no status
    fills (the kernel stores the status).

    ``specs``: ``(node_len, parent, pos_offset, past_bias)`` per tree, with
    ``past_bias`` a float tensor of 0 / -inf over the gateway keys, or None.
    Returns ``[(TreeMetaDevice, KeyPlan)]`` in order; both objects of a tree
    share one status word. Trees beyond the batched limits (65536 tokens,
    2048 query blocks or key tiles) are built with the separate calls."""
    dev = require_device(device)
    specs = [(list(nl), list(pa), int(po), pb) for nl, pa, po, pb in specs]
    if validate:
        for nl, pa, _, _ in specs:
            bad = preorder_violation(pa)
            if bad is not None:
                raise ValueError(f"node {bad}: parent {pa[bad]} breaks DFS pre-order")
    out = []
    small = []
    for i, (nl, pa, po, pb) in enumerate(specs):
        T = int(sum(nl))
        n_past = 0 if pb is None else int(pb.numel())
        n_qb, n_kb = -(-T // 128), -(-(T + n_past) // 128)
        if T <= 65536 and n_qb <= 2048 and n_kb <= 2048:
            small.append(i)
    built = {}
    for b in range(0, len(small), _lib.TT_TREE_JOBS_MAX):
        idx = small[b:b + _lib.TT_TREE_JOBS_MAX]
        for i, pair in zip(idx, _build_batch([specs[i] for i in idx], dev)):
            built[i] = pair
    for i, (nl, pa, po, pb) in enumerate(specs):
        if i not in built:
            meta = TreeMetaDevice(nl, pa, pos_offset=po, device=dev)
            built[i] = (meta, KeyPlan(meta.horizon, pb, topo=(nl, pa)))
        out.append(built[i])
    if validate:
        for meta, plan in out:
            meta.check_status()
    return out


def _build_batch(specs, dev):
    n = len(specs)
    lens = [len(nl) for nl, _, _, _ in specs]
    Ts = [int(sum(nl)) for nl, _, _, _ in specs]
    pasts = [0 if pb is None else int(pb.numel()) for _, _, _, pb in specs]
    topo = upload_i32(np.concatenate([np.concatenate([np.asarray(nl, np.int32), np.asarray(pa, np.int32)])
                                      for nl, pa, _, _ in specs]), dev)
    # one int32 arena: per tree 3 node rows, 3 token rows, 2 key rows and the status word
    sizes = [3 * m + 3 * T + 2 * (T + P) + 1 for m, T, P in zip(lens, Ts, pasts)]
    arena = torch.empty(int(sum(sizes)), dtype=torch.int32, device=dev)
    plan_bytes = [lib().tt_plan_bytes(T, T + P) for T, P in zip(Ts, pasts)]
    ws_bytes = [lib().tt_meta_workspace_bytes(m) for m in lens]
    al = lambda x: (x + 255) & ~255
    blob = torch.empty(int(sum(al(a) + al(b) for a, b in zip(plan_bytes, ws_bytes))), dtype=torch.uint8,
                       device=dev)
    jobs = (_lib.TTTreeJob * n)()
    out, ti, ai, bi = [], 0, 0, 0
    for j, (nl, pa, po, pb) in enumerate(specs):
        m, T, P = lens[j], Ts[j], pasts[j]
        node_len, parent = topo[ti:ti + m], topo[ti + m:ti + 2 * m]
        ti += 2 * m
        seg = arena[ai:ai + sizes[j]]
        ai += sizes[j]
        nodes = seg[:3 * m].view(3, m)
        toks = seg[3 * m:3 * m + 3 * T].view(3, T)
        keys = seg[3 * m + 3 * T:3 * m + 3 * T + 2 * (T + P)].view(2, T + P)
        status = seg[-1:]
        plan = blob[bi:bi + plan_bytes[j]]
        bi += al(plan_bytes[j])
        ws = blob[bi:bi + ws_bytes[j]]
        bi += al(ws_bytes[j])
        bias = None if pb is None else to_device(pb, dev, torch.float32)
        job = jobs[j]
        for name, t in (("node_len", node_len), ("node_parent", parent), ("past_bias", bias),
                        ("node_start", nodes[0]), ("node_off", nodes[1]), ("node_hend", nodes[2]),
                        ("pos", toks[0]), ("node_of", toks[1]), ("horizon", toks[2]), ("key_lo", keys[0]),
                        ("key_hi", keys[1]), ("status", status), ("plan", plan), ("ws", ws)):
            setattr(job, name, t.data_ptr() if t is not None else None)
        job.plan_bytes, job.ws_bytes = plan_bytes[j], ws_bytes[j]
        job.n_nodes, job.n_tokens, job.pos_offset, job.n_past = m, T, po, P
        meta = TreeMetaDevice.__new__(TreeMetaDevice)
        meta.device, meta.n_nodes, meta.T, meta.pos_offset = dev, m, T, po
        meta.node_len, meta.parent = node_len, parent
        meta.node_start, meta.node_off, meta.node_hend = nodes[0], nodes[1], nodes[2]
        meta.pos, meta.node_of, meta.horizon = toks[0], toks[1], toks[2]
        meta.status, meta._ws = status, ws
        kp = KeyPlan.__new__(KeyPlan)
        kp.device, kp.n_q, kp.n_past, kp.n_keys = dev, T, P, T + P
        kp.key_lo, kp.key_hi, kp.status = keys[0], keys[1], status
        kp.plan_bytes, kp.plan, kp._bias = plan_bytes[j], plan, bias
        kp._topo, kp._bias_src, kp._det, kp._split = (nl, pa), pb, None, None
        out.append((meta, kp))
    check(lib().tt_trees_build(jobs, n, _stream(dev)), "tt_trees_build")
    return out


class KeyPlan:
    """Per-key visibility intervals over [gateway | own] keys plus the tile plan."""

    def __init__(self, horizon: torch.Tensor, past_bias: Optional[torch.Tensor] = None,
                 validate: bool = False, topo=None):
        """``topo``: the forest's host ``(node_len, parent)``, from which
        ``det_slots`` and ``split_tiles`` size the backward's workspace exactly."""
        dev = horizon.device
        self._topo, self._bias_src, self._det, self._split = topo, past_bias, None, None
        n_q = int(horizon.numel())
        n_past = 0 if past_bias is None else int(past_bias.numel())
        if past_bias is not None:
            past_bias = to_device(past_bias, dev, torch.float32)
        self.device, self.n_q, self.n_past, self.n_keys = dev, n_q, n_past, n_q + n_past
        keys = torch.empty((2, self.n_keys), dtype=torch.int32, device=dev)
        self.key_lo, self.key_hi = keys[0], keys[1]
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        st = _stream(dev)
        check(lib().tt_keys_build(_ptr(past_bias), n_past, _ptr(horizon), n_q, _ptr(self.key_lo),
                                  _ptr(self.key_hi), _ptr(self.status), st), "tt_keys_build")
        self.plan_bytes = lib().tt_plan_bytes(n_q, self.n_keys)
        self.plan = torch.empty(self.plan_bytes, dtype=torch.uint8, device=dev)
        check(lib().tt_plan_build(_ptr(self.key_lo), _ptr(self.key_hi), self.n_keys, n_q, _ptr(self.plan),
                                  self.plan_bytes, st), "tt_plan_build")
        self._bias = past_bias
        if validate:
            s = int(self.status.item())
            if s:
                raise ValueError(f"gateway bias must be 0 or -inf (status bits {s:#x})")

    def _tree_count(self, fn: str) -> int:
        """``fn`` (tt_attn_det_slots / tt_attn_split_tiles) on the topology and
        the host copy of the gateway bias."""
        nl = np.ascontiguousarray(self._topo[0], dtype=np.int32)
        pa = np.ascontiguousarray(self._topo[1], dtype=np.int32)
        bias = None
        if self._bias_src is not None:
            bias = np.ascontiguousarray(torch.as_tensor(self._bias_src).detach().float().cpu().numpy())
        out = ctypes.c_int64(0)
        check(getattr(lib(), fn)(nl.ctypes.data, pa.ctypes.data, len(nl),
                                 bias.ctypes.data if bias is not None else None, self.n_past, ctypes.byref(out)), fn)
        return int(out.value)

    def det_slots(self) -> int:
        """Partial-sum slots of the deterministic backward for this tree
        (``tt_attn_det_slots``, host arithmetic on the topology; a gateway bias
        held on the device is copied once). 0 — the tree-independent bound —
        when the plan was built without its topology."""
        if self._det is None:
            self._det = self._tree_count("tt_attn_det_slots") if self._topo is not None else 0
        return self._det

    def split_tiles(self) -> int:
        """Key tiles whose dK/dV the backward sums in fp32 rows of its
        workspace (``tt_attn_split_tiles``, host arithmetic on the topology;
        at least 1, since 0 asks for every key tile). 0 — every key tile —
        when the plan was built without its topology, or when the gateway bias
        is held on the device only (reading it back would wait for the device
        on every backward)."""
        if self._split is None:
            on_dev = self._bias_src is not None and torch.as_tensor(self._bias_src).device.type != "cpu"
            known = self._topo is not None and not on_dev
            self._split = max(self._tree_count("tt_attn_split_tiles"), 1) if known else 0
        return self._split

    def visible_pairs(self) -> int:
        """Visible (query, key) pairs per head, P (synchronises)."""
        return int(self.plan[:8].view(torch.int64).item())

    def dense_mask(self) -> torch.Tensor:
        """[n_q, n_keys] bool expansion (compatibility / tests only)."""
        m = torch.empty((self.n_q, self.n_keys), dtype=torch.uint8, device=self.device)
        check(lib().tt_meta_dense_mask(_ptr(self.key_lo), _ptr(self.key_hi), self.n_keys, self.n_q, _ptr(m),
                                       _stream(self.device)), "tt_meta_dense_mask")
        return m.bool()
