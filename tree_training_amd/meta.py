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


class KeyPlan:
    """Per-key visibility intervals over [gateway | own] keys plus the tile plan."""

    def __init__(self, horizon: torch.Tensor, past_bias: Optional[torch.Tensor] = None,
                 validate: bool = False):
        dev = horizon.device
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

    def visible_pairs(self) -> int:
        """Visible (query, key) pairs per head, P (synchronises)."""
        return int(self.plan[:8].view(torch.int64).item())

    def dense_mask(self) -> torch.Tensor:
        """[n_q, n_keys] bool expansion (compatibility / tests only)."""
        m = torch.empty((self.n_q, self.n_keys), dtype=torch.uint8, device=self.device)
        check(lib().tt_meta_dense_mask(_ptr(self.key_lo), _ptr(self.key_hi), self.n_keys, self.n_q, _ptr(m),
                                       _stream(self.device)), "tt_meta_dense_mask")
        return m.bool()
