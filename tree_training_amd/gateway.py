"""Gateway KV between partitions — drop-in for ``GatewayCache``.

``GatewayCache`` keeps the HF-Cache duck type of tree_grad_ckpt_opath.py:66-195
(``update``, ``get_seq_length``, ``get_mask_sizes``, ``_full_kv``). Under the tree-attention implementation it runs in
*segmented* mode: ``update`` records the gateway and the new K/V as two segments
and returns the new K/V unchanged; the attention kernel reads both segments in
place, so the per-layer ``cat`` of the reference never happens.
``_full_kv[layer]`` still yields the concatenation (built on access) for
callers that read it.

``GatewayAccumulator`` is the device-side replacement of the fp32 gradient
hooks (tree_grad_hybrid.py:220-225): the attention backward adds the gateway
gradients into it in float32, with no host round trip.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Tuple

import torch


class GatewayAccumulator:
    """fp32 gradient sums for one layer's gateway K and V ([Lp, Hkv, D] each)."""

    def __init__(self, like: torch.Tensor):
        _, hkv, lp, d = like.shape
        self.k = torch.zeros((lp, hkv, d), dtype=torch.float32, device=like.device)
        self.v = torch.zeros((lp, hkv, d), dtype=torch.float32, device=like.device)
        self.touched = False

    def as_hf(self, which: str) -> torch.Tensor:
        """The sum in the [1, Hkv, Lp, D] layout of the gateway tensors."""
        t = self.k if which == "k" else self.v
        return t.unsqueeze(0).transpose(1, 2)


class _LazyFullKV(dict):
    """layer -> (cat(gate_k, k), cat(gate_v, v)), concatenated on first access."""

    def __init__(self, segments):
        super().__init__()
        self._segments = segments

    def __contains__(self, layer):
        return layer in self._segments

    def keys(self):
        return self._segments.keys()

    def __len__(self):
        return len(self._segments)

    def __iter__(self):
        return iter(self._segments)

    def __getitem__(self, layer):
        if not dict.__contains__(self, layer):
            gk, gv, k, v = self._segments[layer]
            if gk is None:
                dict.__setitem__(self, layer, (k, v))
            else:
                dict.__setitem__(self, layer, (torch.cat([gk, k], dim=-2), torch.cat([gv, v], dim=-2)))
        return dict.__getitem__(self, layer)


class GatewayCache:
    """Per-layer gateway KV (detached leaves [1, Hkv, past, D]) in front of a
    partition's own KV (tree_grad_ckpt_opath.py:66-133)."""

    def __init__(self, gate_kv: List[Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]],
                 segmented: bool = False):
        self._gate_kv = list(gate_kv)
        self.segmented = segmented
        self._segments: Dict[int, tuple] = {}
        self._full_kv = _LazyFullKV(self._segments) if segmented else {}

    # -- HF Cache interface -------------------------------------------------
    def gate(self, layer_idx: int):
        if layer_idx < len(self._gate_kv):
            return self._gate_kv[layer_idx]
        return (None, None)

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs: Optional[dict] = None):
        gk, gv = self.gate(layer_idx)
        if self.segmented:
            self._segments[layer_idx] = (gk, gv, key_states, value_states)
            return key_states, value_states
        if gk is not None:
            full_k = torch.cat([gk, key_states], dim=-2)
            full_v = torch.cat([gv, value_states], dim=-2)
        else:
            full_k, full_v = key_states, value_states
        self._full_kv[layer_idx] = (full_k, full_v)
        return full_k, full_v

    def own_kv(self, layer_idx: int):
        """(k, v) of the partition's own tokens for a layer (segmented mode)."""
        return self._segments[layer_idx][2], self._segments[layer_idx][3]

    def get_seq_length(self, layer_idx: int = 0) -> int:
        gk, _ = self.gate(layer_idx)
        return 0 if gk is None else gk.shape[-2]

    def get_mask_sizes(self, query, layer_idx: int = 0):
        """(kv_length, kv_offset); accepts the query length or a cache_position tensor."""
        q_len = query.shape[0] if isinstance(query, torch.Tensor) else int(query)
        return self.get_seq_length(layer_idx) + q_len, 0

    def get_query_offset(self, layer_idx: int = 0) -> int:
        return self.get_seq_length(layer_idx)

    @property
    def is_compileable(self) -> bool:
        return False
