"""CPU pins for the GatedDeltaNet layer oracle (oracle/gdn.py
``gdn_layer_torch``) and the patch/unpatch mechanics of
tree_training_amd/gdn_layer.py.

The layer oracle is checked against transformers' own module: on every
root-to-leaf path, the stock Qwen3_5MoeGatedDeltaNet forward over the path's
tokens (float64 weights; its gated-delta-rule routine computes in float32)
equals the oracle's tree output on those tokens.
"""
import numpy as np
import pytest
import torch

from oracle import gdn as ogdn
from tree_training_amd import gdn_layer
from tree_training_amd.workloads import random_forest

pytest.importorskip("transformers.models.qwen3_5_moe.modeling_qwen3_5_moe")
from tests.gdn_layer_util import FakeModel, small_gdn_layer  # noqa: E402


def _paths(parent):
    kids = {i: [] for i in range(len(parent))}
    for i, p in enumerate(parent):
        if p >= 0:
            kids[p].append(i)
    out = []
    for i in range(len(parent)):
        if not kids[i]:
            path, j = [], i
            while j >= 0:
                path.append(j)
                j = parent[j]
            out.append(path[::-1])
    return out


def test_layer_oracle_matches_transformers_on_every_path():
    ssm = small_gdn_layer(1).double()
    lens, par = random_forest(2, node_len=(1, 9))
    T = sum(lens)
    h = torch.randn(T, 256, dtype=torch.float64, generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        y = ogdn.gdn_layer_torch(ssm, h, lens, par)
        starts = np.concatenate([[0], np.cumsum(lens)[:-1]])
        for path in _paths(par):
            idx = torch.from_numpy(np.concatenate([np.arange(starts[i], starts[i] + lens[i]) for i in path]))
            y_path = ssm(h[idx][None])[0]
            err = float((y_path - y[idx]).abs().max() / y[idx].abs().max())
            assert err < 1e-5, (path, err)


def test_patch_and_unpatch_restore_forward():
    ssm = small_gdn_layer(0)
    model = FakeModel(ssm)
    bounds, par = [(0, 3), (3, 5)], [-1, 0]
    saved = gdn_layer._patch_ssm(model, bounds, par)
    assert list(saved) == [ssm] and "forward" in ssm.__dict__
    gdn_layer._unpatch_ssm(saved)
    assert "forward" not in ssm.__dict__            # the class method again
    # accelerate-style hooks keep the original in _old_forward: that is patched
    orig = ssm.forward
    ssm._old_forward = orig
    saved = gdn_layer.patch_ssm_for_dfs(model, bounds, par)
    assert saved[ssm][0] == "_old_forward" and ssm._old_forward is not orig
    gdn_layer.unpatch_ssm(saved)
    assert ssm._old_forward is orig
