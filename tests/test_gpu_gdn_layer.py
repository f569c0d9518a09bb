"""GPU parity of the patched GatedDeltaNet layer (tree conv + tree scan
kernels, torch projections and norm) against the float64 layer oracle
(oracle/gdn.py ``gdn_layer_torch``, pinned to transformers' module per path
in tests/test_gdn_layer.py): forward output and the gradients with respect to
the input and every parameter, with the exact scan and with the reference's
own I + R + R^2 scan (reference_truncated).

Bars: float32 max_rel < 1e-5 per tensor; bf16 < 2e-2. With the reference's
node-by-node projections (per_node_projections, tree_dfs_ssm.py:369-373,
416-428) the same bars hold, and the bf16 tree output equals a run of each
root-to-leaf path alone, bit for bit (the reference's "exact 0 alignment").
"""
import numpy as np
import pytest
import torch

from oracle import gdn as ogdn
from tree_training_amd import gdn_layer
from tree_training_amd.workloads import random_forest

pytestmark = pytest.mark.gpu
pytest.importorskip("transformers.models.qwen3_5_moe.modeling_qwen3_5_moe")
from tests.gdn_layer_util import small_gdn_layer  # noqa: E402

DEV = torch.device("cuda", 0)


def _rel(a, b):
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


@pytest.mark.parametrize("reference_truncated,per_node", [(False, False), (True, False), (False, True)],
                         ids=["exact", "reference", "exact-per-node"])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_patched_layer_matches_oracle(dtype, tol, reference_truncated, per_node):
    lens, par = random_forest(5, node_len=(1, 45))
    T = sum(lens)
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]])
    bounds = [(int(s), int(s + n)) for s, n in zip(starts, lens)]
    ssm = small_gdn_layer(2)
    ref_ssm = small_gdn_layer(2).double()
    ssm = ssm.to(DEV, dtype)
    h64 = torch.randn(T, 256, dtype=torch.float64, generator=torch.Generator().manual_seed(4))
    if dtype == torch.bfloat16:      # the oracle sees the same rounded weights and input
        with torch.no_grad():
            for p_ref, p in zip(ref_ssm.parameters(), ssm.parameters()):
                p_ref.copy_(p.double().cpu())
        h64 = h64.bfloat16().double()
    dy64 = torch.randn(T, 256, dtype=torch.float64, generator=torch.Generator().manual_seed(5))
    print(f"gdn layer {dtype} reference_truncated={reference_truncated}: T={T} nodes={len(lens)}", flush=True)

    fwd = gdn_layer._make_dfs_ssm_forward(ssm, bounds, par, reference_truncated=reference_truncated,
                                          per_node_projections=per_node)
    h = h64.to(DEV, dtype).requires_grad_(True)
    y = fwd(h[None])[0]
    y.backward(dy64.to(DEV, dtype))

    hr = h64.clone().requires_grad_(True)
    yr = ogdn.gdn_layer_torch(ref_ssm, hr, lens, par, reference_truncated)
    yr.backward(dy64)

    assert _rel(y.detach().double().cpu(), yr.detach()) < tol
    assert _rel(h.grad.double().cpu(), hr.grad) < tol, "d hidden"
    for (name, p), p_ref in zip(ssm.named_parameters(), ref_ssm.parameters()):
        assert _rel(p.grad.double().cpu(), p_ref.grad) < tol, name


@pytest.mark.parametrize("reference_truncated", [False, True], ids=["exact", "reference"])
def test_per_node_projections_give_per_path_outputs_bitwise(reference_truncated):
    """bf16, node-by-node projections: the tree output on every root-to-leaf
    path equals, bit for bit, the same layer run on that path alone (its
    nodes as a chain): the projections, norm and out_proj see the same GEMM
    shapes, and the conv and scan are per-path exact."""
    lens, par = random_forest(6, node_len=(1, 60))
    T = sum(lens)
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]])
    ssm = small_gdn_layer(3).to(DEV, torch.bfloat16)
    h = torch.randn(T, 256, generator=torch.Generator().manual_seed(6)).to(DEV, torch.bfloat16)
    bounds = [(int(s), int(s + n)) for s, n in zip(starts, lens)]
    print(f"gdn layer per-path bitwise reference_truncated={reference_truncated}: T={T} nodes={len(lens)}",
          flush=True)
    with torch.no_grad():
        y = gdn_layer._make_dfs_ssm_forward(ssm, bounds, par, reference_truncated=reference_truncated,
                                            per_node_projections=True)(h[None])[0]
        kids = set(par)
        for leaf in [i for i in range(len(lens)) if i not in kids]:
            path, j = [], leaf
            while j >= 0:
                path.append(j)
                j = par[j]
            path = path[::-1]
            idx = torch.from_numpy(np.concatenate([np.arange(starts[i], starts[i] + lens[i]) for i in path])).to(DEV)
            plens = [lens[i] for i in path]
            pst = np.concatenate([[0], np.cumsum(plens)[:-1]])
            pb = [(int(s), int(s + n)) for s, n in zip(pst, plens)]
            yp = gdn_layer._make_dfs_ssm_forward(ssm, pb, list(range(-1, len(path) - 1)),
                                                 reference_truncated=reference_truncated,
                                                 per_node_projections=True)(h[idx][None])[0]
            assert torch.equal(yp, y[idx]), (leaf, path)
