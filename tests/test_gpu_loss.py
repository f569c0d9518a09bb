"""GPU parity of the fused leaf loss: the row-wise cross-entropy kernel
(tt_ce_rows) and the chunked lm_head + CE (loss.fused_linear_ce) against
torch's cross_entropy in float64 (library), and the drivers' fused path
(make_tree_loss_fn losses) against the float64 oracle model run.

Bars: float32 max_rel < 1e-5 (loss, logit gradient, hidden and weight
gradients, model parameter gradients); bf16 < 2e-2.
"""
import copy

import pytest
import torch
import torch.nn.functional as F

from oracle.attention import max_rel
from oracle.model_path import sequential_param_grads
from tests.test_gpu_drivers import _grads, _labels, _max_rel_params, _tree
from tests.conftest import make_qwen3
from tree_training_amd.loss import ce_rows, fused_linear_ce

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _rel(a, b):
    return float((a.double() - b.double()).abs().max() / b.double().abs().max().clamp_min(1e-30))


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("N,V,ld", [(37, 1000, 1000), (5, 1001, 1008), (3, 151936, 151936)])
def test_ce_rows_matches_torch(dtype, tol, N, V, ld):
    g = torch.Generator().manual_seed(N + V)
    x = torch.randn(N, ld, generator=g) * 3.0
    labels = torch.randint(0, V, (N,), generator=g)
    labels[1] = -100                                        # ignored row
    scale = torch.rand(N, generator=g) + 0.5
    xd = x.to(DEV, dtype)
    print(f"ce_rows {dtype} N={N} V={V} ld={ld}", flush=True)
    loss = ce_rows(xd[:, :V], labels.to(DEV), scale.to(DEV))
    torch.cuda.synchronize()
    ref_x = x.to(dtype)[:, :V].double().requires_grad_(True)    # xd now holds the gradient
    per = F.cross_entropy(ref_x, labels, ignore_index=-100, reduction="none") * scale.double()
    (gx,) = torch.autograd.grad(per.sum(), ref_x)
    assert _rel(loss.cpu(), per.detach()) < tol
    assert _rel(xd[:, :V].cpu(), gx) < tol                  # the gradient replaced the logits in place
    assert not xd[1, :V].any()                              # the ignored row's gradient is zero


def test_ce_rows_bad_label_gives_nan_not_a_fault():
    x = torch.randn(2, 1000, device=DEV)
    loss = ce_rows(x, torch.tensor([5, 1000], device=DEV), torch.ones(2, device=DEV))
    torch.cuda.synchronize()
    assert torch.isfinite(loss[0]) and torch.isnan(loss[1])


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_fused_linear_ce_matches_torch(dtype, tol):
    g = torch.Generator().manual_seed(0)
    N, H, V = 300, 256, 1000
    h = torch.randn(N, H, generator=g)
    w = torch.randn(V, H, generator=g) * 0.05
    labels = torch.randint(0, V, (N,), generator=g)
    labels[::17] = -100
    scale = torch.full((N,), 1.0 / 7.0)
    hd = h.to(DEV, dtype).requires_grad_(True)
    wd = w.to(DEV, dtype).requires_grad_(True)
    loss = fused_linear_ce(hd, wd, labels.to(DEV), scale.to(DEV), chunk=128)   # 3 chunks, the last ragged
    loss.backward(torch.tensor(2.0, device=DEV))
    hr = hd.detach().double().cpu().requires_grad_(True)
    wr = wd.detach().double().cpu().requires_grad_(True)
    ref = (F.cross_entropy(hr @ wr.t(), labels, ignore_index=-100, reduction="none") * scale.double()).sum()
    ref.backward(torch.tensor(2.0, dtype=torch.float64))
    assert _rel(loss.detach().cpu(), ref.detach()) < tol
    assert _rel(hd.grad.cpu(), hr.grad) < tol
    assert _rel(wd.grad.cpu(), wr.grad) < tol


@pytest.mark.parametrize("driver", ["sequential", "hybrid"])
def test_drivers_fused_leaf_ce_fp32(driver):
    """make_tree_loss_fn losses take the hidden-state path (no [T, V] logits)
    and still give the oracle's parameter gradients."""
    from tree_training_amd.ckpt import make_tree_loss_fn, tree_grad_ckpt_sequential
    from tree_training_amd.hybrid import tree_grad_hybrid
    print(f"fused leaf CE through {driver}", flush=True)
    base = make_qwen3("tiny", layers=2)
    ref_model = copy.deepcopy(base).double()
    model = base.to(DEV)
    roots, leaves = _tree("c1")
    labels = _labels(leaves)
    ref = sequential_param_grads(ref_model, roots, labels, len(leaves))
    fn = make_tree_loss_fn([labels[id(n)] for n in leaves], leaves, len(leaves))
    if driver == "sequential":
        new = _grads(model, lambda: tree_grad_ckpt_sequential(model, roots, fn))
    else:
        new = _grads(model, lambda: tree_grad_hybrid(model, roots, fn, 20, summed_backward=True))
    r = _max_rel_params(ref, new)
    print(f"  max_rel {r:.3e}", flush=True)
    assert r < 1e-5, r


def test_tree_ce_loss_fused_spans_equals_per_leaf_losses():
    """TreeCELoss.fused_spans == the sum of the reference-semantics per-leaf
    losses (F.cross_entropy mean over valid tokens / n_leaves), values and
    gradients (fp32)."""
    from tree_training_amd.loss import TreeCELoss
    g = torch.Generator().manual_seed(1)
    T, H, V = 90, 64, 1000
    spans = [(0, 7), (7, 30), (41, 90)]
    nodes = [object() for _ in spans]
    labels = [torch.randint(0, V, (e - s,), generator=g) for s, e in spans]
    labels[1][::3] = -100
    fn = TreeCELoss(labels, nodes, 5)
    h = torch.randn(T, H, generator=g).to(DEV).requires_grad_(True)
    w = (torch.randn(V, H, generator=g) * 0.1).to(DEV).requires_grad_(True)
    a = fn.fused_spans(h, [(s, e, n) for (s, e), n in zip(spans, nodes)], w)
    ga = torch.autograd.grad(a, (h, w))
    logits = (h @ w.t())[None]
    b = sum(fn(logits[:, s:e, :], n) for (s, e), n in zip(spans, nodes))
    gb = torch.autograd.grad(b, (h, w))
    assert _rel(a.detach(), b.detach()) < 1e-5
    assert _rel(ga[0], gb[0]) < 1e-5 and _rel(ga[1], gb[1]) < 1e-5
