"""Pins for the attention-prologue oracle (oracle/prologue.py), CPU only:
against transformers' Qwen3RMSNorm and apply_rotary_pos_emb (library), values
and gradients. Qwen3RMSNorm normalises in float32 whatever the input dtype, so
the agreement is to float32 rounding (relative 1e-6)."""
import pytest
import torch

from oracle.prologue import qk_prologue

qm = pytest.importorskip("transformers.models.qwen3.modeling_qwen3")


def test_prologue_matches_transformers_values_and_grads():
    g = torch.Generator().manual_seed(0)
    T, H, D = 11, 3, 128
    x = torch.randn(T, H, D, dtype=torch.float64, generator=g).requires_grad_(True)
    w = (torch.rand(D, dtype=torch.float64, generator=g) + 0.5).requires_grad_(True)
    pos = torch.tensor([0, 1, 2, 3, 2, 3, 4, 1, 7, 5, 9])
    inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    f = pos[:, None].double() * inv[None]
    emb = torch.cat([f, f], dim=-1)
    cos, sin = emb.cos(), emb.sin()

    norm = qm.Qwen3RMSNorm(D, eps=1e-6).double()
    with torch.no_grad():
        norm.weight.copy_(w)
    ref, _ = qm.apply_rotary_pos_emb(norm(x).transpose(0, 1)[None], norm(x).transpose(0, 1)[None],
                                     cos[None], sin[None])
    ref = ref[0].transpose(0, 1)
    out = qk_prologue(x, w, 1e-6, cos, sin)
    rel = lambda a, b: float((a - b).abs().max() / b.abs().max())
    assert rel(out, ref) < 1e-6
    dy = torch.randn(T, H, D, dtype=torch.float64, generator=g)
    gx, gw = torch.autograd.grad((out * dy).sum(), (x, w))
    rx, rw = torch.autograd.grad((ref * dy).sum(), (x, norm.weight))
    assert rel(gx, rx) < 1e-6
    assert rel(gw, rw) < 1e-6
