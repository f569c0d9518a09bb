"""A small transformers Qwen3.5-MoE GatedDeltaNet layer (head dims 128, the
size the kernels are built for) for the layer-patch tests."""
import torch

from transformers.models.qwen3_5_moe import configuration_qwen3_5_moe as qcfg
from transformers.models.qwen3_5_moe import modeling_qwen3_5_moe as qmod


def small_gdn_layer(seed=0, hidden=256, hv=4, hk=2, k=4):
    cfg = qcfg.Qwen3_5MoeTextConfig(
        hidden_size=hidden, linear_num_value_heads=hv, linear_num_key_heads=hk, linear_key_head_dim=128,
        linear_value_head_dim=128, linear_conv_kernel_dim=k, num_hidden_layers=2,
        layer_types=["linear_attention", "full_attention"], num_attention_heads=4, num_key_value_heads=2,
        head_dim=128, vocab_size=64, num_experts=4, num_experts_per_tok=2, moe_intermediate_size=64,
        shared_expert_intermediate_size=64)
    torch.manual_seed(seed)
    layer = qmod.Qwen3_5MoeGatedDeltaNet(cfg, 0)
    with torch.no_grad():                      # non-trivial norm weight and decay
        layer.norm.weight.uniform_(0.5, 1.5)
        layer.dt_bias.uniform_(-1.0, 1.0)
    return layer


class FakeModel(torch.nn.Module):
    """model.model.layers[i].linear_attn, the structure the patch walks."""

    def __init__(self, ssm):
        super().__init__()
        layer = torch.nn.Module()
        layer.linear_attn = ssm
        self.model = torch.nn.Module()
        self.model.layers = torch.nn.ModuleList([layer, torch.nn.Module()])


def small_hybrid_model(seed=0):
    """A two-layer Qwen3.5-MoE text model: one gated-delta-rule layer, one
    full-attention layer (head_dim 128, GQA 4/2), vocabulary 64."""
    cfg = qcfg.Qwen3_5MoeTextConfig(
        hidden_size=256, linear_num_value_heads=4, linear_num_key_heads=2, linear_key_head_dim=128,
        linear_value_head_dim=128, linear_conv_kernel_dim=4, num_hidden_layers=2,
        layer_types=["linear_attention", "full_attention"], num_attention_heads=4, num_key_value_heads=2,
        head_dim=128, vocab_size=64, num_experts=4, num_experts_per_tok=2, moe_intermediate_size=64,
        shared_expert_intermediate_size=64)
    cfg._attn_implementation = "eager"
    cfg._experts_implementation = "eager"      # plain per-expert matmuls (any dtype, float64 included)
    torch.manual_seed(seed)
    model = qmod.Qwen3_5MoeForCausalLM(cfg)
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, qmod.Qwen3_5MoeGatedDeltaNet):
                m.norm.weight.uniform_(0.5, 1.5)
                m.dt_bias.uniform_(-1.0, 1.0)
    return model.eval()


def strong_recurrence(model, seed=0):
    """Makes every GatedDeltaNet layer's keys nearly parallel (a rank-one key
    projection plus 2 % of the random one) and its decay slow (dt_bias -4),
    so that the delta rule's within-node correction T = (I - N)^-1 has large
    higher powers: the reference's truncation I + R + R^2 then moves the leaf
    logits by ~1e-3 on the c1 forest instead of ~1e-7."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, qmod.Qwen3_5MoeGatedDeltaNet):
                W, kd = m.in_proj_qkv.weight, m.key_dim
                u = torch.randn(kd, 1, generator=g).to(W.dtype)
                v = torch.randn(1, W.shape[1], generator=g).to(W.dtype)
                W[kd:2 * kd] = 0.2 * (u @ v) / W.shape[1] ** 0.5 + 0.02 * W[kd:2 * kd]
                m.dt_bias.fill_(-4.0)
                m.in_proj_b.weight.mul_(0.1)
    return model
