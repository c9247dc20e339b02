"""Synthetic MoE inputs of BASELINE.json's distributions (numpy)."""
import numpy as np

from molten_amd import layout


def moe_weights(rng, n_experts: int, d_model: int, n_inter: int, bits: int = 4):
    """Stacked experts: gate/up [E*I, H], down [E*H, I], MLX Q4 group 64."""
    gate = layout.synth_quant(rng, n_experts * n_inter, d_model, bits)
    up = layout.synth_quant(rng, n_experts * n_inter, d_model, bits)
    down = layout.synth_quant(rng, n_experts * d_model, n_inter, bits)
    return gate, up, down


def router_weights(rng, n_experts: int, d_model: int, f32: bool = False):
    w = rng.normal(0, 0.02, (n_experts, d_model)).astype(np.float32)
    return w if f32 else layout.f32_to_bf16(w)
