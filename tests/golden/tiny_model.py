"""The tiny Wan DiT model of the model-level fixtures: configuration, seeded
parameters and inputs.

Parameters are not stored in the fixture: each one is regenerated from its
name (sorted order, one CPU generator per parameter), so the fixture holds
only inputs and outputs.  Every value is bf16-representable.
"""
import math

import torch

SEED = 4321
CONFIG = dict(patch_size=(1, 2, 2), num_attention_heads=2, attention_head_dim=128, in_channels=48,
              out_channels=48, action_dim=30, text_dim=128, freq_dim=256, ffn_dim=512, num_layers=2,
              cross_attn_norm=True, eps=1e-6)
DIM = CONFIG["num_attention_heads"] * CONFIG["attention_head_dim"]
FP32_NAMES = ("scale_shift_table", "norm2.weight", "norm2.bias")


def param_value(name, shape, index):
    g = torch.Generator().manual_seed(SEED * 1000 + index)
    n = torch.randn(shape, generator=g)
    if name.endswith(("norm_q.weight", "norm_k.weight", "norm2.weight")):
        v = 1 + 0.02 * n
    elif name.endswith("scale_shift_table"):
        v = n / math.sqrt(DIM)
    else:
        v = 0.02 * n
    return v.to(torch.bfloat16).float()


def make_params(shapes):
    """{name: shape} -> {name: fp32 tensor}, generated in sorted-name order."""
    return {name: param_value(name, shapes[name], i) for i, name in enumerate(sorted(shapes))}


def video_inputs(get_mesh_id, B=2, F=2, H=8, W=10, Lc=16, f_shift=3):
    g = torch.Generator().manual_seed(SEED + 1)
    c = CONFIG
    latents = torch.randn(B, c["in_channels"], F, H, W, generator=g).bfloat16().float()
    text = torch.randn(B, Lc, c["text_dim"], generator=g).bfloat16().float()
    p = c["patch_size"]
    grid = get_mesh_id(F // p[0], H // p[1], W // p[2], 0, 1, f_shift)[None].repeat(B, 1, 1)
    t = torch.tensor([[0.0, 812.5], [0.0, 377.25]])[:B, :F]
    return {"noisy_latents": latents, "text_emb": text, "grid_id": grid, "timesteps": t}


def action_inputs(get_mesh_id, B=2, F=2, H=4, W=1, Lc=16, f_shift=3):
    g = torch.Generator().manual_seed(SEED + 2)
    c = CONFIG
    latents = torch.randn(B, c["action_dim"], F, H, W, generator=g).bfloat16().float()
    text = torch.randn(B, Lc, c["text_dim"], generator=g).bfloat16().float()
    grid = get_mesh_id(F, H, W, 1, 1, f_shift, action=True)[None].repeat(B, 1, 1)
    t = torch.tensor([[0.0, 640.0], [0.0, 99.5]])[:B, :F]
    return {"noisy_latents": latents, "text_emb": text, "grid_id": grid, "timesteps": t}
