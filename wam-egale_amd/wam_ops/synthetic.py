"""Seeded synthetic parameters and inputs for the Wan DiT block workloads.

Distributions: projection weights N(0, 0.02), biases N(0, 0.02); RMSNorm
weights N(1, 0.02); norm2 weight N(1, 0.02) and bias N(0, 0.02) in fp32;
scale_shift_table N(0, 1)/sqrt(D) in fp32 (model.py:738-739); hidden states and
context N(0, 1) in bf16; timestep modulation temb N(0, 0.1) in fp32.  Every
tensor has its own generator seeded from (seed, tensor index), so a workload
is reproducible on any device.

The 3D RoPE frequencies use the model's construction (grid ids from
utils.get_mesh_id, WanRotaryPosEmbed base frequencies, model.py:243-286).
"""
from dataclasses import dataclass
import math

import torch


@dataclass(frozen=True)
class BlockShape:
    dim: int = 3072
    heads: int = 24
    ffn: int = 14336
    eps: float = 1e-6
    cross_attn_norm: bool = True

    @property
    def head_dim(self):
        return self.dim // self.heads


WAN22_5B = BlockShape(3072, 24, 14336)
WAN_1_3B = BlockShape(1536, 12, 8960)

PARAM_NAMES = (
    "scale_shift_table", "norm2.weight", "norm2.bias",
    *(f"{a}.{m}.{t}" for a in ("attn1", "attn2")
      for m in ("to_q", "to_k", "to_v", "to_out.0") for t in ("weight", "bias")),
    "attn1.norm_q.weight", "attn1.norm_k.weight", "attn2.norm_q.weight", "attn2.norm_k.weight",
    "ffn.net.0.proj.weight", "ffn.net.0.proj.bias", "ffn.net.2.weight", "ffn.net.2.bias",
)


def _gen(device, seed, index):
    g = torch.Generator(device=device)
    g.manual_seed((seed * 1000003 + index * 7919) % (2 ** 63))
    return g


def _normal(shape, mean, std, device, seed, index, dtype):
    g = _gen(device, seed, index)
    t = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    return (t * std + mean).to(dtype)


def block_params(shape: BlockShape, seed=0, device="cpu", dtype=torch.bfloat16, bias_std=0.02):
    """state_dict-named parameters of one block."""
    D, F_ = shape.dim, shape.ffn
    p = {}
    for i, name in enumerate(PARAM_NAMES):
        if name == "scale_shift_table":
            p[name] = _normal((1, 6, D), 0.0, 1.0 / math.sqrt(D), device, seed, i, torch.float32)
        elif name == "norm2.weight":
            p[name] = _normal((D,), 1.0, 0.02, device, seed, i, torch.float32)
        elif name == "norm2.bias":
            p[name] = _normal((D,), 0.0, 0.02, device, seed, i, torch.float32)
        elif "norm_" in name:
            p[name] = _normal((D,), 1.0, 0.02, device, seed, i, dtype)
        elif name.startswith("ffn.net.0.proj"):
            sh = (F_, D) if name.endswith("weight") else (F_,)
            p[name] = _normal(sh, 0.0, 0.02 if name.endswith("weight") else bias_std, device, seed, i, dtype)
        elif name.startswith("ffn.net.2"):
            sh = (D, F_) if name.endswith("weight") else (D,)
            p[name] = _normal(sh, 0.0, 0.02 if name.endswith("weight") else bias_std, device, seed, i, dtype)
        else:
            sh = (D, D) if name.endswith("weight") else (D,)
            p[name] = _normal(sh, 0.0, 0.02 if name.endswith("weight") else bias_std, device, seed, i, dtype)
    if not shape.cross_attn_norm:
        del p["norm2.weight"], p["norm2.bias"]
    return p


def model_io_params(model, seed=0, device="cpu", dtype=torch.bfloat16):
    """state_dict-named values for every model parameter outside the blocks:
    N(0, 0.02) weights and biases, fp32 for time_embedder (the model's
    _keep_in_fp32_modules, model.py:809-821) and `dtype` otherwise;
    scale_shift_table N(0, 1)/sqrt(D) in fp32 (model.py:878-879)."""
    p = {}
    for i, (name, prm) in enumerate(sorted(model.named_parameters())):
        if name.startswith("blocks."):
            continue
        if name == "scale_shift_table":
            p[name] = _normal(tuple(prm.shape), 0.0, 1.0 / math.sqrt(prm.shape[-1]), device, seed, 500 + i,
                              torch.float32)
        elif "time_embedder" in name:
            p[name] = _normal(tuple(prm.shape), 0.0, 0.02, device, seed, 500 + i, torch.float32)
        else:
            p[name] = _normal(tuple(prm.shape), 0.0, 0.02, device, seed, 500 + i, dtype)
    return p


def mesh_grid_ids(f, h, w):
    """[3, f*h*w] (frame, row, col) ids in raster order (utils.get_mesh_id)."""
    ff, hh, ww = torch.meshgrid(torch.arange(f), torch.arange(h), torch.arange(w), indexing="ij")
    return torch.stack([ff.flatten(), hh.flatten(), ww.flatten()]).double()


def rope_freqs(grid, head_dim=128, theta=10000.0):
    """complex64 [1, L, 1, head_dim/2] for grid ids [3, L]."""
    f_dim = head_dim - 2 * (head_dim // 3)
    hw_dim = head_dim // 3

    def base(dim):
        return 1.0 / (theta ** (torch.arange(0, dim, 2)[: dim // 2].double() / dim))
    ang = torch.cat([grid[0][:, None] * base(f_dim), grid[1][:, None] * base(hw_dim),
                     grid[2][:, None] * base(hw_dim)], dim=-1).float()
    return torch.polar(torch.ones_like(ang), ang)[None, :, None]


def block_inputs(shape: BlockShape, batch, tokens, grid, context_len=512, context_batch=1,
                 seed=1, device="cpu", per_token_temb=False):
    """x [B, M, D] bf16, context [Bc, Lc, D] bf16, temb [B, 1|M, 6, D] fp32,
    rotary_emb complex64 [1, M, 1, hd/2] from a (f, h, w) grid with f*h*w == M."""
    D = shape.dim
    f, h, w = grid
    assert f * h * w == tokens, "grid must cover the tokens"
    x = _normal((batch, tokens, D), 0.0, 1.0, device, seed, 100, torch.bfloat16)
    ctx = _normal((context_batch, context_len, D), 0.0, 1.0, device, seed, 101, torch.bfloat16)
    L = tokens if per_token_temb else 1
    temb = _normal((batch, L, 6, D), 0.0, 0.1, device, seed, 102, torch.float32)
    freqs = rope_freqs(mesh_grid_ids(f, h, w), shape.head_dim).to(device)
    return x, ctx, temb, freqs


def kv_pool(shape: BlockShape, pool, prefix, batch=1, seed=3, device="cpu", dtype=torch.bfloat16):
    """An original-mode pool with `prefix` valid slots holding N(0, 1) K/V rows,
    committed as chunk ids 0.. in one id (an observation chunk)."""
    H, hd = shape.heads, shape.head_dim
    k = _normal((batch, pool, H, hd), 0.0, 1.0, device, seed, 200, dtype)
    v = _normal((batch, pool, H, hd), 0.0, 1.0, device, seed, 201, dtype)
    ids = torch.full((pool,), -1, dtype=torch.int64, device=device)
    mask = torch.zeros(pool, dtype=torch.bool, device=device)
    ids[:prefix] = 0
    mask[:prefix] = True
    return {"k": k, "v": v, "id": ids, "mask": mask,
            "is_pred": torch.zeros(pool, dtype=torch.bool, device=device)}
