#!/usr/bin/env python3
"""Write golden vectors of the reference block (run in the build container only).

Pins the two things no closed form fixes: the composition of
WanTransformerBlock.forward (stage order, modulation chunk order, rounding
points) and the original-mode KV cache protocol of WanAttention (slot
allocation, eviction, ids, is_pred, restore, candidate rows).

The reference module 投机采样/wam-p0-worktree/wan_va/modules/model.py cannot be
imported here (diffusers and flash_attn are absent), so this script parses it,
takes the definitions custom_sdpa, WanRotaryPosEmbed, WanAttention and
WanTransformerBlock (plus get_mesh_id from wan_va/utils/utils.py) and executes
them with two stand-ins for the diffusers 0.35 modules the block builds:
FP32LayerNorm (layer_norm on float32 input, cast back) and
FeedForward(activation_fn="gelu-approximate") (Linear, GELU tanh, Dropout,
Linear).  The fixtures therefore pin model.py's composition, not diffusers.

Outputs (data only): reference_block_tiny.safetensors and
reference_cache_tiny.safetensors next to this script.
"""
import ast
import math
import sys
from pathlib import Path

import torch
import torch.nn as nn
import torch.nn.functional as F
from einops import rearrange
from safetensors.torch import save_file

REF = Path("/root/reference/投机采样/wam-p0-worktree/wan_va")
OUT = Path(__file__).resolve().parent
SEED = 1234
DIM, HEADS, FFN = 256, 2, 512


class FP32LayerNorm(nn.LayerNorm):
    def forward(self, inputs):
        dtype = inputs.dtype
        return F.layer_norm(inputs.float(), self.normalized_shape,
                            self.weight.float() if self.weight is not None else None,
                            self.bias.float() if self.bias is not None else None, self.eps).to(dtype)


class _GELU(nn.Module):
    def __init__(self, dim_in, dim_out):
        super().__init__()
        self.proj = nn.Linear(dim_in, dim_out, bias=True)

    def forward(self, x):
        return F.gelu(self.proj(x), approximate="tanh")


class FeedForward(nn.Module):
    def __init__(self, dim, inner_dim=None, activation_fn="gelu-approximate"):
        super().__init__()
        assert activation_fn == "gelu-approximate"
        self.net = nn.ModuleList([_GELU(dim, inner_dim), nn.Dropout(0.0), nn.Linear(inner_dim, dim, bias=True)])

    def forward(self, x):
        for m in self.net:
            x = m(x)
        return x


class FlexAttnFunc(nn.Module):  # only referenced by isinstance checks here
    pass


def load_reference():
    wanted = {"custom_sdpa", "WanRotaryPosEmbed", "WanAttention", "WanTransformerBlock"}
    src = (REF / "modules" / "model.py").read_text()
    tree = ast.parse(src)
    nodes = [n for n in tree.body if isinstance(n, (ast.FunctionDef, ast.ClassDef)) and n.name in wanted]
    assert {n.name for n in nodes} == wanted, "reference definitions not found"
    util = ast.parse((REF / "utils" / "utils.py").read_text())
    nodes += [n for n in util.body if isinstance(n, ast.FunctionDef) and n.name == "get_mesh_id"]
    ns = {"torch": torch, "nn": nn, "F": F, "math": math, "rearrange": rearrange,
          "FeedForward": FeedForward, "FP32LayerNorm": FP32LayerNorm, "FlexAttnFunc": FlexAttnFunc,
          "flash_attn_func": None}
    exec(compile(ast.Module(body=nodes, type_ignores=[]), "reference_model", "exec"), ns)
    return ns


def make_block(ns, dtype):
    torch.manual_seed(SEED)
    blk = ns["WanTransformerBlock"](DIM, FFN, HEADS, cross_attn_norm=True, eps=1e-6, attn_mode="torch")
    g = torch.Generator().manual_seed(SEED)
    with torch.no_grad():
        for name, p in blk.named_parameters():
            if name.endswith("norm_q.weight") or name.endswith("norm_k.weight") or name == "norm2.weight":
                p.copy_(1 + 0.02 * torch.randn(p.shape, generator=g))
            elif name == "scale_shift_table":
                p.copy_(torch.randn(p.shape, generator=g) / DIM ** 0.5)
            else:
                p.copy_(0.02 * torch.randn(p.shape, generator=g))
    # bf16-representable values everywhere, then the model's dtype policy:
    # bf16 weights except scale_shift_table and norm2 (_keep_in_fp32_modules).
    for name, p in blk.named_parameters():
        p.data = p.data.to(torch.bfloat16).float()
    if dtype == torch.bfloat16:
        for name, p in blk.named_parameters():
            if name not in ("scale_shift_table", "norm2.weight", "norm2.bias"):
                p.data = p.data.to(torch.bfloat16)
    return blk.eval()


def inputs(ns, B, grid, Lc, seed):
    g = torch.Generator().manual_seed(seed)
    f, h, w = grid
    M = f * h * w
    x = torch.randn(B, M, DIM, generator=g).bfloat16()
    ctx = torch.randn(B, Lc, DIM, generator=g).bfloat16()
    temb = 0.1 * torch.randn(B, 1, 6, DIM, generator=g)
    rope = ns["WanRotaryPosEmbed"](DIM // HEADS, [1, 2, 2], 1024)
    grid_ids = ns["get_mesh_id"](f, h, w, 0)[None]
    freqs = rope(grid_ids)[:, :, None]
    return x, ctx, temb, freqs, grid_ids


def run(blk, x, ctx, temb, freqs, dtype, **kw):
    with torch.no_grad():
        return blk(x.to(dtype), ctx.to(dtype), temb, freqs, **kw)


def main():
    if not REF.exists():
        sys.exit(f"{REF} not found: fixtures are generated in the build container only")
    ns = load_reference()
    tensors = {}
    b32 = make_block(ns, torch.float32)
    b16 = make_block(ns, torch.bfloat16)
    for name, p in b32.named_parameters():
        keep32 = name in ("scale_shift_table", "norm2.weight", "norm2.bias")
        tensors[f"param.{name}"] = p.detach().clone() if keep32 else p.detach().to(torch.bfloat16)
    x, ctx, temb, freqs, grid_ids = inputs(ns, 1, (3, 4, 5), 16, SEED + 1)
    tensors.update({"x": x, "context": ctx, "temb": temb, "freqs": torch.view_as_real(freqs).contiguous(),
                    "grid_ids": grid_ids.float()})
    tensors["out_fp32"] = run(b32, x, ctx, temb, freqs, torch.float32)
    tensors["out_bf16"] = run(b16, x, ctx, temb, freqs, torch.bfloat16)
    save_file(tensors, str(OUT / "reference_block_tiny.safetensors"),
              metadata={"dim": str(DIM), "heads": str(HEADS), "ffn": str(FFN), "grid": "3,4,5",
                        "source": "model.py WanTransformerBlock (AST-extracted), see script"})

    # KV cache protocol, fp32 block, pool of 100 slots.
    cache_t = {}
    P = 100
    b32.attn1.init_kv_cache("pos", P, HEADS, DIM // HEADS, "cpu", torch.float32, 1)
    steps = [(2, (2, 3, 5)), (1, (2, 3, 5)), (0, (2, 3, 5)), (2, (4, 3, 5)), (1, (1, 5, 5))]
    for i, (upd, grid) in enumerate(steps):
        x, ctx, temb, freqs, _ = inputs(ns, 1, grid, 16, SEED + 10 + i)
        out = run(b32, x, ctx, temb, freqs, torch.float32, update_cache=upd, cache_name="pos")
        c = b32.attn1.attn_caches["pos"]
        cache_t.update({f"s{i}.x": x, f"s{i}.context": ctx, f"s{i}.temb": temb,
                        f"s{i}.freqs": torch.view_as_real(freqs).contiguous(), f"s{i}.out": out,
                        f"s{i}.mask": c["mask"].clone(), f"s{i}.id": c["id"].clone(),
                        f"s{i}.is_pred": c["is_pred"].clone()})
    cache_t.update({"final.k": c["k"].clone(), "final.v": c["v"].clone()})
    x, ctx, temb, freqs, _ = inputs(ns, 2, (2, 3, 5), 16, SEED + 50)
    rows = torch.zeros(2, dtype=torch.long)
    out = run(b32, x, ctx, temb, freqs, torch.float32, update_cache=0, cache_name="pos",
              candidate_cache_rows=rows)
    cache_t.update({"cand.x": x, "cand.context": ctx, "cand.temb": temb,
                    "cand.freqs": torch.view_as_real(freqs).contiguous(), "cand.rows": rows, "cand.out": out})
    save_file(cache_t, str(OUT / "reference_cache_tiny.safetensors"),
              metadata={"pool": str(P), "steps": ";".join(f"{u}:{g}" for u, g in steps)})
    print("wrote", OUT / "reference_block_tiny.safetensors", OUT / "reference_cache_tiny.safetensors")


if __name__ == "__main__":
    main()
