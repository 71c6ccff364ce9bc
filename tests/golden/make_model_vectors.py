#!/usr/bin/env python3
"""Write golden vectors of the reference model forward (build container only).

Pins what no closed form fixes at the model level: the composition of
WanTransformer3DModel.forward (patch / action embedding, text embedder, RoPE
from grid ids, per-frame timesteps repeated over tokens, the condition
embedder, the block loop, norm_out with the scale_shift_table + temb
modulation, proj_out and the unpatchify rearrange) for the video path and the
action path.

The reference module 投机采样/wam-p0-worktree/wan_va/modules/model.py cannot be
imported here (diffusers and flash_attn are absent).  This script parses it,
takes custom_sdpa, WanTimeTextImageEmbedding, WanRotaryPosEmbed, WanAttention,
WanTransformerBlock and WanTransformer3DModel (plus get_mesh_id from
wan_va/utils/utils.py) and executes them with stand-ins for the diffusers
0.36.0 pieces (requirements.txt:4) restated from their published definitions:
ModelMixin / ConfigMixin / register_to_config (plain nn.Module), Timesteps
(get_timestep_embedding), TimestepEmbedding (Linear, SiLU, Linear),
PixArtAlphaTextProjection (Linear, GELU tanh, Linear), FP32LayerNorm and
FeedForward("gelu-approximate").  The fixture therefore pins model.py's
composition; the sinusoid itself is pinned by closed forms in
tests/test_oracle.py.

Everything runs in float32.  Parameters are regenerated from tiny_model.py;
the fixture (reference_model_tiny.safetensors) holds inputs and outputs only.
"""
import ast
import math
import sys
from copy import deepcopy
from pathlib import Path

import torch
import torch.nn as nn
import torch.nn.functional as F
from einops import rearrange
from safetensors.torch import save_file

sys.path.insert(0, str(Path(__file__).resolve().parent))
import tiny_model  # noqa: E402
from make_reference_vectors import FeedForward, FlexAttnFunc, FP32LayerNorm  # noqa: E402

REF = Path("/root/reference/投机采样/wam-p0-worktree/wan_va")
OUT = Path(__file__).resolve().parent


class ModelMixin(nn.Module):
    pass


class ConfigMixin:
    pass


def register_to_config(fn):
    return fn


class Timesteps(nn.Module):
    """diffusers Timesteps -> get_timestep_embedding (max_period 10000, scale 1)."""

    def __init__(self, num_channels, flip_sin_to_cos, downscale_freq_shift, scale=1):
        super().__init__()
        self.num_channels, self.flip, self.shift, self.scale = num_channels, flip_sin_to_cos, downscale_freq_shift, scale

    def forward(self, timesteps):
        half = self.num_channels // 2
        exponent = -math.log(10000) * torch.arange(0, half, dtype=torch.float32)
        exponent = exponent / (half - self.shift)
        emb = timesteps[:, None].float() * torch.exp(exponent)[None, :]
        emb = self.scale * emb
        emb = torch.cat([torch.sin(emb), torch.cos(emb)], dim=-1)
        if self.flip:
            emb = torch.cat([emb[:, half:], emb[:, :half]], dim=-1)
        return emb


class TimestepEmbedding(nn.Module):
    def __init__(self, in_channels, time_embed_dim):
        super().__init__()
        self.linear_1 = nn.Linear(in_channels, time_embed_dim, True)
        self.act = nn.SiLU()
        self.linear_2 = nn.Linear(time_embed_dim, time_embed_dim, True)

    def forward(self, sample):
        return self.linear_2(self.act(self.linear_1(sample)))


class PixArtAlphaTextProjection(nn.Module):
    def __init__(self, in_features, hidden_size, act_fn="gelu_tanh"):
        super().__init__()
        assert act_fn == "gelu_tanh"
        self.linear_1 = nn.Linear(in_features, hidden_size, bias=True)
        self.act_1 = nn.GELU(approximate="tanh")
        self.linear_2 = nn.Linear(hidden_size, hidden_size, bias=True)

    def forward(self, caption):
        return self.linear_2(self.act_1(self.linear_1(caption)))


def load_reference():
    wanted = {"custom_sdpa", "WanTimeTextImageEmbedding", "WanRotaryPosEmbed", "WanAttention",
              "WanTransformerBlock", "WanTransformer3DModel"}
    tree = ast.parse((REF / "modules" / "model.py").read_text())
    nodes = [n for n in tree.body if isinstance(n, (ast.FunctionDef, ast.ClassDef)) and n.name in wanted]
    assert {n.name for n in nodes} == wanted, "reference definitions not found"
    util = ast.parse((REF / "utils" / "utils.py").read_text())
    nodes += [n for n in util.body if isinstance(n, ast.FunctionDef) and n.name == "get_mesh_id"]
    ns = {"torch": torch, "nn": nn, "F": F, "math": math, "rearrange": rearrange, "deepcopy": deepcopy,
          "FeedForward": FeedForward, "FP32LayerNorm": FP32LayerNorm, "FlexAttnFunc": FlexAttnFunc,
          "flash_attn_func": None, "ModelMixin": ModelMixin, "ConfigMixin": ConfigMixin,
          "register_to_config": register_to_config, "Timesteps": Timesteps,
          "TimestepEmbedding": TimestepEmbedding, "PixArtAlphaTextProjection": PixArtAlphaTextProjection}
    exec(compile(ast.Module(body=nodes, type_ignores=[]), "reference_model", "exec"), ns)
    return ns


def main():
    if not REF.exists():
        sys.exit(f"{REF} not found: fixtures are generated in the build container only")
    ns = load_reference()
    cfg = dict(tiny_model.CONFIG)
    cfg["patch_size"] = list(cfg["patch_size"])
    model = ns["WanTransformer3DModel"](**cfg, attn_mode="torch").eval()
    shapes = {n: tuple(p.shape) for n, p in model.named_parameters()}
    params = tiny_model.make_params(shapes)
    with torch.no_grad():
        for n, p in model.named_parameters():
            p.copy_(params[n])
    tensors = {}
    for mode, make in (("video", tiny_model.video_inputs), ("action", tiny_model.action_inputs)):
        inp = make(ns["get_mesh_id"])
        for k, v in inp.items():
            tensors[f"{mode}.{k}"] = v.contiguous()
        with torch.no_grad():
            out = model(dict(inp), update_cache=0, action_mode=mode == "action")
        tensors[f"{mode}.out"] = out.contiguous()
    save_file(tensors, str(OUT / "reference_model_tiny.safetensors"),
              metadata={"config": repr(tiny_model.CONFIG), "seed": str(tiny_model.SEED),
                        "params": ";".join(f"{n}:{'x'.join(map(str, s))}" for n, s in sorted(shapes.items())),
                        "source": "model.py WanTransformer3DModel.forward (AST-extracted), see script"})
    print("wrote", OUT / "reference_model_tiny.safetensors", len(shapes), "parameters")


if __name__ == "__main__":
    main()
