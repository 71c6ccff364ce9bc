"""WanTransformer3DModel.forward (inference) restated on the CPU (oracle).

TEST INFRASTRUCTURE ONLY (see the package docstring).

Follows 投机采样/wam-p0-worktree/wan_va/modules/model.py:
  patch embedding     :1064-1071  rearrange 'b c (f p1) (h p2) (w p3) -> b (f h w) (c p1 p2 p3)'
                                 then patch_embedding_mlp
  action embedding    :1060-1063  rearrange 'b c f h w -> b (f h w) c' then action_embedder
  text embedder       :1072-1073  condition_embedder.text_embedder (Linear, GELU tanh, Linear)
  RoPE                :1076-1077  rope(grid_id)[:, :, None] (oracle.rope)
  timesteps           :1078-1086  repeat_interleave(timesteps [B, F], tokens per frame)
  condition embedder  :226-240    sinusoid -> time_embedder (Linear, SiLU, Linear) = temb;
                                 time_proj(SiLU(temb)) = timestep_proj, unflatten(2, (6, -1))
  blocks              :1088-1095  oracle.block.block_forward per layer
  norm_out            :1096-1103  LN(x.float()) * (1 + scale) + shift with
                                 [shift, scale] = scale_shift_table[None] + temb[:, :, None]
  proj_out            :1105-1112  proj_out + rearrange 'b l (n c) -> b (l n) c' (video) or
                                 action_proj_out (action)

The diffusers 0.36.0 modules (requirements.txt:4; not installed) are restated
from their published definitions: Timesteps(freq_dim, flip_sin_to_cos=True,
downscale_freq_shift=0) is get_timestep_embedding (fp32 frequencies
exp(-ln(10000) * i / (half - shift)), [sin, cos] flipped to [cos, sin]);
TimestepEmbedding is linear_1 -> SiLU -> linear_2; PixArtAlphaTextProjection is
linear_1 -> GELU(tanh) -> linear_2.  Everything here is fp32.

Pinning: the composition by tests/golden/reference_model_tiny.safetensors
(written by tests/golden/make_model_vectors.py from model.py); the sinusoid
by closed forms (t = 0, the first and last frequencies, cos^2 + sin^2 = 1,
the flip order) in tests/test_oracle.py; patchify by einops with the
reference's pattern strings and by a brute-force loop.
"""
import math

import torch
import torch.nn.functional as F

from .block import block_forward
from .rope import rope_freqs


def timestep_sinusoid(t, dim=256, flip_sin_to_cos=True, shift=0.0, max_period=10000):
    """get_timestep_embedding: t [R] -> [R, dim] fp32."""
    half = dim // 2
    exponent = -math.log(max_period) * torch.arange(0, half, dtype=torch.float32)
    exponent = exponent / (half - shift)
    arg = t.reshape(-1)[:, None].float() * torch.exp(exponent)[None, :]
    emb = torch.cat([torch.sin(arg), torch.cos(arg)], dim=-1)
    if flip_sin_to_cos:
        emb = torch.cat([emb[:, half:], emb[:, :half]], dim=-1)
    if dim % 2:
        emb = F.pad(emb, (0, 1))
    return emb


def _lin(P, name, x):
    return F.linear(x, P[f"{name}.weight"].float(), P[f"{name}.bias"].float())


def condition_embedding(P, prefix, t, freq_dim=256):
    """WanTimeTextImageEmbedding.forward (model.py:226-240) for t [B, L]:
    (temb [B, L, D], timestep_proj [B, L, 6D])."""
    B, L = t.shape
    s = timestep_sinusoid(t.reshape(-1), freq_dim)
    temb = _lin(P, f"{prefix}.time_embedder.linear_2", F.silu(_lin(P, f"{prefix}.time_embedder.linear_1", s)))
    proj = _lin(P, f"{prefix}.time_proj", F.silu(temb))
    return temb.reshape(B, L, -1), proj.reshape(B, L, -1)


def text_embedding(P, text, prefix="condition_embedder.text_embedder"):
    """PixArtAlphaTextProjection: linear_1 -> GELU(tanh) -> linear_2."""
    h = F.gelu(_lin(P, f"{prefix}.linear_1", text.float()), approximate="tanh")
    return _lin(P, f"{prefix}.linear_2", h)


def patchify(latents, patch):
    """'b c (f p1) (h p2) (w p3) -> b (f h w) (c p1 p2 p3)'."""
    B, C, Fr, H, W = latents.shape
    p1, p2, p3 = patch
    x = latents.reshape(B, C, Fr // p1, p1, H // p2, p2, W // p3, p3)
    x = x.permute(0, 2, 4, 6, 1, 3, 5, 7)
    return x.reshape(B, (Fr // p1) * (H // p2) * (W // p3), C * p1 * p2 * p3)


def unpatchify(y, patch):
    """'b l (n c) -> b (l n) c' with n = prod(patch)."""
    B, L, NC = y.shape
    n = math.prod(patch)
    return y.reshape(B, L * n, NC // n)


def head(P, x, temb, eps=1e-6, proj="proj_out"):
    """norm_out + modulation + the output projection (model.py:1096-1107)."""
    mod = P["scale_shift_table"].float()[None] + temb.float()[:, :, None, :]  # [B, L, 2, D]
    shift, scale = mod[:, :, 0], mod[:, :, 1]
    D = x.shape[-1]
    h = F.layer_norm(x.float(), (D,), eps=eps) * (1.0 + scale) + shift
    return _lin(P, proj, h)


def block_params(P, i):
    pre = f"blocks.{i}."
    return {k[len(pre):]: v for k, v in P.items() if k.startswith(pre)}


def model_forward(P, inp, cfg, action_mode=False, caches=None, update_cache=0, candidate_rows=None):
    """WanTransformer3DModel.forward, inference path, fp32.

    P: state_dict-named parameters; inp: noisy_latents [B, C, F, H, W],
    text_emb [B, Lc, text_dim], grid_id [B, >=3, L], timesteps [B, F];
    caches: one oracle cache dict per layer (or None)."""
    patch = tuple(cfg["patch_size"])
    heads = cfg["num_attention_heads"]
    eps = cfg.get("eps", 1e-6)
    lat = inp["noisy_latents"].float()
    if action_mode:
        x = _lin(P, "action_embedder", patchify(lat, (1, 1, 1)))
        per_frame = lat.shape[-2] * lat.shape[-1]
    else:
        x = _lin(P, "patch_embedding_mlp", patchify(lat, patch))
        per_frame = (lat.shape[-2] // patch[1]) * (lat.shape[-1] // patch[2])
    ctx = text_embedding(P, inp["text_emb"])
    freqs = rope_freqs(inp["grid_id"], cfg["attention_head_dim"])
    t = torch.repeat_interleave(inp["timesteps"].float(), per_frame, dim=1)
    prefix = "condition_embedder_action" if action_mode else "condition_embedder"
    temb, proj = condition_embedding(P, prefix, t, cfg.get("freq_dim", 256))
    proj = proj.unflatten(2, (6, -1))
    for i in range(cfg["num_layers"]):
        x = block_forward(block_params(P, i), x, ctx, proj, freqs, heads, eps,
                          cache=None if caches is None else caches[i], update_cache=update_cache,
                          candidate_rows=candidate_rows)
    if action_mode:
        return head(P, x, temb, eps, "action_proj_out")
    return unpatchify(head(P, x, temb, eps, "proj_out"), patch)
