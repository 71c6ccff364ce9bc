"""TransformerModel / WholeModel: the whole WanTransformer3DModel inference
forward on the GPU.

``TransformerModel`` keeps the constructor and state_dict keys of
WanTransformer3DModel (投机采样/wam-p0-worktree/wan_va/modules/model.py:797-880):
patch_embedding_mlp, action_embedder, condition_embedder(_action) with
time_embedder / time_proj / text_embedder, blocks, norm_out, proj_out,
action_proj_out and scale_shift_table.  diffusers is not a dependency; its
Timesteps / TimestepEmbedding / PixArtAlphaTextProjection are stood in for
by holders with the same attribute paths.

``WholeModel`` runs WanTransformer3DModel.forward (model.py:1033-1116,
inference path) on any module with that layout (this class or the reference's
own), every step a HIP kernel of libwam_block:

  patch / action embedding   wam_patchify + wam_linear (model.py:1060-1071)
  text embedder              wam_linear (GELU epilogue) x 2 (model.py:1072-1073)
  RoPE frequencies           wam_rope_freqs (model.py:1076-1077)
  condition embedder         wam_timestep_embedding + wam_rows_linear x 3
                             (model.py:1078-1087, 226-240)
  blocks                     BlockStack (one workspace, no host syncs)
  norm_out + modulation      wam_ln_modulate with a one-vector temb (model.py:1096-1103)
  proj_out                   wam_linear, then the 'b l (n c) -> b (l n) c' view
                             (action: wam_rows_linear, N = 30) (model.py:1105-1112)

Two choices differ from the reference's op sequence and give the same values:
the condition embedder runs once per (sample, latent frame) timestep instead
of once per token (the reference repeats each frame's timestep over the
frame's tokens, model.py:1078-1082, and the embedder is row-wise), and the
blocks and the head read those per-frame rows (temb length F, each row
serving one frame's tokens).  The action embedder's K = 30 is zero-padded to
64 (gathered rows and weights), which adds zeros to every dot product.

``prepare_text(text_emb)`` runs the text embedder once and precomputes every
layer's cross-attention K/V (WholeLayerBlock.prepare_context,
算子研究/wam_ops/optimized/whole_layer.py:41-67, for each block); later calls
then skip the text path entirely.  The text must be prepared again whenever
its contents change.  Without it, every call embeds the text and every layer
projects its own cross K/V, as the reference does.
"""
import math

import torch
from torch import nn

from . import ops
from .block import TransformerBlock
from .verify import BlockStack


class Timesteps(nn.Module):
    """Holder for diffusers Timesteps (no parameters)."""

    def __init__(self, num_channels, flip_sin_to_cos, downscale_freq_shift, scale=1):
        super().__init__()
        self.num_channels = num_channels
        self.flip_sin_to_cos = flip_sin_to_cos
        self.downscale_freq_shift = downscale_freq_shift
        self.scale = scale


class TimestepEmbedding(nn.Module):
    """Holder for diffusers TimestepEmbedding(in, dim): linear_1, SiLU, linear_2."""

    def __init__(self, in_channels, time_embed_dim):
        super().__init__()
        self.linear_1 = nn.Linear(in_channels, time_embed_dim, True)
        self.act = nn.SiLU()
        self.linear_2 = nn.Linear(time_embed_dim, time_embed_dim, True)


class PixArtAlphaTextProjection(nn.Module):
    """Holder for diffusers PixArtAlphaTextProjection: linear_1, GELU(tanh), linear_2."""

    def __init__(self, in_features, hidden_size):
        super().__init__()
        self.linear_1 = nn.Linear(in_features, hidden_size, bias=True)
        self.act_1 = nn.GELU(approximate="tanh")
        self.linear_2 = nn.Linear(hidden_size, hidden_size, bias=True)


class TimeTextEmbedding(nn.Module):
    """WanTimeTextImageEmbedding's layout (model.py:203-224)."""

    def __init__(self, dim, time_freq_dim, time_proj_dim, text_embed_dim):
        super().__init__()
        self.timesteps_proj = Timesteps(time_freq_dim, flip_sin_to_cos=True, downscale_freq_shift=0)
        self.time_embedder = TimestepEmbedding(time_freq_dim, dim)
        self.act_fn = nn.SiLU()
        self.time_proj = nn.Linear(dim, time_proj_dim)
        self.text_embedder = PixArtAlphaTextProjection(text_embed_dim, dim)


class RotaryPosEmbed(nn.Module):
    """WanRotaryPosEmbed's configuration (model.py:243-262; no parameters)."""

    def __init__(self, attention_head_dim, patch_size, max_seq_len, theta=10000.0):
        super().__init__()
        self.attention_head_dim = attention_head_dim
        self.patch_size = patch_size
        self.max_seq_len = max_seq_len
        self.theta = theta


class FP32LayerNorm(nn.LayerNorm):
    """Holder for diffusers FP32LayerNorm."""


class TransformerModel(nn.Module):
    """WanTransformer3DModel's constructor and parameters; ``forward`` is
    WholeModel (inference only)."""

    def __init__(self, patch_size=(1, 2, 2), num_attention_heads=24, attention_head_dim=128,
                 in_channels=48, out_channels=48, action_dim=30, text_dim=4096, freq_dim=256,
                 ffn_dim=14336, num_layers=30, cross_attn_norm=True, eps=1e-06, rope_max_seq_len=1024,
                 pos_embed_seq_len=None, attn_mode="torch"):
        super().__init__()
        self.patch_size = list(patch_size)
        self.num_attention_heads = num_attention_heads
        self.attention_head_dim = attention_head_dim
        inner = num_attention_heads * attention_head_dim
        self.rope = RotaryPosEmbed(attention_head_dim, self.patch_size, rope_max_seq_len)
        self.patch_embedding_mlp = nn.Linear(in_channels * math.prod(self.patch_size), inner)
        self.action_embedder = nn.Linear(action_dim, inner)
        self.condition_embedder = TimeTextEmbedding(inner, freq_dim, inner * 6, text_dim)
        self.condition_embedder_action = TimeTextEmbedding(inner, freq_dim, inner * 6, text_dim)
        self.blocks = nn.ModuleList([TransformerBlock(inner, ffn_dim, num_attention_heads, cross_attn_norm,
                                                      eps, attn_mode=attn_mode) for _ in range(num_layers)])
        self.norm_out = FP32LayerNorm(inner, eps, elementwise_affine=False)
        self.proj_out = nn.Linear(inner, out_channels * math.prod(self.patch_size))
        self.action_proj_out = nn.Linear(inner, action_dim)
        self.scale_shift_table = nn.Parameter(torch.randn(1, 2, inner) / inner ** 0.5)

    # cache management, model.py:880-896
    def clear_cache(self, cache_name):
        for block in self.blocks:
            block.attn1.clear_cache(cache_name)

    def clear_pred_cache(self, cache_name):
        for block in self.blocks:
            block.attn1.clear_pred_cache(cache_name)

    def create_empty_cache(self, cache_name, attn_window, latent_token_per_chunk, action_token_per_chunk,
                           device, dtype, batch_size):
        total = (attn_window // 2) * latent_token_per_chunk + (attn_window // 2) * action_token_per_chunk
        for block in self.blocks:
            block.attn1.init_kv_cache(cache_name, total, self.num_attention_heads, self.attention_head_dim,
                                      device, dtype, batch_size)

    def native(self, **options):
        whole = self.__dict__.get("_whole_model")
        if whole is None:
            whole = WholeModel(self, **options)
            object.__setattr__(self, "_whole_model", whole)
        return whole

    def forward(self, input_dict, update_cache=0, cache_name="pos", action_mode=False, train_mode=False,
                candidate_cache_rows=None):
        return self.native()(input_dict, update_cache=update_cache, cache_name=cache_name,
                             action_mode=action_mode, train_mode=train_mode,
                             candidate_cache_rows=candidate_cache_rows)


def _frozen(t, dev):
    return t.detach().to(dev).contiguous()


class _Condition:
    """Bound condition-embedder weights (one of condition_embedder(_action))."""

    def __init__(self, mod, dev):
        tp = mod.timesteps_proj
        self.freq_dim = int(getattr(tp, "num_channels", 256))
        self.flip = bool(getattr(tp, "flip_sin_to_cos", True))
        self.shift = float(getattr(tp, "downscale_freq_shift", 0))
        self.scale = float(getattr(tp, "scale", 1))
        te = mod.time_embedder
        self.w1, self.b1 = _frozen(te.linear_1.weight, dev), _frozen(te.linear_1.bias, dev)
        self.w2, self.b2 = _frozen(te.linear_2.weight, dev), _frozen(te.linear_2.bias, dev)
        self.wp, self.bp = _frozen(mod.time_proj.weight, dev), _frozen(mod.time_proj.bias, dev)
        tx = mod.text_embedder
        self.t1, self.tb1 = _frozen(tx.linear_1.weight, dev), _frozen(tx.linear_1.bias, dev)
        self.t2, self.tb2 = _frozen(tx.linear_2.weight, dev), _frozen(tx.linear_2.bias, dev)

    def time(self, timesteps, dtype):
        """timesteps [B, F] -> (temb [B, F, D], timestep_proj [B, F, 6, D]), both
        in `dtype` (model.py:226-240 with one row per frame)."""
        B, Fr = timesteps.shape
        if self.scale != 1:
            raise NotImplementedError("Timesteps(scale != 1) is not part of the model")
        t = timesteps.reshape(-1).to(torch.float32).contiguous()
        s = ops.timestep_embedding(t, self.freq_dim, self.flip, self.shift, out_dtype=self.w1.dtype)
        h = ops.rows_linear(s, self.w1, self.b1, act_out="silu", out_dtype=self.w1.dtype)
        temb = ops.rows_linear(h, self.w2, self.b2, out_dtype=dtype)
        proj = ops.rows_linear(temb, self.wp, self.bp, act_in="silu", out_dtype=dtype)
        D = self.w2.shape[0]
        return temb.view(B, Fr, D), proj.view(B, Fr, 6, D)

    def text(self, text_emb):
        """PixArtAlphaTextProjection on the GPU: [B, Lc, text_dim] -> [B, Lc, D]."""
        h = ops.linear(text_emb.contiguous(), self.t1, self.tb1, epilogue=ops.EPI_BIAS_GELU)
        return ops.linear(h, self.t2, self.tb2)


class WholeModel:
    def __init__(self, model, ffn_fp8=False):
        self.model = model
        self.stack = BlockStack(list(model.blocks), ffn_fp8=ffn_fp8)
        self.patch_size = tuple(int(p) for p in model.patch_size)
        self.head_dim = int(model.attention_head_dim)
        self.theta = float(getattr(model.rope, "theta", 10000.0))
        self.eps = float(model.norm_out.eps)
        self._bound = None
        self._text = None

    # ------------------------------------------------------------ weights
    def _bind(self):
        if self._bound is not None:
            return self._bound
        m = self.model
        dev = m.proj_out.weight.device
        if dev.type != "cuda":
            raise RuntimeError("WholeModel needs the model on the GPU")
        b = {}
        for name in ("patch_embedding_mlp", "action_embedder"):
            lin = getattr(m, name)
            w = _frozen(lin.weight, dev)
            k_pad = -(-w.shape[1] // 64) * 64
            if k_pad != w.shape[1]:
                w = torch.nn.functional.pad(w, (0, k_pad - w.shape[1])).contiguous()
            b[name] = (w, _frozen(lin.bias, dev), k_pad)
        b["cond"] = _Condition(m.condition_embedder, dev)
        b["cond_action"] = _Condition(m.condition_embedder_action, dev)
        b["table"] = _frozen(m.scale_shift_table, dev)
        b["proj_out"] = (_frozen(m.proj_out.weight, dev), _frozen(m.proj_out.bias, dev))
        b["action_proj_out"] = (_frozen(m.action_proj_out.weight, dev), _frozen(m.action_proj_out.bias, dev))
        self._bound = b
        return b

    # --------------------------------------------------------------- text
    def prepare_text(self, text_emb, precompute=True):
        """Embed the text once and precompute every layer's cross K/V."""
        with torch.no_grad():
            ctx = self._bind()["cond"].text(text_emb)
            self.stack.prepare_context(ctx, precompute=precompute)
        self._text = ctx
        return ctx

    def clear_text(self):
        self._text = None
        for layer in self.stack.layers:
            layer.context_rows = layer.context_roots = None
            layer.context_kv = []
            layer.context_batch = None

    # ------------------------------------------------------------ forward
    def embed(self, latents, action_mode):
        """Patch (or action) embedding: [B, C, F, H, W] -> [B, L, D] bf16."""
        b = self._bind()
        name = "action_embedder" if action_mode else "patch_embedding_mlp"
        w, bias, k_pad = b[name]
        patch = (1, 1, 1) if action_mode else self.patch_size
        rows = ops.patchify(latents.contiguous(), patch, k_pad)
        return ops.linear(rows, w, bias)

    def head(self, x, temb, action_mode):
        """norm_out + modulation + proj_out (model.py:1096-1112)."""
        b = self._bind()
        h = ops.head_norm(x, b["table"], temb, self.eps)
        if action_mode:
            w, bias = b["action_proj_out"]
            return ops.rows_linear(h, w, bias, out_dtype=h.dtype)
        w, bias = b["proj_out"]
        y = ops.linear(h, w, bias)
        n = math.prod(self.patch_size)
        B, L, NC = y.shape
        return y.view(B, L * n, NC // n)

    def __call__(self, input_dict, update_cache=0, cache_name="pos", action_mode=False, train_mode=False,
                 candidate_cache_rows=None):
        if candidate_cache_rows is not None and (train_mode or update_cache != 0):
            raise ValueError("candidate read-only forward requires inference and update_cache=0")
        if train_mode:
            raise NotImplementedError("the native model runs the inference forward only")
        if torch.is_grad_enabled():
            raise RuntimeError("WholeModel is inference-only; use no_grad/inference_mode")
        b = self._bind()
        lat = input_dict["noisy_latents"]
        if lat.dtype != torch.bfloat16:
            raise RuntimeError("noisy_latents must be bfloat16 (the native blocks run in bf16)")
        x = self.embed(lat, action_mode)
        B, L, _ = x.shape
        if self._text is not None:
            ctx = self._text
        else:
            ctx = b["cond"].text(input_dict["text_emb"])
        freqs = ops.rope_freqs(input_dict["grid_id"], self.head_dim, self.theta)
        timesteps = input_dict["timesteps"]
        if timesteps.dim() != 2 or timesteps.shape[0] != B or L % timesteps.shape[1] != 0:
            raise ValueError("timesteps must be [B, F] with one entry per latent frame")
        cond = b["cond_action"] if action_mode else b["cond"]
        temb, proj = cond.time(timesteps, x.dtype)
        x = self.stack(x, ctx, proj, freqs, update_cache=update_cache, cache_name=cache_name,
                       candidate_cache_rows=candidate_cache_rows)
        return self.head(x, temb, action_mode)
