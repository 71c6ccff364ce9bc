"""TransformerBlock: the reference block's parameter layout, native forward.

Submodules keep the state_dict keys of WanTransformerBlock (model.py:694-739):
norm1/norm2/norm3, attn1/attn2, ffn.net[0].proj / ffn.net[2] and
scale_shift_table.  ``forward`` runs the HIP block through NativeBlock, like
算子研究/wam_ops/optimized/block.py:10-79.  diffusers is not a dependency: the
two diffusers modules the reference builds (FeedForward with
"gelu-approximate", FP32LayerNorm) are stood in for by parameter holders with
the same attribute paths.
"""
import torch
from torch import nn

from .native import NativeBlock
from .parameters import Attention


class FP32LayerNorm(nn.LayerNorm):
    """Parameter holder for diffusers' FP32LayerNorm (same state_dict keys)."""


class _GELUProj(nn.Module):
    def __init__(self, dim_in, dim_out):
        super().__init__()
        self.proj = nn.Linear(dim_in, dim_out, bias=True)
        self.approximate = "tanh"


class FeedForward(nn.Module):
    """Parameter holder for diffusers FeedForward(dim, inner_dim, "gelu-approximate"):
    net = [GELU(proj: D->F, tanh), Dropout, Linear(F->D)]."""

    def __init__(self, dim, inner_dim):
        super().__init__()
        self.net = nn.ModuleList([_GELUProj(dim, inner_dim), nn.Dropout(0.0),
                                  nn.Linear(inner_dim, dim, bias=True)])


class TransformerBlock(nn.Module):
    attention_cls = Attention
    native_fused_ffn1 = False
    execution_mode = "sequential"

    def __init__(self, dim, ffn_dim, num_heads, cross_attn_norm=False, eps=1e-6,
                 attn_mode: str = "torch"):
        super().__init__()
        self.attn_mode = attn_mode
        self.norm1 = FP32LayerNorm(dim, eps, elementwise_affine=False)
        self.attn1 = self.attention_cls(dim=dim, heads=num_heads, dim_head=dim // num_heads, eps=eps,
                                        cross_attention_dim_head=None, attn_mode=attn_mode)
        self.attn2 = self.attention_cls(dim=dim, heads=num_heads, dim_head=dim // num_heads, eps=eps,
                                        cross_attention_dim_head=dim // num_heads, attn_mode=attn_mode)
        self.norm2 = FP32LayerNorm(dim, eps, elementwise_affine=True) if cross_attn_norm else nn.Identity()
        self.ffn = FeedForward(dim, ffn_dim)
        self.norm3 = FP32LayerNorm(dim, eps, elementwise_affine=False)
        self.scale_shift_table = nn.Parameter(torch.randn(1, 6, dim) / dim ** 0.5)

    def forward(self, hidden_states, encoder_hidden_states, temb, rotary_emb, update_cache=0,
                cache_name="pos", candidate_cache_rows=None) -> torch.Tensor:
        native = self.__dict__.get("_native_block")
        if native is None:
            native = NativeBlock(self, fused_ffn1=self.native_fused_ffn1, mode=self.execution_mode)
            object.__setattr__(self, "_native_block", native)
        return native(hidden_states, encoder_hidden_states, temb, rotary_emb, update_cache,
                      cache_name, candidate_cache_rows)
