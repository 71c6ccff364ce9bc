"""Parameter and KV-cache container with the reference's attention layout.

state_dict-compatible with WanAttention (model.py:289-346): to_q/to_k/to_v/
to_out[0] Linear layers and across-heads RMSNorm weights.  The cache dict is
the original mode (model.py:417-434): k, v [B_cfg, P, H, hd], id [P] int64,
mask [P] bool, is_pred [P] bool.  ``forward`` raises: the math runs in the
native block.  Same behaviour as 算子研究/wam_ops/optimized/parameters.py:6-45.
"""
import torch


class Attention(torch.nn.Module):

    def __init__(self, dim, heads=8, dim_head=64, eps=1e-05, dropout=0.0,
                 cross_attention_dim_head=None, attn_mode="torch"):
        super().__init__()
        if attn_mode != "torch":
            raise ValueError("the native block supports the torch parameter protocol only")
        self.inner_dim = dim_head * heads
        self.heads = heads
        self.cross_attention_dim_head = cross_attention_dim_head
        self.kv_inner_dim = self.inner_dim if cross_attention_dim_head is None else cross_attention_dim_head * heads
        self.to_q = torch.nn.Linear(dim, self.inner_dim, bias=True)
        self.to_k = torch.nn.Linear(dim, self.kv_inner_dim, bias=True)
        self.to_v = torch.nn.Linear(dim, self.kv_inner_dim, bias=True)
        self.to_out = torch.nn.ModuleList([torch.nn.Linear(self.inner_dim, dim, bias=True),
                                           torch.nn.Dropout(dropout)])
        self.norm_q = torch.nn.RMSNorm(dim_head * heads, eps=eps, elementwise_affine=True)
        self.norm_k = torch.nn.RMSNorm(dim_head * heads, eps=eps, elementwise_affine=True)
        self.attn_caches = {} if cross_attention_dim_head is None else None
        self.cache_mode = "original"

    def clear_pred_cache(self, cache_name):
        if self.attn_caches is not None:
            cache = self.attn_caches[cache_name]
            cache["mask"][cache["is_pred"]] = False

    def clear_cache(self, cache_name):
        if self.attn_caches is not None:
            self.attn_caches[cache_name] = None

    def init_kv_cache(self, cache_name, total_tolen, num_head, head_dim, device, dtype, batch_size):
        if self.attn_caches is not None:
            self.attn_caches[cache_name] = self._original_cache(
                total_tolen, num_head, head_dim, device, dtype, batch_size)

    @staticmethod
    def _original_cache(total_tolen, num_head, head_dim, device, dtype, batch_size):
        return {
            "k": torch.empty([batch_size, total_tolen, num_head, head_dim], device=device, dtype=dtype),
            "v": torch.empty([batch_size, total_tolen, num_head, head_dim], device=device, dtype=dtype),
            "id": torch.full((total_tolen,), -1, device=device),
            "mask": torch.zeros((total_tolen,), dtype=torch.bool, device=device),
            "is_pred": torch.zeros((total_tolen,), dtype=torch.bool, device=device),
        }

    def forward(self, *args, **kwargs):
        raise RuntimeError("Attention is a parameter/cache container; call the native TransformerBlock")
