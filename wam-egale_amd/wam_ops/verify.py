"""BlockStack: the model-level block loop of the speculative verify forward.

The reference's ``WanTransformer3DModel.forward`` runs every block in turn
(投机采样/wam-p0-worktree/wan_va/modules/model.py:1091-1098) and, for a
verify call, passes ``candidate_cache_rows`` with ``update_cache=0``
(model.py:1056-1057; the server's caller is wan_va_server.py:1904-1935).
Each block then validates the rows against its own read-only cache
(model.py:647-653), which reads the rows back to the host once per layer.

``BlockStack`` keeps that contract and error behaviour but checks the rows
once per forward against every layer's cache batch, runs all layers on the
current stream with one reused workspace and two ping-pong activation
buffers, and never synchronises in between.  Outputs are identical to calling
each ``WholeLayerBlock`` in turn.
"""
import torch

from .native import validate_candidate_rows
from .whole_layer import WholeLayerBlock


class BlockStack:
    def __init__(self, blocks, ffn_fp8=False):
        self.layers = [b if isinstance(b, WholeLayerBlock) else WholeLayerBlock(b, ffn_fp8=ffn_fp8)
                       for b in blocks]
        if not self.layers:
            raise ValueError("BlockStack needs at least one block")
        self._ws = None

    def __len__(self):
        return len(self.layers)

    def prepare_context(self, context, precompute=True):
        """Per-layer cross-attention K/V of the shared text context
        (whole_layer.py:41-67 for every block)."""
        for layer in self.layers:
            layer.prepare_context(context, precompute=precompute)

    def _cache_batches(self, cache_name):
        batches = []
        for layer in self.layers:
            caches = layer.block.attn1.attn_caches or {}
            cache = caches.get(cache_name)
            if cache is None or cache.get("k") is None:
                raise ValueError("candidate verification requires existing read-only KV")
            batches.append(cache["k"].shape[0])
        return batches

    def __call__(self, hidden_states, encoder_hidden_states, temb, rotary_emb,
                 update_cache=0, cache_name="pos", candidate_cache_rows=None):
        if candidate_cache_rows is not None and update_cache != 0:
            raise ValueError("candidate read-only forward requires inference and update_cache=0")
        if torch.is_grad_enabled():
            raise RuntimeError("BlockStack is inference-only; use no_grad/inference_mode")
        rows = candidate_cache_rows
        if rows is not None:
            # One host read-back for the whole stack: the rows must index every
            # layer's history batch.
            validate_candidate_rows(rows, hidden_states.shape[0], min(self._cache_batches(cache_name)),
                                    hidden_states.device)
        x = hidden_states
        ws = self._workspace(x, encoder_hidden_states, cache_name)
        bufs = [torch.empty_like(x), torch.empty_like(x)] if len(self.layers) > 2 else []
        for i, layer in enumerate(self.layers):
            last = i == len(self.layers) - 1
            out = None if last or not bufs else bufs[i % 2]
            x = layer(x, encoder_hidden_states, temb, rotary_emb, update_cache=update_cache,
                      cache_name=cache_name, candidate_cache_rows=rows,
                      rows_checked=rows is not None, workspace=ws, out=out)
        return x

    def _workspace(self, x, ctx, cache_name):
        """One workspace sized for the largest layer; kept and grown across calls."""
        from . import _lib
        B, M, D = x.shape
        need = 0
        for lyr in self.layers:
            caches = lyr.block.attn1.attn_caches or {}
            cache = caches.get(cache_name)
            pool = cache["k"].shape[1] if cache is not None and cache.get("k") is not None else 0
            c = lyr.context_kv[0] if lyr.context_kv else ctx
            need = max(need, _lib.lib().wam_block_workspace_bytes(B, M, D, lyr.bound().ffn_dim,
                                                                  c.shape[0], c.shape[1], pool))
        if self._ws is None or self._ws.numel() < need or self._ws.device != x.device:
            self._ws = torch.empty(need, dtype=torch.uint8, device=x.device)
        return self._ws
