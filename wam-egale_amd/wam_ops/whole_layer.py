"""WholeLayerBlock: the block with a prepared text context.

Mirrors 算子研究/wam_ops/optimized/whole_layer.py:17-85: ``prepare_context``
groups byte-identical context rows and, with ``precompute=True``, computes the
cross-attention K (RMS-normed) and V of each distinct row once, outside the
timed/graph region; ``__call__`` then skips those two GEMMs per layer.  The
context must be prepared again whenever its contents, the weights, the device
or the dtype change.
"""
import ctypes

import torch

from . import _lib
from .native import BoundWeights, block_eps, block_parameters, run_block
from .ops import stream_handle


class WholeLayerBlock:
    production_admitted = False

    def __init__(self, block, ffn_fp8=False, ffn_act_fp8=False):
        """ffn_fp8=True runs FFN1/FFN2 with e4m3 weights and per-output-channel
        fp32 scales (quantized once here); everything else stays bf16.
        ffn_act_fp8=True / 1 (with ffn_fp8) also quantizes FFN1's input per row
        (absmax / 448, inside LayerNorm 3) and runs FFN1 on the fp8 MFMA;
        ffn_act_fp8=2 also hands the hidden layer to FFN2 as MX e4m3 (one
        e8m0 exponent per 32 values) and runs FFN2 on the fp8 MFMA."""
        self.block = block
        self.ffn_fp8 = bool(ffn_fp8)
        self.ffn_act_fp8 = int(ffn_act_fp8)
        self.weights = block_parameters(block)
        self.eps = block_eps(block)
        self.context_rows = self.context_roots = None
        self.context_kv = []
        self.context_batch = None
        self._bound = None

    def bound(self):
        if self._bound is None:
            self._bound = BoundWeights(self.weights, self.eps, self.block.attn1.heads, ffn_fp8=self.ffn_fp8,
                                       ffn_act_fp8=self.ffn_act_fp8)
        return self._bound

    def prepare_context(self, context, precompute=False):
        """Group identical context rows (by bytes); optionally precompute K/V.

        Unlike the reference (which groups only a 14-row CFG batch), any batch
        size is grouped."""
        self.context_rows = self.context_roots = None
        self.context_kv = []
        batch = context.shape[0]
        self.context_batch = batch
        bits = context.detach().contiguous().view(torch.uint8).reshape(batch, -1)
        roots, rows = [], []
        for r in range(batch):
            group = next((g for g, root in enumerate(roots) if torch.equal(bits[r], bits[root])), None)
            if group is None:
                group = len(roots)
                roots.append(r)
            rows.append(group)
        if len(roots) < batch:
            self.context_rows = torch.tensor(rows, dtype=torch.int64, device=context.device)
            self.context_roots = torch.tensor(roots, dtype=torch.int64, device=context.device)
        if precompute:
            compact = context if self.context_roots is None else context.index_select(0, self.context_roots)
            compact = compact.contiguous()
            n, L, D = compact.shape
            k = torch.empty_like(compact)
            v = torch.empty_like(compact)
            bound = self.bound()
            _lib.check(_lib.lib().wam_prepare_context(ctypes.byref(bound.struct), compact.data_ptr(),
                                                       n * L, k.data_ptr(), v.data_ptr(),
                                                       stream_handle(compact.device)),
                       "wam_prepare_context")
            self.context_kv = [k, v]

    def __call__(self, hidden_states, encoder_hidden_states, temb, rotary_emb,
                 update_cache=0, cache_name="pos", candidate_cache_rows=None, debug=False,
                 timer=None, rows_checked=False, workspace=None, out=None):
        if torch.is_grad_enabled():
            raise RuntimeError("WholeLayerBlock is inference-only; use no_grad/inference_mode")
        caches = self.block.attn1.attn_caches or {}
        cache = caches.get(cache_name)
        ctx = encoder_hidden_states
        rows = self.context_rows
        if self.context_batch is not None:
            # The prepared grouping maps hidden_states row b to a context row:
            # both batches must be the one prepare_context saw, or the kernels
            # would index past the prepared rows.
            if encoder_hidden_states.shape[0] != self.context_batch:
                raise RuntimeError(f"context batch {encoder_hidden_states.shape[0]} differs from the "
                                   f"{self.context_batch} rows prepared by prepare_context")
            if (rows is not None or self.context_kv) and hidden_states.shape[0] != self.context_batch \
                    and not (self.context_batch == 1 and rows is None):
                raise RuntimeError(f"hidden_states batch {hidden_states.shape[0]} does not match the "
                                   f"{self.context_batch} prepared context rows")
        cross_kv = None
        if self.context_kv:
            cross_kv = self.context_kv
            ctx = self.context_kv[0]
        elif self.context_roots is not None:
            ctx = encoder_hidden_states.index_select(0, self.context_roots).contiguous()
        res = run_block(self.bound(), hidden_states, ctx, temb, rotary_emb, cache, update_cache,
                        candidate_cache_rows, debug=debug, cross_kv=cross_kv, context_rows=rows,
                        timer=timer, rows_checked=rows_checked, workspace=workspace, out=out)
        if debug:
            return res[1]
        return res
