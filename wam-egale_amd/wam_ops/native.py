"""NativeBlock: the whole DiT block as one C-ABI call (wam_block_forward).

Mirrors the reference's operator surface: the 27 parameters are bound as
detached aliases in the reference order, the cache is read from
``block.attn1.attn_caches[cache_name]`` and ``__call__`` has the reference
signature (算子研究/wam_ops/optimized/native.py:27-65).
"""
import ctypes
import weakref

import torch

from . import _lib
from .ops import dtype_code, stream_handle

MODES = ("sequential", "tiled", "persistent")


def block_parameters(block):
    """The 27 tensors in the reference order (optimized/native.py:35-49)."""
    weights = [block.scale_shift_table]
    if hasattr(block.norm2, "weight"):
        weights += [block.norm2.weight, block.norm2.bias]
    else:
        empty = block.scale_shift_table.new_empty(0)
        weights += [empty, empty]
    for attn in (block.attn1, block.attn2):
        for m in (attn.to_q, attn.to_k, attn.to_v, attn.to_out[0]):
            weights += [m.weight, m.bias]
        weights += [attn.norm_q.weight, attn.norm_k.weight]
    for m in (block.ffn.net[0].proj, block.ffn.net[2]):
        weights += [m.weight, m.bias]
    return [w.detach() for w in weights]


def block_eps(block):
    """eps[7] = [norm1, norm2, norm3, attn1.q, attn1.k, attn2.q, attn2.k]."""
    return [block.norm1.eps, getattr(block.norm2, "eps", block.norm1.eps), block.norm3.eps,
            block.attn1.norm_q.eps, block.attn1.norm_k.eps, block.attn2.norm_q.eps,
            block.attn2.norm_k.eps]


def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


class BoundWeights:
    """Validated parameter pointers packed into a wam_block_weights struct."""

    def __init__(self, weights, eps, heads, ffn_fp8=False, ffn_act_fp8=False):
        _check(len(weights) == 27 and len(eps) == 7, "native parameter schema: 27 weights, 7 eps")
        dev = weights[3].device
        _check(dev.type == "cuda", "native block parameters must live on the GPU")
        for i, t in enumerate(weights):
            ok_dtype = t.dtype == torch.bfloat16 or (i <= 2 and t.dtype == torch.float32)
            _check(t.device == dev and ok_dtype and t.is_contiguous() and not t.requires_grad,
                   f"frozen canonical parameter index {i} dtype {t.dtype}")
        self.tensors = weights
        dim = weights[3].shape[1]
        self.dim, self.ffn_dim, self.heads, self.device = dim, weights[23].shape[0], heads, dev
        st = _lib.BlockWeights()
        for i, t in enumerate(weights):
            st.w[i] = t.data_ptr() if t.numel() else None
        st.table_dtype = dtype_code(weights[0])
        st.norm2_dtype = dtype_code(weights[1]) if weights[1].numel() else _lib.WAM_F32
        st.dim, st.heads, st.head_dim, st.ffn_dim = dim, heads, dim // heads, self.ffn_dim
        for i, e in enumerate(eps):
            st.eps[i] = float(e)
        self.ffn_fp8 = None
        if ffn_fp8:
            # e4m3 FFN weights with per-output-channel scales (no counterpart in
            # the reference; the biases stay bf16)
            from .ops import quantize_fp8_rows
            q1, s1 = quantize_fp8_rows(weights[23])
            q2, s2 = quantize_fp8_rows(weights[25])
            self.ffn_fp8 = (q1, s1, q2, s2)
            st.ffn_fp8[0], st.ffn_fp8[1] = q1.data_ptr(), q2.data_ptr()
            st.ffn_scale[0], st.ffn_scale[1] = s1.data_ptr(), s2.data_ptr()
        if ffn_act_fp8:
            # 1: FFN1 input quantized per row inside LayerNorm 3, FFN1 on the
            # fp8 MFMA; 2: also the hidden layer as MX e4m3 and FFN2 on the
            # fp8 MFMA
            _check(ffn_fp8, "fp8 FFN activations need the fp8 FFN weights")
            _check(int(ffn_act_fp8) in (1, 2), "ffn_act_fp8 must be 0, 1 (FFN1) or 2 (FFN1 and FFN2)")
            st.ffn_act_fp8 = int(ffn_act_fp8)
        self.struct = st


# Candidate-row tensors already validated: id -> (weakref, torch version
# counter, batch, pool batch, device).  The same tensor object, unmodified
# since (its version counter moves with every in-place torch write), passes
# again without reading it back to the host.  Inference tensors (created
# under torch.inference_mode) have no version counter, so they are checked on
# every call.
_validated_rows = {}


def validate_candidate_rows(rows, batch, pool_batch, device):
    # Same contract and error type as model.py:639-647 (this reads the rows
    # back to the host, as the reference's validation does, unless this very
    # tensor passed before and has not been written since).
    if (rows.ndim != 1 or rows.numel() != batch or rows.dtype != torch.long
            or rows.device != device):
        raise ValueError("invalid candidate_cache_rows for this KV cache")
    key = None if rows.is_inference() else (rows._version, batch, pool_batch, device)
    if key is not None:
        hit = _validated_rows.get(id(rows))
        if hit is not None and hit[0]() is rows and hit[1] == key:
            return
    if not bool(((rows >= 0) & (rows < pool_batch)).all()):
        raise ValueError("invalid candidate_cache_rows for this KV cache")
    if key is None:
        return
    if len(_validated_rows) > 64:
        _validated_rows.clear()
    _validated_rows[id(rows)] = (weakref.ref(rows), key)


def run_block(bound, hidden_states, encoder_hidden_states, temb, rotary_emb, cache,
              update_cache, candidate_cache_rows, debug=False, cross_kv=None,
              context_rows=None, timer=None, rows_checked=False, workspace=None, out=None):
    """One wam_block_forward call.  Returns the output, or (output, debug dict).

    ``rows_checked``: the caller has already validated the candidate rows'
    values against this cache's batch (no host read-back here).
    ``workspace``: a uint8 device tensor to use if it is large enough.
    ``out``: a preallocated [B, M, D] output (must not alias the input):
    bf16, or fp32 for the block's result before its final bf16 rounding (a
    parity diagnostic; not with ``debug``)."""
    x = hidden_states
    dev = bound.device
    _check(x.is_cuda and x.device == dev and x.dtype == torch.bfloat16 and x.is_contiguous()
           and x.dim() == 3 and x.shape[2] == bound.dim,
           f"BF16 block contract: x must be [B, M, {bound.dim}] contiguous bf16 on {dev}")
    B, M, D = x.shape
    ctx = encoder_hidden_states
    _check(ctx.device == dev and ctx.dtype == torch.bfloat16 and ctx.is_contiguous()
           and ctx.dim() == 3 and ctx.shape[2] == D, "context must be [Bc, Lc, D] contiguous bf16")
    _check(temb.device == dev and temb.dim() == 4 and temb.shape[0] == B and temb.shape[2] == 6
           and temb.shape[3] == D and temb.shape[1] >= 1 and M % temb.shape[1] == 0,
           "temb must be [B, L, 6, D] with L = 1, M, or a divisor of M (one row per frame)")
    temb = temb.contiguous()
    table = bound.tensors[0]
    args = _lib.BlockArgs()
    args.weights = ctypes.pointer(bound.struct)
    args.B, args.M, args.x = B, M, x.data_ptr()
    args.context, args.context_batch, args.context_len = ctx.data_ptr(), ctx.shape[0], ctx.shape[1]
    if context_rows is not None:
        args.context_rows = context_rows.data_ptr()
    mod = _lib.Modulation()
    mod.table, mod.table_dtype = table.data_ptr(), dtype_code(table)
    mod.temb, mod.temb_dtype, mod.temb_len, mod.tokens = temb.data_ptr(), dtype_code(temb), temb.shape[1], M
    mod.temb_mods = 6
    args.mod = mod
    freq = None
    if rotary_emb is not None:
        freq = rotary_emb
        _check(freq.dtype == torch.complex64 and freq.device == dev, "rotary_emb must be complex64")
        freq = freq.reshape(freq.shape[0], freq.shape[1], -1).contiguous()
        _check(freq.shape[1] == M and freq.shape[2] == bound.struct.head_dim // 2
               and freq.shape[0] in (1, B), "rotary_emb must be [B or 1, M, 1, head_dim/2]")
        args.freq, args.freq_batch = freq.data_ptr(), freq.shape[0]
    pool = 0
    if cache is not None:
        k, v, ids, mask, pred = (cache[n] for n in ("k", "v", "id", "mask", "is_pred"))
        _check(k.dtype == torch.bfloat16 and k.is_contiguous() and v.is_contiguous()
               and k.shape == v.shape and k.dim() == 4 and k.shape[2] * k.shape[3] == D,
               "cache schema: K,V [B_cfg, P, H, hd] bf16")
        _check(ids.dtype == torch.int64 and mask.dtype == torch.bool and pred.dtype == torch.bool,
               "cache schema: id int64, mask/is_pred bool")
        pool = k.shape[1]
        args.cache_k, args.cache_v = k.data_ptr(), v.data_ptr()
        args.cache_id, args.cache_mask, args.cache_is_pred = ids.data_ptr(), mask.data_ptr(), pred.data_ptr()
        args.cache_batch, args.pool = k.shape[0], pool
        if candidate_cache_rows is not None:
            if update_cache != 0:
                raise ValueError("candidate verification requires existing read-only KV")
            if rows_checked:
                _check(candidate_cache_rows.ndim == 1 and candidate_cache_rows.numel() == B
                       and candidate_cache_rows.dtype == torch.long
                       and candidate_cache_rows.device == dev, "candidate_cache_rows schema")
            else:
                validate_candidate_rows(candidate_cache_rows, B, k.shape[0], dev)
            args.candidate_rows = candidate_cache_rows.data_ptr()
        elif k.shape[0] != B:
            raise RuntimeError(f"KV branch contract: cache batch {k.shape[0]} != {B}")
    elif candidate_cache_rows is not None:
        raise ValueError("candidate verification requires existing read-only KV")
    args.update = int(update_cache)
    if cross_kv is not None:
        args.cross_k, args.cross_v = cross_kv[0].data_ptr(), cross_kv[1].data_ptr()
    if out is None:
        out = torch.empty_like(x)
    else:
        _check(out.shape == x.shape and out.dtype in (torch.bfloat16, torch.float32) and out.device == dev
               and out.is_contiguous() and out.data_ptr() != x.data_ptr(),
               "out must be a separate [B, M, D] bf16 or fp32 tensor")
        _check(out.dtype == torch.bfloat16 or not debug, "debug outputs need a bf16 out")
    args.out = out.data_ptr()
    args.out_dtype = dtype_code(out)
    nbytes = _lib.lib().wam_block_workspace_bytes(B, M, D, bound.ffn_dim, ctx.shape[0],
                                                   ctx.shape[1], pool)
    if workspace is not None and workspace.numel() >= nbytes and workspace.device == dev:
        ws = workspace
    else:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    args.workspace, args.workspace_bytes = ws.data_ptr(), nbytes
    dbg = None
    if debug:
        R = B * M
        Lc = ctx.shape[0] * ctx.shape[1]
        F = bound.ffn_dim
        shapes = ([(R, D)] * 8 + [(Lc, D), (Lc, D)] + [(R, D)] * 3 + [(R, F), (R, D)]
                  + [(R, D)] * 5 + [(R, D), (Lc, D), (R, D), (R, F)] + [(R, D)] * 3
                  + [(temb.shape[0], temb.shape[1], 6, D)])
        # the block's residual stream is fp32, and so is the modulation table
        fp32 = ("residual1", "residual2", "modulation")
        dbg = {n: torch.empty(s, dtype=torch.float32 if n in fp32 else torch.bfloat16, device=dev)
               for n, s in zip(_lib.DEBUG_NAMES, shapes)}
        if cross_kv is not None:
            del dbg["cross_k_linear"]  # the context is not projected in this call
        arr = (ctypes.c_void_p * _lib.DEBUG_SLOTS)()
        for i, n in enumerate(_lib.DEBUG_NAMES):
            arr[i] = dbg[n].data_ptr() if n in dbg else None
        args.debug = ctypes.cast(arr, ctypes.c_void_p)
    if timer is not None:
        args.timer = timer
    _lib.check(_lib.lib().wam_block_forward(ctypes.byref(args), stream_handle(dev)),
               "wam_block_forward")
    # Keep the transient buffers alive until the stream has consumed them.
    ws.record_stream(torch.cuda.current_stream(dev))
    if debug:
        dbg["output"] = out
        return out, dbg
    return out


class NativeBlock:
    """Bind the original parameter tensors; forward contains no Torch math ops."""

    def __init__(self, block, fused_ffn1=False, mode="sequential"):
        if mode not in MODES:
            raise ValueError("mode must be sequential, tiled or persistent")
        self.mode = mode
        self.block = weakref.ref(block)
        self.fused_ffn1 = fused_ffn1
        self.weights = block_parameters(block)
        self.eps = block_eps(block)
        self._bound = None

    def bound(self):
        if self._bound is None:
            self._bound = BoundWeights(self.weights, self.eps, self.block().attn1.heads)
        return self._bound

    def __call__(self, hidden_states, encoder_hidden_states, temb, rotary_emb,
                 update_cache=0, cache_name="pos", candidate_cache_rows=None, debug=False):
        if torch.is_grad_enabled():
            raise RuntimeError("NativeBlock is inference-only; use no_grad/inference_mode")
        block = self.block()
        caches = block.attn1.attn_caches or {}
        cache = caches.get(cache_name)
        res = run_block(self.bound(), hidden_states, encoder_hidden_states, temb, rotary_emb,
                        cache, update_cache, candidate_cache_rows, debug=debug)
        if debug:
            out, dbg = res
            return dbg
        return res
