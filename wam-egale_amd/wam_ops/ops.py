"""Per-stage operators over torch tensors, each one C-ABI call into libwam_block.

These are the building blocks of the native block (native.py) and the units
the parity tests exercise one by one.  Tensors must be CUDA (HIP) tensors;
shape/dtype contract violations raise RuntimeError before any launch, like
the reference's TORCH_CHECKs (算子研究/wam_ops/optimized/csrc/block.cu:320-330).
"""
import ctypes
import math

import torch

from . import _lib
from ._lib import (EPI_BIAS, EPI_BIAS_GATE_RES, EPI_BIAS_GELU, EPI_BIAS_RES, WAM_BF16,
                   WAM_F32)

__all__ = ["linear", "ln_modulate", "layer_norm_affine", "rms_rope", "attention",
           "kv_layout", "kv_commit", "modulation", "stream_handle", "patchify",
           "timestep_embedding", "rows_linear", "rope_freqs", "head_norm",
           "EPI_BIAS", "EPI_BIAS_GELU", "EPI_BIAS_GATE_RES", "EPI_BIAS_RES"]


def _req(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def dtype_code(t):
    if t.dtype == torch.float32:
        return WAM_F32
    if t.dtype == torch.bfloat16:
        return WAM_BF16
    raise RuntimeError(f"unsupported dtype {t.dtype} (need float32 or bfloat16)")


def stream_handle(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _dev(*ts):
    dev = None
    for t in ts:
        if t is None:
            continue
        _req(t.is_cuda, "native operators need GPU tensors")
        if dev is None:
            dev = t.device
        _req(t.device == dev, "all tensors must be on one device")
    return dev


def _bf16(t, name):
    _req(t.dtype == torch.bfloat16, f"{name} must be bfloat16 (got {t.dtype})")


def modulation(table, temb, tokens):
    """Describe mod = table + temb for the C side.

    Block modulation: table [1, 6, D] or [6, D] (model.py:738-739), temb
    [B, L, 6, D] (model.py:751-759).  Output head: table [1, 2, D], temb
    [B, L, D], one vector for both shift and scale (model.py:1096-1101).
    L is 1 (per sample), the token count (per token), or a divisor of it: each
    temb row then serves tokens / L consecutive tokens (one latent frame)."""
    _req(table.is_contiguous() and temb.is_contiguous(), "table/temb must be contiguous")
    if temb.dim() == 3:
        mods, D = 1, temb.shape[2]
        _req(table.numel() == 2 * D, "the output head's scale_shift_table must hold 2 x D values")
    else:
        _req(temb.dim() == 4 and temb.shape[2] == 6, "temb must be [B, L, 6, D]")
        mods, D = 6, temb.shape[3]
        _req(table.numel() == 6 * D, "scale_shift_table must hold 6 x D values")
    L = temb.shape[1]
    _req(L >= 1 and tokens % L == 0,
         "temb length must be 1, the token count, or a divisor of it (one row per frame)")
    m = _lib.Modulation()
    m.table, m.table_dtype = table.data_ptr(), dtype_code(table)
    m.temb, m.temb_dtype = temb.data_ptr(), dtype_code(temb)
    m.temb_len, m.tokens, m.temb_mods = L, tokens, mods
    return m


FP8 = torch.float8_e4m3fn


def quantize_fp8_rows(w, out=None, scale=None):
    """Per-row e4m3 weights: scale[r] = max|w[r]| / 448, q = e4m3(w * (448 /
    max|w[r]|)) (round to nearest even).  Returns (q [rows, cols] float8_e4m3fn, scale fp32)."""
    dev = _dev(w)
    _bf16(w, "w")
    _req(w.dim() == 2 and w.stride(-1) == 1, "w must be [rows, cols] with contiguous rows")
    rows, cols = w.shape
    q = out if out is not None else torch.empty(rows, cols, dtype=FP8, device=dev)
    sc = scale if scale is not None else torch.empty(rows, dtype=torch.float32, device=dev)
    _req(q.dtype == FP8 and q.is_contiguous() and q.shape == (rows, cols), "q must be [rows, cols] e4m3")
    _req(sc.dtype == torch.float32 and sc.is_contiguous() and sc.numel() == rows, "scale must be [rows] fp32")
    _lib.check(_lib.lib().wam_quantize_fp8_rows(w.data_ptr(), rows, cols, w.stride(0), q.data_ptr(),
                                                 sc.data_ptr(), stream_handle(dev)), "wam_quantize_fp8_rows")
    return q, sc


def linear(x, weights, biases=None, *, epilogue=EPI_BIAS, residual=None, table=None,
           temb=None, tokens=None, gate_index=None, out=None, out_dtype=torch.bfloat16, w_scale=None,
           norm_gamma=None, norm_freq=None, norm_head_dim=128, x_scale=None, x_block_scale=None,
           mx_out=False):
    """Y = epilogue(x W^T + b) on MFMA.  weights: one tensor or a list of up to 3
    (one launch, outputs split per weight).  Returns a tensor or a list.
    The residual may be bf16 or fp32; out_dtype=float32 is allowed for the
    residual epilogues (the block keeps its residual stream in fp32).
    Weights may be float8_e4m3fn with per-output-column fp32 w_scale (one
    tensor or a list matching the weights): y = acc * w_scale + b.

    norm_gamma (the q/k-norm epilogue; one bf16 [N] tensor or None per
    segment): segment i with a gamma returns bf16(rope(y * gamma)) with
    y = bf16(x W^T + b), rotated by norm_freq (complex64 [Bf, tokens, 1 or
    absent, head_dim / 2], or None), and the call returns (outputs, sums)
    where sums[i] is the fp32 [M, ceil(N / 256)] sum of y^2 per row and
    256-column group (None for segments without a gamma).

    x may be float8_e4m3fn with x_scale, fp32 [M] per-row scales (from
    quantize_fp8_rows), when the weights are fp8 too: the product then runs
    on the fp8 MFMA, y = acc * x_scale[m] * w_scale[n] + b (bias or GELU
    epilogue, one weight, N a multiple of 256, K of 128).  mx_out=True (fp8
    x with x_scale) returns (q, e): q float8_e4m3fn [M, N] and e uint8 [M,
    N / 32], one e8m0 exponent per row and 32 columns (y = q * 2^(e - 127)).
    x may instead carry x_block_scale, uint8 [M, K / 32] e8m0 exponents of
    its 32-value blocks (an MX operand, e.g. an mx_out result): the MFMA
    applies them, y = acc * w_scale[n] + b with the bias, gated-residual or
    residual epilogue and a bf16 output."""
    single = torch.is_tensor(weights)
    ws = [weights] if single else list(weights)
    bs = [biases] if (single or biases is None) else list(biases)
    if biases is None:
        bs = [None] * len(ws)
    _req(1 <= len(ws) <= 3 and len(bs) == len(ws), "1 to 3 weight segments")
    f8 = ws[0].dtype == FP8
    scs = []
    if f8:
        _req(w_scale is not None, "fp8 weights need w_scale")
        scs = [w_scale] if torch.is_tensor(w_scale) else list(w_scale)
        _req(len(scs) == len(ws), "one w_scale per weight")
    else:
        _req(w_scale is None, "w_scale is only for fp8 weights")
    dev = _dev(x, *ws, *[b for b in bs if b is not None], residual, *scs, x_scale)
    x8 = x.dtype == FP8
    xmx = x8 and x_block_scale is not None
    if xmx:
        _req(f8 and x_scale is None and x_block_scale.dtype == torch.uint8 and x_block_scale.is_contiguous(),
             "MX activations need fp8 weights and uint8 x_block_scale [M, K / 32] (no x_scale)")
    elif x8:
        _req(f8 and x_scale is not None and x_scale.dtype == torch.float32 and x_scale.is_contiguous(),
             "fp8 activations need fp8 weights and fp32 x_scale [M]")
    else:
        _req(x_scale is None and x_block_scale is None, "x_scale / x_block_scale are only for fp8 activations")
        _bf16(x, "x")
    _req(not mx_out or (x8 and not xmx and single and out is None), "mx_out needs fp8 x with x_scale, one weight")
    _req(x.dim() >= 2 and x.stride(-1) == 1, "x must have a contiguous last dim")
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    M = x2.shape[0]
    N = ws[0].shape[0]
    for i, (w, b) in enumerate(zip(ws, bs)):
        if f8:
            _req(w.dtype == FP8, "all weights must share one dtype")
            _req(scs[i].dtype == torch.float32 and scs[i].is_contiguous() and scs[i].numel() == N,
                 "w_scale must be [N] fp32")
        else:
            _bf16(w, "weight")
        _req(w.is_contiguous() and w.shape == (N, K), f"weight must be [{N}, {K}] contiguous")
        if b is not None:
            _bf16(b, "bias")
            _req(b.is_contiguous() and b.numel() == N, "bias must be [N]")
    if mx_out:
        out_dtype = FP8
    outs = out if out is not None else [torch.empty(*x.shape[:-1], N, dtype=out_dtype, device=dev)
                                        for _ in ws]
    if torch.is_tensor(outs):
        outs = [outs]
    a = _lib.LinearArgs()
    a.a, a.lda, a.M, a.K = x2.data_ptr(), x2.stride(0), M, K
    a.n_seg, a.seg_n, a.ldw = len(ws), N, K
    for i, (w, b, o) in enumerate(zip(ws, bs, outs)):
        _req(o.is_contiguous() and o.numel() == M * N and o.dtype == out_dtype, "out shape/dtype")
        a.w[i] = w.data_ptr()
        a.bias[i] = b.data_ptr() if b is not None else None
        a.out[i] = o.data_ptr()
    a.ldo = N
    a.epilogue = epilogue
    if f8:
        a.w_dtype = _lib.WAM_FP8
        for i, sc in enumerate(scs):
            a.w_scale[i] = sc.data_ptr()
    mx_scale = None
    if mx_out:
        _req(N % 32 == 0, "mx_out needs N a multiple of 32")
        mx_scale = torch.empty(M, N // 32, dtype=torch.uint8, device=dev)
        a.out_dtype, a.out_block_scale = _lib.WAM_FP8_MX, mx_scale.data_ptr()
    else:
        a.out_dtype = dtype_code(outs[0])
    if xmx:
        _req(K % 32 == 0 and x_block_scale.shape == (M, K // 32), "x_block_scale must be [M, K / 32]")
        a.a_dtype, a.a_block_scale = _lib.WAM_FP8_MX, x_block_scale.data_ptr()
    elif x8:
        _req(x_scale.numel() == M, "x_scale must be [M]")
        a.a_dtype, a.a_scale = _lib.WAM_FP8, x_scale.data_ptr()
    ssqs = None
    if norm_gamma is not None:
        gs = [norm_gamma] if torch.is_tensor(norm_gamma) else list(norm_gamma)
        _req(len(gs) == len(ws) and any(g is not None for g in gs), "one norm gamma (or None) per segment")
        ssqs = []
        for i, g in enumerate(gs):
            if g is None:
                ssqs.append(None)
                continue
            _bf16(g, "norm gamma")
            _req(g.is_contiguous() and g.numel() == N and g.device == dev, "norm gamma must be [N]")
            sq = torch.empty(M, (N + 255) // 256, dtype=torch.float32, device=dev)
            a.norm_ssq[i], a.norm_gamma[i] = sq.data_ptr(), g.data_ptr()
            ssqs.append(sq)
        if norm_freq is not None:
            _req(norm_freq.dtype == torch.complex64 and norm_freq.is_contiguous() and norm_freq.device == dev,
                 "norm_freq must be contiguous complex64 on the device")
            _req(norm_freq.shape[-1] == norm_head_dim // 2, "norm_freq must be [Bf, tokens, 1, hd/2]")
            toks = norm_freq.shape[1]
            _req(M % toks == 0, "rows must be whole samples of the freq table's tokens")
            a.norm_freq, a.norm_freq_batch, a.norm_tokens = norm_freq.data_ptr(), norm_freq.shape[0], toks
            a.norm_head_dim = norm_head_dim
    if epilogue in (EPI_BIAS_GATE_RES, EPI_BIAS_RES):
        _req(residual is not None, "residual required")
        r2 = residual.reshape(-1, N)
        _req(r2.shape[0] == M and r2.stride(-1) == 1, "residual must be [M, N]")
        a.res, a.ldr, a.res_dtype = r2.data_ptr(), r2.stride(0), dtype_code(r2)
    if epilogue == EPI_BIAS_GATE_RES:
        _req(table is not None and temb is not None and gate_index is not None, "gate needs table/temb")
        a.gate = modulation(table, temb, tokens if tokens is not None else M)
        a.gate_index = gate_index
    scratch = None
    nbytes = _lib.lib().wam_linear_workspace_bytes(M, N, len(ws), K)
    if nbytes > 0:
        # fp32 partial sums of the split-K tail
        scratch = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        a.workspace, a.workspace_bytes = scratch.data_ptr(), nbytes
    _lib.check(_lib.lib().wam_linear(ctypes.byref(a), stream_handle(dev)), "wam_linear")
    if scratch is not None:
        scratch.record_stream(torch.cuda.current_stream(dev))
    res = outs[0] if single else outs
    if mx_out:
        return res, mx_scale
    if ssqs is not None:
        return res, (ssqs[0] if single else ssqs)
    return res


def ln_modulate(x, table, temb, shift_index, eps=1e-6, out=None, fp8=False, bf16_out=True):
    """bf16(LN(x) * (1 + mod[shift+1]) + mod[shift]), x [B, M, D] bf16 or fp32.

    fp8=True also writes the result as float8_e4m3fn rows with fp32 scales
    [B * M] (max |row| / 448, as quantize_fp8_rows of the bf16 result) and
    returns (y, q, scale); bf16_out=False then skips the bf16 output (y None)."""
    dev = _dev(x, table, temb)
    _req(x.dim() == 3 and x.is_contiguous(), "x must be [B, M, D] contiguous")
    _req(fp8 or bf16_out, "bf16_out=False needs fp8=True")
    B, M, D = x.shape
    y = None
    if bf16_out:
        y = out if out is not None else torch.empty(x.shape, dtype=torch.bfloat16, device=dev)
    a = _lib.LnArgs()
    a.x, a.y, a.rows, a.D, a.eps, a.affine = x.data_ptr(), y.data_ptr() if y is not None else None, B * M, D, eps, 0
    a.x_dtype = dtype_code(x)
    a.mod = modulation(table, temb, M)
    a.shift_index = shift_index
    if fp8:
        q = torch.empty(x.shape, dtype=FP8, device=dev)
        sc = torch.empty(B * M, dtype=torch.float32, device=dev)
        a.y8, a.y8_scale = q.data_ptr(), sc.data_ptr()
    _lib.check(_lib.lib().wam_ln_modulate(ctypes.byref(a), stream_handle(dev)), "wam_ln_modulate")
    return (y, q, sc) if fp8 else y


def layer_norm_affine(x, gamma, beta, eps=1e-6, out=None):
    """bf16(LN(x) * gamma + beta) with fp32 statistics (norm2); x bf16 or fp32."""
    dev = _dev(x, gamma, beta)
    _req(x.is_contiguous(), "x must be contiguous")
    D = x.shape[-1]
    _req(gamma.numel() == D and beta.numel() == D and gamma.dtype == beta.dtype, "gamma/beta [D]")
    y = out if out is not None else torch.empty(x.shape, dtype=torch.bfloat16, device=dev)
    a = _lib.LnArgs()
    a.x, a.y, a.rows, a.D, a.eps, a.affine = x.data_ptr(), y.data_ptr(), x.numel() // D, D, eps, 1
    a.x_dtype = dtype_code(x)
    a.gamma, a.beta, a.gb_dtype = gamma.data_ptr(), beta.data_ptr(), dtype_code(gamma)
    _lib.check(_lib.lib().wam_ln_modulate(ctypes.byref(a), stream_handle(dev)), "wam_ln_modulate")
    return y


def rms_rope(tensors, gammas, eps, freq=None, head_dim=128, out=None):
    """RMSNorm across the full row (+ RoPE when freq is given) for 1-2 tensors
    [B, M, D] bf16.  freq: complex64 [Bf, M, 1 or absent, head_dim/2]."""
    ts = list(tensors)
    gs = list(gammas)
    es = list(eps) if isinstance(eps, (list, tuple)) else [eps] * len(ts)
    dev = _dev(*ts, *gs, freq)
    _req(1 <= len(ts) <= 2 and len(gs) == len(ts), "1 or 2 tensors")
    B, M, D = ts[0].shape
    outs = out if out is not None else [torch.empty_like(t) for t in ts]
    a = _lib.RmsRopeArgs()
    for i, (t, g, o) in enumerate(zip(ts, gs, outs)):
        _bf16(t, "x")
        _bf16(g, "gamma")
        _req(t.shape == (B, M, D) and t.stride(-1) == 1 and t.stride(0) == M * t.stride(1),
             "rms_rope tensors must be [B, M, D] with unit last stride")
        _req(g.numel() == D, "gamma must be [D]")
        a.x[i], a.y[i], a.gamma[i], a.eps[i] = t.data_ptr(), o.data_ptr(), g.data_ptr(), es[i]
    _req(all(t.stride(1) == ts[0].stride(1) for t in ts), "equal row strides")
    a.ldx, a.ldy = ts[0].stride(1), outs[0].stride(1)
    a.n_tensors, a.rows, a.D, a.head_dim = len(ts), B * M, D, head_dim
    if freq is not None:
        _req(freq.dtype == torch.complex64 and freq.is_contiguous(), "freq must be contiguous complex64")
        _req(freq.shape[1] == M and freq.shape[-1] == head_dim // 2, "freq must be [Bf, M, 1, hd/2]")
        a.freq, a.freq_batch, a.tokens = freq.data_ptr(), freq.shape[0], M
    _lib.check(_lib.lib().wam_rms_rope(ctypes.byref(a), stream_handle(dev)), "wam_rms_rope")
    return outs


def attention(q, k, v, *, pool_k=None, pool_v=None, slots=None, n_hist=None, pool_rows=None,
              kv_rows=None, scale=None, out=None, q_ssq=None, q_eps=1e-6, hist_base=None):
    """softmax(q [history || k]^T / sqrt(hd)) [history || v] per head.

    q [B, Mq, H, 128]; k, v [Bk, Mk, H, 128] (any row stride, unit last dim);
    history = pool_k/pool_v [Bp, P, H, 128] at slots[:n_hist] (int32, device),
    pool row pool_rows[b] (int64) or b; own row kv_rows[b] or b.
    q_ssq: fp32 [B * Mq, n] partial sums of squares of each query row (the
    norm epilogue of linear); query rows are then scaled by
    rsqrt(sum / (H * 128) + q_eps) (RMSNorm across heads).
    hist_base: int32 device scalar (kv_layout's info[2]); when it holds
    s >= 0 the caller asserts slots[j] == s + j and the kernel reads the pool
    rows at that base instead of through the slot list."""
    dev = _dev(q, k, v, pool_k, pool_v, slots, n_hist, pool_rows, kv_rows)
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _bf16(t, n)
        _req(t.dim() == 4 and t.shape[-1] == 128 and t.stride(-1) == 1 and t.stride(-2) == 128,
             f"{n} must be [B, M, H, 128] with packed heads")
    B, Mq, H, hd = q.shape
    _req(k.shape == v.shape and k.shape[2] == H and k.stride() == v.stride(), "k/v shape")
    o = out if out is not None else torch.empty(B, Mq, H, hd, dtype=torch.bfloat16, device=dev)
    a = _lib.AttentionArgs()
    a.q, a.q_bstride, a.q_rstride = q.data_ptr(), q.stride(0), q.stride(1)
    a.o, a.o_bstride, a.o_rstride = o.data_ptr(), o.stride(0), o.stride(1)
    a.B, a.Mq, a.H, a.head_dim = B, Mq, H, hd
    if n_hist is not None:
        _req(n_hist.dtype == torch.int32 and slots.dtype == torch.int32, "slots/n_hist are int32")
        for t in (pool_k, pool_v):
            _bf16(t, "pool")
            _req(t.is_contiguous() and t.shape[2:] == (H, hd), "pool must be [Bp, P, H, 128]")
        a.pool_k, a.pool_v = pool_k.data_ptr(), pool_v.data_ptr()
        a.pool_bstride, a.pool_rstride = pool_k.stride(0), pool_k.stride(1)
        a.pool_batch = pool_k.shape[0]
        a.slots, a.n_hist_dev = slots.data_ptr(), n_hist.data_ptr()
        if hist_base is not None:
            _req(hist_base.dtype == torch.int32 and hist_base.device == dev, "hist_base is an int32 device scalar")
            a.hist_base_dev = hist_base.data_ptr()
        if pool_rows is not None:
            _req(pool_rows.dtype == torch.int64 and pool_rows.numel() == B, "pool_rows int64 [B]")
            a.pool_rows = pool_rows.data_ptr()
    a.k, a.v, a.kv_bstride, a.kv_rstride = k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1)
    a.Mk, a.kv_batch = k.shape[1], k.shape[0]
    if kv_rows is not None:
        _req(kv_rows.dtype == torch.int64 and kv_rows.numel() == B, "kv_rows int64 [B]")
        a.kv_rows = kv_rows.data_ptr()
    a.scale = scale if scale is not None else 1.0 / math.sqrt(hd)
    if q_ssq is not None:
        _req(q_ssq.dtype == torch.float32 and q_ssq.is_contiguous() and q_ssq.dim() == 2 and
             q_ssq.shape[0] == B * Mq and q_ssq.device == dev, "q_ssq must be fp32 [B * Mq, n]")
        a.q_ssq, a.q_ssq_n, a.q_norm_dim, a.q_eps = q_ssq.data_ptr(), q_ssq.shape[1], H * hd, q_eps
    # the key count bound plans the split: own keys plus the whole pool
    a.max_keys = a.Mk + (pool_k.shape[1] if n_hist is not None else 0)
    ws = None
    nbytes = _lib.lib().wam_attention_workspace_bytes(a.B, a.Mq, a.H, a.max_keys)
    if nbytes > 0:
        # partial results of the key-range splits
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    _lib.check(_lib.lib().wam_attention(ctypes.byref(a), stream_handle(dev)), "wam_attention")
    if ws is not None:
        ws.record_stream(torch.cuda.current_stream(dev))
    return o


def kv_layout(cache, tokens, update, candidate_rows=None):
    """Pool bookkeeping of one self-attention call; mutates cache['mask'/'id'/'is_pred']
    unless candidate_rows is given.  Returns (hist_slots, new_slots, info) int32."""
    mask, ids, pred = cache["mask"], cache["id"], cache["is_pred"]
    dev = _dev(mask, ids, pred, candidate_rows)
    _req(mask.dtype == torch.bool and pred.dtype == torch.bool and ids.dtype == torch.int64,
         "cache schema: mask/is_pred bool, id int64")
    P = mask.numel()
    hist = torch.empty(P, dtype=torch.int32, device=dev)
    new = torch.empty(max(tokens, 1), dtype=torch.int32, device=dev)
    info = torch.zeros(4, dtype=torch.int32, device=dev)
    a = _lib.KvLayoutArgs()
    a.mask, a.ids, a.is_pred, a.pool = mask.data_ptr(), ids.data_ptr(), pred.data_ptr(), P
    a.tokens, a.update = tokens, update
    a.candidate = 0 if candidate_rows is None else 1
    if candidate_rows is not None:
        a.rows, a.batch, a.pool_batch = candidate_rows.data_ptr(), candidate_rows.numel(), cache["k"].shape[0]
    a.hist_slots, a.new_slots, a.info = hist.data_ptr(), new.data_ptr(), info.data_ptr()
    _lib.check(_lib.lib().wam_kv_layout(ctypes.byref(a), stream_handle(dev)), "wam_kv_layout")
    return hist, new, info


def kv_commit(cache, k, v, new_slots):
    """pool[b, new_slots[t]] = k[b, t] (and v), k/v [B, M, D] with unit last stride."""
    dev = _dev(k, v, cache["k"], new_slots)
    B, M = k.shape[:2]
    D = cache["k"].shape[2] * cache["k"].shape[3]
    a = _lib.KvCommitArgs()
    a.k, a.v, a.ld = k.data_ptr(), v.data_ptr(), k.stride(1)
    a.pool_k, a.pool_v = cache["k"].data_ptr(), cache["v"].data_ptr()
    a.pool_bstride, a.pool_rstride = cache["k"].stride(0), cache["k"].stride(1)
    a.new_slots, a.B, a.tokens, a.D = new_slots.data_ptr(), B, M, D
    _lib.check(_lib.lib().wam_kv_commit(ctypes.byref(a), stream_handle(dev)), "wam_kv_commit")


# ---------------------------------------------------------- model input / output
def patchify(latents, patch, k_pad=None, out=None):
    """'b c (f p1) (h p2) (w p3) -> b (f h w) (c p1 p2 p3)' of bf16 latents
    [B, C, F, H, W] (model.py:1064-1069; patch (1, 1, 1) is the action path's
    'b c f h w -> b (f h w) c').  Returns [B, L, k_pad] bf16 whose columns
    past C*p1*p2*p3 are zero (k_pad defaults to that product)."""
    dev = _dev(latents)
    _bf16(latents, "latents")
    _req(latents.dim() == 5 and latents.is_contiguous(), "latents must be [B, C, F, H, W] contiguous")
    B, C, F, H, W = latents.shape
    p1, p2, p3 = (int(v) for v in patch)
    _req(F % p1 == 0 and H % p2 == 0 and W % p3 == 0, "latent F/H/W must be multiples of the patch")
    K = C * p1 * p2 * p3
    k_pad = K if k_pad is None else int(k_pad)
    L = (F // p1) * (H // p2) * (W // p3)
    y = out if out is not None else torch.empty(B, L, k_pad, dtype=torch.bfloat16, device=dev)
    _req(y.dtype == torch.bfloat16 and y.is_contiguous() and y.numel() == B * L * k_pad, "out [B, L, k_pad]")
    a = _lib.PatchifyArgs()
    a.x, a.out = latents.data_ptr(), y.data_ptr()
    a.B, a.C, a.F, a.H, a.W = B, C, F, H, W
    a.p1, a.p2, a.p3, a.k_pad = p1, p2, p3, k_pad
    _lib.check(_lib.lib().wam_patchify(ctypes.byref(a), stream_handle(dev)), "wam_patchify")
    return y


def timestep_embedding(t, dim=256, flip_sin_to_cos=True, shift=0.0, max_period=10000.0,
                       out_dtype=torch.float32, out=None):
    """diffusers Timesteps (get_timestep_embedding): t [R] fp32 -> [R, dim]."""
    dev = _dev(t)
    _req(t.dtype == torch.float32 and t.is_contiguous(), "timesteps must be contiguous float32")
    R = t.numel()
    y = out if out is not None else torch.empty(R, dim, dtype=out_dtype, device=dev)
    _req(y.is_contiguous() and y.shape == (R, dim), "out must be [R, dim]")
    a = _lib.TimestepArgs()
    a.t, a.rows, a.dim, a.flip_sin_to_cos = t.data_ptr(), R, dim, int(bool(flip_sin_to_cos))
    a.shift, a.max_period, a.out, a.out_dtype = shift, max_period, y.data_ptr(), dtype_code(y)
    _lib.check(_lib.lib().wam_timestep_embedding(ctypes.byref(a), stream_handle(dev)),
               "wam_timestep_embedding")
    return y


_ACTS = {None: _lib.WAM_ACT_NONE, "silu": _lib.WAM_ACT_SILU}


def rows_linear(x, w, b=None, act_in=None, act_out=None, out_dtype=None, out=None):
    """out = act_out(act_in(x) W^T + b) for few rows on the vector ALUs; x, w,
    b and out may each be float32 or bfloat16 (torch's per-op roundings)."""
    dev = _dev(x, w, b)
    _req(x.dim() >= 1 and x.stride(-1) == 1 and w.dim() == 2 and w.stride(-1) == 1,
         "x and w need contiguous rows")
    K = x.shape[-1]
    N = w.shape[0]
    _req(w.shape[1] == K, f"weight must be [N, {K}]")
    x2 = x.reshape(-1, K)
    R = x2.shape[0]
    _req(act_in in _ACTS and act_out in _ACTS, "activations: None or 'silu'")
    y = out if out is not None else torch.empty(*x.shape[:-1], N, dtype=out_dtype or x.dtype, device=dev)
    _req(y.is_contiguous() and y.numel() == R * N, "out must be [..., N] contiguous")
    a = _lib.RowsLinearArgs()
    a.x, a.x_dtype, a.ldx = x2.data_ptr(), dtype_code(x2), x2.stride(0)
    a.w, a.w_dtype, a.ldw = w.data_ptr(), dtype_code(w), w.stride(0)
    if b is not None:
        _req(b.is_contiguous() and b.numel() == N, "bias must be [N]")
        a.bias, a.bias_dtype = b.data_ptr(), dtype_code(b)
    a.out, a.out_dtype, a.ldo = y.data_ptr(), dtype_code(y), N
    a.R, a.N, a.K = R, N, K
    a.act_in, a.act_out = _ACTS[act_in], _ACTS[act_out]
    _lib.check(_lib.lib().wam_rows_linear(ctypes.byref(a), stream_handle(dev)), "wam_rows_linear")
    return y


def rope_freqs(grid_ids, head_dim=128, theta=10000.0, out=None):
    """WanRotaryPosEmbed.forward: grid ids [B, >=3, L] (int64, float32 or
    float64) -> complex64 [B, L, 1, head_dim/2] (model.py:276-286, with the
    [:, :, None] of model.py:1077)."""
    dev = _dev(grid_ids)
    codes = {torch.int64: _lib.WAM_I64, torch.float32: _lib.WAM_F32, torch.float64: _lib.WAM_F64}
    _req(grid_ids.dtype in codes, "grid ids must be int64, float32 or float64")
    _req(grid_ids.dim() == 3 and grid_ids.shape[1] >= 3, "grid ids must be [B, >=3, L]")
    B, _, L = grid_ids.shape
    y = out if out is not None else torch.empty(B, L, 1, head_dim // 2, dtype=torch.complex64, device=dev)
    _req(y.dtype == torch.complex64 and y.is_contiguous() and y.numel() == B * L * (head_dim // 2),
         "out must be complex64 [B, L, 1, head_dim/2]")
    a = _lib.RopeFreqArgs()
    a.grid, a.grid_dtype = grid_ids.data_ptr(), codes[grid_ids.dtype]
    a.grid_bstride, a.grid_rstride, a.grid_lstride = grid_ids.stride()
    a.B, a.L, a.head_dim, a.theta, a.out = B, L, head_dim, theta, y.data_ptr()
    _lib.check(_lib.lib().wam_rope_freqs(ctypes.byref(a), stream_handle(dev)), "wam_rope_freqs")
    return y


def head_norm(x, table, temb, eps=1e-6, out=None):
    """norm_out + modulation of the output head (model.py:1096-1103):
    bf16(LN(x) * (1 + table[1] + temb) + table[0] + temb), x [B, M, D],
    table [1, 2, D] fp32, temb [B, L, D] with L dividing M."""
    dev = _dev(x, table, temb)
    _req(x.dim() == 3 and x.is_contiguous(), "x must be [B, M, D] contiguous")
    B, M, D = x.shape
    _req(temb.dim() == 3 and temb.shape[0] == B and temb.shape[2] == D, "temb must be [B, L, D]")
    y = out if out is not None else torch.empty(x.shape, dtype=torch.bfloat16, device=dev)
    a = _lib.LnArgs()
    a.x, a.y, a.rows, a.D, a.eps, a.affine = x.data_ptr(), y.data_ptr(), B * M, D, eps, 0
    a.x_dtype = dtype_code(x)
    a.mod = modulation(table, temb, M)
    a.shift_index = 0
    _lib.check(_lib.lib().wam_ln_modulate(ctypes.byref(a), stream_handle(dev)), "wam_ln_modulate")
    return y
