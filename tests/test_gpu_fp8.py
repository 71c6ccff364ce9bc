"""fp8 e4m3 weights (per-output-channel fp32 scales) with bf16 activations.

* wam_quantize_fp8_rows is bit-exact against the oracle's quantization.
* wam_linear with fp8 weights matches an fp32 reference that uses the same
  dequantized weights, at the bf16 GEMM bound (the quantization is shared, only
  the accumulation order differs).
* The FFN unit (FFN1 + GELU(tanh) + FFN2 + gated residual, M=4680, 3072 ->
  14336 -> 3072) in the fp8 variant, against the fp32 reference with the
  ORIGINAL bf16 weights: the looser fp8 bound, max |err| <= 0.25, relative L2
  <= 2e-2 and cosine >= 0.9999 (the e4m3 rounding of every weight, about 2^-5
  relative RMS, is the dominant term; measured 0.135 / 0.0092 / 0.99996);
  against the dequantized-weight reference: 2e-2 / 0.9999.
"""
import pytest
import torch

from oracle import fp8 as ofp8
from oracle.metrics import assert_close, compare

pytestmark = pytest.mark.gpu


def _randn(shape, dev, seed, std=1.0, dtype=torch.bfloat16):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=dev) * std).to(dtype)


def _ulp_bound(ref):
    return 2 ** -8 * ref.abs().max().item() + 2e-3


def test_quantize_rows_bit_exact(dev):
    from wam_ops import ops
    w = _randn((300, 512), dev, 1, 0.02)
    w[7] = 0
    w[11] *= 1e4
    w[12] *= 1e-4
    w[13, 5] = 3.0  # one outlier sets the row scale
    q, s = ops.quantize_fp8_rows(w)
    torch.cuda.synchronize()
    qr, sr = ofp8.quantize_rows(w.cpu())
    assert torch.equal(s.cpu(), sr)
    assert torch.equal(q.cpu().view(torch.uint8), qr.view(torch.uint8))
    # strided rows (ldw > cols)
    wide = _randn((64, 1024), dev, 2, 0.02)
    q2, s2 = ops.quantize_fp8_rows(wide[:, :512])
    qr2, sr2 = ofp8.quantize_rows(wide[:, :512].cpu())
    assert torch.equal(q2.cpu().view(torch.uint8), qr2.view(torch.uint8)) and torch.equal(s2.cpu(), sr2)


# (6240, 3072, 2816): 275 256x256 tiles; the last column of tiles runs split
# over k in 8 ranges (fp32 partials, reduce pass with scale + epilogue).
@pytest.mark.parametrize("M,K,N", [(130, 1024, 2048), (4680, 256, 3584), (4680, 512, 14336),
                                   (6240, 3072, 2816)])
def test_fp8_linear_epilogues(dev, M, K, N):
    from wam_ops import ops
    x = _randn((M, K), dev, 3)
    w = _randn((N, K), dev, 4, 0.05)
    b = _randn((N,), dev, 5, 0.05)
    q, s = ops.quantize_fp8_rows(w)
    wd = ofp8.dequantize_rows(q.cpu(), s.cpu()).to(dev)
    ref = x.float() @ wd.t() + b.float()
    y = ops.linear(x, q, b, w_scale=s)
    assert_close(y, ref, _ulp_bound(ref), 0.99999, f"fp8 bias {M}x{K}x{N}")
    y = ops.linear(x, q, b, w_scale=s, epilogue=ops.EPI_BIAS_GELU)
    g = torch.nn.functional.gelu(ref, approximate="tanh")
    assert_close(y, g, _ulp_bound(g), 0.99999, "fp8 gelu")
    res32 = _randn((M, N), dev, 6, 1.0, torch.float32)
    table = _randn((1, 6, N), dev, 7, 0.1, torch.float32)
    temb = _randn((1, 1, 6, N), dev, 8, 0.1, torch.float32)
    gate = (table[0, 5] + temb[0, 0, 5])[None]
    y = ops.linear(x, q, b, w_scale=s, epilogue=ops.EPI_BIAS_GATE_RES, residual=res32, table=table,
                   temb=temb, tokens=M, gate_index=5, out_dtype=torch.float32)
    r = res32 + ref * gate
    assert_close(y, r, 2e-3 + 2 ** -16 * r.abs().max().item(), 0.999999, "fp8 gated residual fp32")


def test_fp8_rejects_missing_scale(dev):
    from wam_ops import ops
    x = _randn((8, 128), dev, 1)
    q, s = ops.quantize_fp8_rows(_randn((128, 128), dev, 2, 0.02))
    with pytest.raises(RuntimeError, match="w_scale"):
        ops.linear(x, q, None)


def test_fp8_ffn_unit_vs_fp32(dev):
    """The C3 FFN unit at its full size, fp8 weights vs the bf16 weights."""
    from wam_ops import ops
    M, D, F = 4680, 3072, 14336
    x = _randn((M, D), dev, 11)
    w1 = _randn((F, D), dev, 12, 0.02)
    b1 = _randn((F,), dev, 13, 0.02)
    w2 = _randn((D, F), dev, 14, 0.02)
    b2 = _randn((D,), dev, 15, 0.02)
    res = _randn((M, D), dev, 16, 1.0, torch.float32)
    table = _randn((1, 6, D), dev, 17, 0.1, torch.float32)
    temb = _randn((1, 1, 6, D), dev, 18, 0.1, torch.float32)
    gate = (table[0, 5] + temb[0, 0, 5])[None]
    q1, s1 = ops.quantize_fp8_rows(w1)
    q2, s2 = ops.quantize_fp8_rows(w2)
    h = ops.linear(x, q1, b1, w_scale=s1, epilogue=ops.EPI_BIAS_GELU)
    y = ops.linear(h, q2, b2, w_scale=s2, epilogue=ops.EPI_BIAS_GATE_RES, residual=res, table=table,
                   temb=temb, tokens=M, gate_index=5, out_dtype=torch.float32)
    torch.cuda.synchronize()
    ref_q = ofp8.ffn_gated(x, ofp8.dequantize_rows(q1, s1), b1, ofp8.dequantize_rows(q2, s2), b2, res, gate)
    m = assert_close(y, ref_q, 2e-2, 0.9999, "fp8 FFN vs dequantized fp32")
    ref = ofp8.ffn_gated(x, w1, b1, w2, b2, res, gate)
    m2 = assert_close(y, ref, 0.25, 0.9999, "fp8 FFN vs bf16-weight fp32")
    assert m2["rel_l2"] <= 2e-2, m2
    print("fp8 FFN unit", m, m2, compare(y - res, ref - res))


def test_block_with_fp8_ffn(dev):
    """The whole block with the fp8 FFN: against the fp32 oracle fed the
    dequantized FFN weights at the block bound, and against the bf16-weight
    oracle at the fp8 bound."""
    from oracle.block import block_forward
    from wam_ops import synthetic
    from wam_ops.block import TransformerBlock
    from wam_ops.whole_layer import WholeLayerBlock
    shape = synthetic.BlockShape(3072, 24, 14336)
    params = synthetic.block_params(shape, seed=21)
    x, ctx, temb, freqs = synthetic.block_inputs(shape, 1, 4 * 8 * 8, (4, 8, 8), context_len=512, seed=22)
    blk = TransformerBlock(shape.dim, shape.ffn, shape.heads, cross_attn_norm=True, eps=shape.eps)
    with torch.no_grad():
        for name, prm in blk.named_parameters():
            prm.data = params[name].to(dev)
    wl = WholeLayerBlock(blk.to(dev), ffn_fp8=True)
    with torch.no_grad():
        wl.prepare_context(ctx.to(dev), precompute=True)
        out = wl(x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev))
    torch.cuda.synchronize()
    q1, s1, q2, s2 = wl.bound().ffn_fp8
    pq = dict(params)
    pq["ffn.net.0.proj.weight"] = ofp8.dequantize_rows(q1.cpu(), s1.cpu())
    pq["ffn.net.2.weight"] = ofp8.dequantize_rows(q2.cpu(), s2.cpu())
    ref_q = block_forward(pq, x, ctx, temb, freqs, shape.heads, shape.eps)
    assert_close(out.cpu(), ref_q, 2e-2, 0.9999, "block fp8 FFN vs dequantized oracle")
    ref = block_forward(params, x, ctx, temb, freqs, shape.heads, shape.eps)
    m = assert_close(out.cpu(), ref, 0.25, 0.9999, "block fp8 FFN vs bf16-weight oracle")
    print("block fp8 FFN", m)


# fp8 activations on the fp8 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4): the
# activations are quantized per row like the weights (absmax / 448).  Against
# an fp32 product of the same dequantized operands the only differences are
# the accumulation order and the output rounding: the bf16 ulp bound.  Against
# the original bf16 operands, the e4m3 rounding of both (about 2^-5 relative
# RMS each, so about 3% per output) is the bound's dominant term: relative L2
# <= 5e-2, cosine >= 0.998 (a single row has only N outputs to average over).
@pytest.mark.parametrize("M,K,N", [(4680, 3072, 14336), (300, 256, 512), (4680, 128, 256), (1, 3072, 256)])
def test_fp8_activations_linear(dev, M, K, N):
    from wam_ops import ops
    print(f"fp8 x fp8 linear {M}x{K}x{N}", flush=True)
    x = _randn((M, K), dev, 21)
    w = _randn((N, K), dev, 22, 0.02)
    b = _randn((N,), dev, 23, 0.02)
    qw, sw = ops.quantize_fp8_rows(w)
    qx, sx = ops.quantize_fp8_rows(x)
    xd = ofp8.dequantize_rows(qx.cpu(), sx.cpu()).to(dev)
    wd = ofp8.dequantize_rows(qw.cpu(), sw.cpu()).to(dev)
    ref = xd @ wd.t() + b.float()
    y = ops.linear(qx, qw, b, w_scale=sw, x_scale=sx)
    assert_close(y, ref, _ulp_bound(ref), 0.99999, f"fp8 x fp8 bias {M}x{K}x{N}")
    y = ops.linear(qx, qw, b, w_scale=sw, x_scale=sx, epilogue=ops.EPI_BIAS_GELU)
    g = torch.nn.functional.gelu(ref, approximate="tanh")
    assert_close(y, g, _ulp_bound(g), 0.99999, f"fp8 x fp8 gelu {M}x{K}x{N}")
    full = x.float() @ w.float().t() + b.float()
    m = compare(ops.linear(qx, qw, b, w_scale=sw, x_scale=sx), full)
    print(f"fp8 x fp8 vs bf16 operands: {m}")
    assert m["rel_l2"] <= 5e-2 and m["cosine"] >= 0.998, m


def test_fp8_activations_rejected_without_fp8_weights(dev):
    from wam_ops import ops
    x = _randn((64, 256), dev, 1)
    w = _randn((256, 256), dev, 2, 0.02)
    qx, sx = ops.quantize_fp8_rows(x)
    with pytest.raises(RuntimeError):
        ops.linear(qx, w, None, x_scale=sx)
    qw, sw = ops.quantize_fp8_rows(w)
    with pytest.raises(RuntimeError, match="fp8 activations"):
        ops.linear(qx, qw, None, w_scale=sw, x_scale=sx, epilogue=ops.EPI_BIAS_RES,
                   residual=torch.zeros(64, 256, device=dev))


# LayerNorm 3 with e4m3 rows: the fused quantization equals the row quantizer
# applied to the kernel's own bf16 output, byte for byte (and the oracle's
# quantization of it), for every row-chunk count of the kernel (D 128, 1024,
# 3072, 4096), fp32 and bf16 inputs, a row count that leaves a partial
# workgroup, per-token modulation, and an all-zero output row (scale 1).
@pytest.mark.parametrize("D", [128, 1024, 3072, 4096])
@pytest.mark.parametrize("xdtype", [torch.float32, torch.bfloat16])
def test_ln_modulate_fp8_rows(dev, D, xdtype):
    from wam_ops import ops
    B, M = 2, 13
    g = torch.Generator(device=dev).manual_seed(D)
    x = (torch.randn(B, M, D, generator=g, device=dev) * 3).to(xdtype)
    table = torch.randn(1, 6, D, generator=g, device=dev) * 0.1
    temb = torch.randn(B, M, 6, D, generator=g, device=dev) * 0.1
    x[1, 4] = 1.5            # constant row: LN gives 0 ...
    table[0, 3] = 0
    temb[1, 4, 3] = 0        # ... and a zero shift keeps it 0
    y, q, sc = ops.ln_modulate(x, table, temb, 3, fp8=True)
    y_only = ops.ln_modulate(x, table, temb, 3)
    _, q2, sc2 = ops.ln_modulate(x, table, temb, 3, fp8=True, bf16_out=False)
    qr, sr = ops.quantize_fp8_rows(y_only.reshape(B * M, D))
    torch.cuda.synchronize()
    assert torch.equal(y, y_only)
    assert torch.equal(q.view(torch.uint8).reshape(B * M, D), qr.view(torch.uint8))
    assert torch.equal(sc, sr)
    assert torch.equal(q2.view(torch.uint8), q.view(torch.uint8)) and torch.equal(sc2, sc)
    assert sc[B * M - M + 4].item() == 1.0 and not q.view(torch.uint8)[1, 4].any()
    qo, so = ofp8.quantize_rows(y_only.reshape(B * M, D).cpu())
    assert torch.equal(sc.cpu(), so) and torch.equal(q.cpu().view(torch.uint8).reshape(B * M, D), qo.view(torch.uint8))


@pytest.mark.parametrize("mode", [1, 2])
def test_block_with_fp8_ffn_activations(dev, mode):
    """The block with e4m3 FFN weights and e4m3 FFN1 activations (quantized
    per row inside LayerNorm 3); mode 2 also hands the hidden layer to FFN2
    as MX e4m3 (both FFN GEMMs on the fp8 MFMA).  FFN1 before GELU against
    the fp32 product of the oracle's quantization of the block's own
    LayerNorm-3 rows and the dequantized weight: the bf16 ulp bound (only the
    accumulation order and the output rounding differ).  Mode 2: the hidden
    layer (dequantized debug copy) within half an e4m3 step of GELU of that
    product plus the bf16 bound, and FFN2 before the gate against the fp32
    product of that hidden layer and the dequantized weight at the bf16 ulp
    bound.  The output against the bf16-weight oracle at the fp8 bound; a
    debug call leaves the output unchanged."""
    from oracle.block import block_forward
    from wam_ops import synthetic
    from wam_ops.block import TransformerBlock
    from wam_ops.whole_layer import WholeLayerBlock
    shape = synthetic.BlockShape(3072, 24, 14336)
    params = synthetic.block_params(shape, seed=21)
    x, ctx, temb, freqs = synthetic.block_inputs(shape, 1, 4 * 8 * 8, (4, 8, 8), context_len=512, seed=22)
    blk = TransformerBlock(shape.dim, shape.ffn, shape.heads, cross_attn_norm=True, eps=shape.eps)
    with torch.no_grad():
        for name, prm in blk.named_parameters():
            prm.data = params[name].to(dev)
    wl = WholeLayerBlock(blk.to(dev), ffn_fp8=True, ffn_act_fp8=mode)
    with torch.no_grad():
        wl.prepare_context(ctx.to(dev), precompute=True)
        out = wl(x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev))
        dbg = wl(x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev), debug=True)
    torch.cuda.synchronize()
    assert torch.equal(dbg["output"], out), "a debug call changed the block output"
    q1, s1, q2, s2 = wl.bound().ffn_fp8
    h = dbg["modulated3"].reshape(-1, shape.dim).cpu()
    qh, sh = ofp8.quantize_rows(h)
    ffn1 = ofp8.dequantize_rows(qh, sh) @ ofp8.dequantize_rows(q1.cpu(), s1.cpu()).t() \
        + params["ffn.net.0.proj.bias"].float()
    got = dbg["ffn1"].reshape(ffn1.shape).cpu()
    assert_close(got, ffn1, _ulp_bound(ffn1), 0.99999, f"block fp8 FFN1 (fp8 activations, mode {mode})")
    if mode == 2:
        g = torch.nn.functional.gelu(ffn1, approximate="tanh")
        hid = dbg["gelu"].reshape(g.shape).cpu().float()
        assert ((hid - g).abs() <= g.abs() * 2 ** -4 + _ulp_bound(g)).all()
        ffn2 = hid @ ofp8.dequantize_rows(q2.cpu(), s2.cpu()).t() + params["ffn.net.2.bias"].float()
        got2 = dbg["ffn2"].reshape(ffn2.shape).cpu()
        assert_close(got2, ffn2, _ulp_bound(ffn2), 0.99999, "block MX FFN2 (before the gate)")
    ref = block_forward(params, x, ctx, temb, freqs, shape.heads, shape.eps)
    m = assert_close(out.cpu(), ref, 0.5, 0.9995, f"block fp8 FFN activations mode {mode} vs bf16-weight oracle")
    print(f"block fp8 FFN activations mode {mode}", m)


# MX output of the fp8 MFMA (the FFN1 -> FFN2 hand-over of the fp8 FFN): e4m3
# with one e8m0 exponent per row and 32 columns.  The same launch with a bf16
# output rounds the same fp32 values y (same tiles, accumulation order and
# epilogue math), so against that bf16 output yb: every value is within half
# an e4m3 step at its block's exponent X (max(|yb| 2^-4, 2^(X-10))) plus the
# bf16 rounding of yb (2^-8 |yb|); the exponents equal the oracle's rule on
# the block maxima of yb except where the bf16 rounding of a maximum can
# cross the rule's boundary (then by one).  Every nonzero block's largest
# |q| lies in [224, 448]: the exponent is the smallest that keeps the block
# within e4m3 (one too large would leave it below 224, one too small above
# 448).  Against the fp32 product of the dequantized
# operands, the dequantized output is within the e4m3 step plus the bf16
# GEMM bound (2^-8 of the largest |y| + 2e-3).
@pytest.mark.parametrize("M,K,N,gelu", [(4680, 3072, 14336, True), (300, 256, 512, False), (1, 3072, 256, True)])
def test_fp8_mx_output(dev, M, K, N, gelu):
    from wam_ops import ops
    print(f"fp8 MX output {M}x{K}x{N} gelu={gelu}", flush=True)
    x = _randn((M, K), dev, 31)
    w = _randn((N, K), dev, 32, 0.02)
    b = _randn((N,), dev, 33, 0.02)
    qw, sw = ops.quantize_fp8_rows(w)
    qx, sx = ops.quantize_fp8_rows(x)
    epi = ops.EPI_BIAS_GELU if gelu else ops.EPI_BIAS
    q, e = ops.linear(qx, qw, b, w_scale=sw, x_scale=sx, epilogue=epi, mx_out=True)
    yb = ops.linear(qx, qw, b, w_scale=sw, x_scale=sx, epilogue=epi)
    torch.cuda.synchronize()
    assert q.dtype == torch.float8_e4m3fn and q.shape == (M, N) and e.shape == (M, N // 32)
    q, e, yb = q.cpu(), e.cpu(), yb.float().cpu()
    d = ofp8.dequantize_mx32(q, e)
    half = torch.maximum(yb.abs() * 2 ** -4, torch.pow(2.0, e.double() - 127 - 10).float().repeat_interleave(32, 1))
    assert ((d - yb).abs() <= half + yb.abs() * 2 ** -8 + 1e-30).all()
    amax = yb.reshape(M, N // 32, 32).abs().amax(dim=2).double()
    er = ofp8.mx_exponent(amax.float()) + 127
    diff = e.int() != er
    assert ((e.int() - er).abs() <= 1).all()
    # a differing exponent only where the bf16 rounding of the block maximum
    # can cross the rule's boundary 448 * 2^X (or 448 * 2^(X-1))
    X = (er - 127).double()
    near = torch.minimum((amax - 448 * torch.pow(2.0, X)).abs(), (amax - 448 * torch.pow(2.0, X - 1)).abs())
    assert (near[diff] <= amax[diff] * 2 ** -8).all()
    assert diff.float().mean().item() <= 0.01
    bm = q.float().reshape(M, N // 32, 32).abs().amax(dim=2)
    assert ((bm >= 224) | (bm == 0)).all() and (bm <= 448).all()
    xd = ofp8.dequantize_rows(qx.cpu(), sx.cpu())
    wd = ofp8.dequantize_rows(qw.cpu(), sw.cpu())
    y = xd @ wd.t() + b.float().cpu()
    if gelu:
        y = torch.nn.functional.gelu(y, approximate="tanh")
    assert ((d - y).abs() <= y.abs() * 2 ** -4 + _ulp_bound(y)).all()


# MX activations into the fp8 MFMA (the FFN2 side): the operand is the
# oracle's MX quantization of bf16 values; against the fp32 product of the
# same dequantized operands the only differences are the accumulation order
# and the output rounding (the bf16 ulp bound), for the bias, gated-residual
# (fp32 residual stream, per-sample gate) and plain bf16 residual epilogues.
@pytest.mark.parametrize("M,K,N", [(4680, 14336, 3072), (300, 256, 512), (1, 128, 256), (455, 1024, 256)])
def test_fp8_mx_input(dev, M, K, N):
    from wam_ops import ops
    print(f"fp8 MX input {M}x{K}x{N}", flush=True)
    x = _randn((M, K), dev, 41).float().cpu()
    x[0, :32] = 0  # an all-zero block
    qx, ex = ofp8.quantize_mx32(x)
    w = _randn((N, K), dev, 42, 0.02)
    b = _randn((N,), dev, 43, 0.02)
    qw, sw = ops.quantize_fp8_rows(w)
    ref = ofp8.dequantize_mx32(qx, ex).to(dev) @ ofp8.dequantize_rows(qw.cpu(), sw.cpu()).to(dev).t() + b.float()
    qx, ex = qx.to(dev), ex.to(dev)
    y = ops.linear(qx, qw, b, w_scale=sw, x_block_scale=ex)
    assert_close(y, ref, _ulp_bound(ref), 0.99999, f"MX input bias {M}x{K}x{N}")
    res32 = _randn((M, N), dev, 44, 1.0, torch.float32)
    tokens = M // 2 if M % 2 == 0 else M
    table = _randn((1, 6, N), dev, 45, 0.1, torch.float32)
    temb = _randn((M // tokens, 1, 6, N), dev, 46, 0.1, torch.float32)
    gate = (table[0, 5][None] + temb[:, 0, 5]).repeat_interleave(tokens, 0)
    y = ops.linear(qx, qw, b, w_scale=sw, x_block_scale=ex, epilogue=ops.EPI_BIAS_GATE_RES, residual=res32,
                   table=table, temb=temb, tokens=tokens, gate_index=5)
    r = res32 + ref * gate
    assert_close(y, r, _ulp_bound(r), 0.99999, f"MX input gated residual {M}x{K}x{N}")
    res = _randn((M, N), dev, 47)
    y = ops.linear(qx, qw, b, w_scale=sw, x_block_scale=ex, epilogue=ops.EPI_BIAS_RES, residual=res)
    r = res.float() + ref
    assert_close(y, r, _ulp_bound(r), 0.99999, f"MX input residual {M}x{K}x{N}")


def test_fp8_mx_rejects(dev):
    from wam_ops import ops
    x = _randn((64, 256), dev, 1)
    w = _randn((256, 256), dev, 2, 0.02)
    qw, sw = ops.quantize_fp8_rows(w)
    qx, ex = ofp8.quantize_mx32(x.float().cpu())
    qx, ex = qx.to(dev), ex.to(dev)
    with pytest.raises(RuntimeError, match="MX activations"):
        ops.linear(qx, qw, None, w_scale=sw, x_block_scale=ex, epilogue=ops.EPI_BIAS_GELU)
    with pytest.raises(RuntimeError, match="mx_out"):
        ops.linear(x, w, None, mx_out=True)
