"""Per-stage parity of the HIP kernels (one C-ABI call each) on the GPU.

References: a plain fp32 torch computation of the same op on the same
device (GEMM, norms, attention), or the CPU oracle (RoPE, KV pool).
Tolerances are stated per test; bf16 outputs carry up to half an ulp of
rounding (2^-9 relative).
"""
import math

import pytest
import torch

from oracle import kvcache as okv
from oracle.block import apply_rope
from oracle.metrics import assert_close

pytestmark = pytest.mark.gpu


def _randn(shape, dev, seed, std=1.0, dtype=torch.bfloat16):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=dev) * std).to(dtype)


def _ulp_bound(ref, extra=2e-3):
    """Half an ulp of the largest bf16 output (2^-8 |y|max) plus fp32-order noise."""
    return 2.0 ** -8 * ref.abs().max().item() + extra


def _ref_linear(x, w, b):
    return x.float() @ w.float().t() + (b.float() if b is not None else 0.0)


@pytest.mark.parametrize("M,K,N,nseg", [(1, 64, 128, 1), (300, 256, 384, 1), (77, 512, 256, 3),
                                        (4680, 3072, 3072, 1), (520, 3072, 3072, 3),
                                        (300, 256, 192, 1), (70, 192, 200, 1), (4680, 3072, 192, 1),
                                        # 224-row tiles: 21 x 36 tiles over three segments
                                        (4680, 3072, 3072, 3)])
def test_linear_bias(dev, M, K, N, nseg):
    from wam_ops import ops
    x = _randn((M, K), dev, 1)
    ws = [_randn((N, K), dev, 10 + i, 0.02) for i in range(nseg)]
    bs = [_randn((N,), dev, 20 + i, 0.02) for i in range(nseg)]
    outs = ops.linear(x, ws if nseg > 1 else ws[0], bs if nseg > 1 else bs[0])
    outs = outs if nseg > 1 else [outs]
    for o, w, b in zip(outs, ws, bs):
        ref = _ref_linear(x, w, b)
        # bf16 output: rounding <= half an ulp = 2^-8 |y|; fp32 accumulation-order noise is far below
        bound = 2.0 ** -8 * ref.abs().max().item() + 1e-3
        assert_close(o, ref, max_abs=bound, min_cos=0.99999, what=f"linear {M}x{K}x{N}")


# (4680, 256, 3584) has 266 256x256 tiles, just above a multiple of the 256
# CUs, so its last columns run as a second 128x128-tile launch (column offsets
# into bias, residual, output and the modulation table); (4680, 256, 14336)
# (1064 such tiles) runs on 224-row tiles instead, which take 4.375 rounds
# against 4 rounds and a tail counted as 0.4.  (6240, 3072, 2816) and (6240, 6144, 3072) run their last
# columns split over k (8 and 5 ranges of fp32 partials, then a reduce pass
# with the epilogue); (3900, 4160, 4352) does so with a partial last row tile
# and 65 k-tiles in 8 uneven ranges.  (300, 512, 200) ends in a partial
# column tile (72 of 128 columns), so lanes past N skip the residual loads
# issued ahead of the LDS staging as well as the stores.  (4680, 3072, 3072),
# (4680, 14336, 3072) and (4500, 4160, 3072) run on 224-row tiles (21 row
# tiles; the last one of 4500 holds 20 rows, over 65 k-tiles), every
# epilogue included.  (6240, 6144, 3072), (6240, 3072, 3072) and (6000,
# 1024, 3072) run as one round of 320-row tiles (the last one of 6000 holds
# 240 rows).  (6240, 3072, 14336) is the verify layer's FFN1: 51 column
# tiles of 256-row tiles and the last 5 as a split-K tail in 2 ranges.
@pytest.mark.parametrize("M,K,N", [(130, 1024, 2048), (4680, 1024, 2048), (4680, 256, 3584),
                                   (4680, 256, 14336), (6240, 3072, 2816), (6240, 6144, 3072),
                                   (3900, 4160, 4352), (300, 512, 200), (4680, 3072, 3072),
                                   (4680, 14336, 3072), (4500, 4160, 3072), (6240, 3072, 3072),
                                   (6000, 1024, 3072), (6240, 3072, 14336)])
def test_linear_epilogues(dev, M, K, N):
    from wam_ops import ops
    D = N
    x = _randn((M, K), dev, 2)
    w = _randn((N, K), dev, 3, 0.05)
    b = _randn((N,), dev, 4, 0.05)
    ref = _ref_linear(x, w, b)
    y = ops.linear(x, w, b, epilogue=ops.EPI_BIAS_GELU)
    g = torch.nn.functional.gelu(ref, approximate="tanh")
    assert_close(y, g, _ulp_bound(g), 0.99999, "gelu")
    res = _randn((M, N), dev, 5)
    y = ops.linear(x, w, b, epilogue=ops.EPI_BIAS_RES, residual=res)
    assert_close(y, res.float() + ref, _ulp_bound(res.float() + ref), 0.99999, "residual")
    res32 = _randn((M, N), dev, 5, 1.0, torch.float32)
    y = ops.linear(x, w, b, epilogue=ops.EPI_BIAS_RES, residual=res32, out_dtype=torch.float32)
    assert y.dtype == torch.float32
    assert_close(y, res32 + ref, 1e-3, 0.999999, "fp32 residual, fp32 out")
    # gated residual with a per-sample modulation: rows split into 2 samples
    tokens = M // 2 if M % 2 == 0 else M
    B = M // tokens
    table = _randn((1, 6, D), dev, 6, 0.1, torch.float32)
    temb = _randn((B, 1, 6, D), dev, 7, 0.1, torch.float32)
    gate = (table[0, 2][None] + temb[:, 0, 2]).repeat_interleave(tokens, 0)
    y = ops.linear(x, w, b, epilogue=ops.EPI_BIAS_GATE_RES, residual=res, table=table, temb=temb,
                   tokens=tokens, gate_index=2)
    r = res.float() + ref * gate
    assert_close(y, r, _ulp_bound(r), 0.99999, "gated residual")
    # per-token bf16 temb
    tembt = _randn((B, tokens, 6, D), dev, 8, 0.1, torch.bfloat16)
    gate = (table[0, 5][None, None] + tembt[:, :, 5].float()).reshape(M, D)
    y = ops.linear(x, w, b, epilogue=ops.EPI_BIAS_GATE_RES, residual=res, table=table, temb=tembt,
                   tokens=tokens, gate_index=5)
    r = res.float() + ref * gate
    assert_close(y, r, _ulp_bound(r), 0.99999, "gated residual per-token")
    # fp32 residual stream, per-token gate, bf16 output (the FFN2 epilogue of
    # the block with a per-token temb)
    y = ops.linear(x, w, b, epilogue=ops.EPI_BIAS_GATE_RES, residual=res32, table=table, temb=tembt,
                   tokens=tokens, gate_index=5)
    r = res32 + ref * gate
    assert_close(y, r, _ulp_bound(r), 0.99999, "gated fp32 residual per-token")
    # per-frame temb (one modulation row per group of consecutive tokens): long
    # frames put one boundary in some row tiles (the two-row gate), short ones
    # several (the per-row gate)
    divs = [f for f in range(1, tokens + 1) if tokens % f == 0]
    for frames in sorted({max(f for f in divs if f <= 4), min(divs, key=lambda f: abs(tokens // f - 130))}):
        tembf = _randn((B, frames, 6, D), dev, 9 + frames, 0.1, torch.float32)
        fr = (torch.arange(tokens, device=dev) // (tokens // frames)).repeat(B)
        bi = torch.arange(M, device=dev) // tokens
        gate = table[0, 2][None] + tembf[bi, fr, 2]
        y = ops.linear(x, w, b, epilogue=ops.EPI_BIAS_GATE_RES, residual=res32, table=table, temb=tembf,
                       tokens=tokens, gate_index=2, out_dtype=torch.float32)
        r = res32 + ref * gate
        assert_close(y, r, 1e-3, 0.999999, f"gated fp32 residual, {frames} frames per sample")


def test_linear_rejects_bad_shapes(dev):
    from wam_ops import ops
    x = _randn((8, 100), dev, 1)
    w = _randn((128, 100), dev, 2)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        ops.linear(x, w)


@pytest.mark.parametrize("B,M,D,L", [(1, 37, 256, 1), (2, 300, 3072, 1), (2, 64, 3072, 64), (1, 5, 1536, 1)])
def test_ln_modulate(dev, B, M, D, L):
    from wam_ops import ops
    x = _randn((B, M, D), dev, 1, 2.0)
    x = x + _randn((1, 1, D), dev, 9, 1.0)  # non-zero mean
    table = _randn((1, 6, D), dev, 2, 1 / math.sqrt(D), torch.float32)
    temb = _randn((B, L, 6, D), dev, 3, 0.1, torch.float32)
    for shift in (0, 3):
        y = ops.ln_modulate(x, table, temb, shift, eps=1e-6)
        y32 = ops.ln_modulate(x.float(), table, temb, shift, eps=1e-6)
        assert torch.equal(y, y32)  # exact bf16 values read as fp32 give the same result
        mod = table[None] + temb
        ref = torch.nn.functional.layer_norm(x.float(), (D,), eps=1e-6) * (1 + mod[:, :, shift + 1]) + mod[:, :, shift]
        assert_close(y, ref, _ulp_bound(ref), 0.99999, f"ln_modulate shift {shift}")
    g = _randn((D,), dev, 4, 0.02, torch.float32) + 1
    bb = _randn((D,), dev, 5, 0.02, torch.float32)
    y = ops.layer_norm_affine(x, g, bb, eps=1e-6)
    ref = torch.nn.functional.layer_norm(x.float(), (D,), g, bb, eps=1e-6)
    assert_close(y, ref, _ulp_bound(ref), 0.99999, "norm2 affine")


@pytest.mark.parametrize("B,M,H", [(1, 60, 2), (2, 4680 // 4, 24)])
def test_rms_rope(dev, B, M, H):
    from wam_ops import ops, synthetic
    D = H * 128
    q = _randn((B, M, D), dev, 1, 3.0)
    k = _randn((B, M, D), dev, 2, 0.5)
    gq = _randn((D,), dev, 3, 0.02) + 1
    gk = _randn((D,), dev, 4, 0.02) + 1
    f = {60: (3, 4, 5), 1170: (3, 26, 15)}[M]
    freqs = synthetic.rope_freqs(synthetic.mesh_grid_ids(*f)).to(dev)
    yq, yk = ops.rms_rope([q, k], [gq, gk], [1e-6, 1e-6], freq=freqs)
    for y, x, g in ((yq, q, gq), (yk, k, gk)):
        n = torch.nn.functional.rms_norm(x.float(), (D,), g.float(), 1e-6)
        ref = apply_rope(n.unflatten(2, (H, 128)), freqs).flatten(2)
        assert_close(y, ref, _ulp_bound(ref), 0.99999, "rms+rope")
    # no RoPE (cross q/k), in place
    q2 = q.clone()
    ops.rms_rope([q2], [gq], [1e-6], out=[q2])
    ref = torch.nn.functional.rms_norm(q.float(), (D,), gq.float(), 1e-6)
    assert_close(q2, ref, _ulp_bound(ref), 0.99999, "rms in place")


def test_rms_rope_head_size_not_dividing_512(dev):
    """Heads of 96 (a lane's chunks, 512 columns apart, sit at different
    places in their heads): the rotation factors are read per chunk."""
    from wam_ops import ops
    B, M, hd, H = 2, 60, 96, 16
    D = H * hd
    x = _randn((B, M, D), dev, 1, 2.0)
    g = _randn((D,), dev, 3, 0.02) + 1
    gen = torch.Generator(device=dev).manual_seed(5)
    ang = torch.rand((B, M, 1, hd // 2), generator=gen, device=dev) * 6.283
    freq = torch.polar(torch.ones_like(ang), ang).contiguous()
    (y,) = ops.rms_rope([x], [g], [1e-6], freq=freq, head_dim=hd)
    n = torch.nn.functional.rms_norm(x.float(), (D,), g.float(), 1e-6).reshape(B, M, H, hd // 2, 2)
    rot = torch.view_as_real(torch.view_as_complex(n.contiguous()) * freq).reshape(B, M, D)
    assert_close(y, rot, _ulp_bound(rot), 0.99999, "rms+rope, 96-wide heads")


# The q/k-norm epilogue of the projection: checked against the plain bias
# GEMM's own bf16 output y (same kernels, same accumulation), so both the
# sums of squares and bf16(rope(y * gamma)) have exact references.  4680
# rows end in the four-wave kernel (224-row tiles; three segments = QKV, one
# = cross q); 520 and 120 rows in other tile kernels plus the norm pass; 6240
# rows = 4 samples of 1560 tokens sharing one RoPE table (row modulo tokens,
# one wrap per row); 4680 rows of 26 samples of 180 tokens (a modulo per row);
# 5120 rows, one segment: 256-row tiles in one round.  "per-sample": a
# [2, tokens, 1, 64] table whose two samples differ (row m reads table row m,
# no modulo), on the fused four-wave path (4680 rows) and on the norm pass
# (520 rows).  6240 rows, one segment: one round of 320-row tiles and the
# norm pass (with RoPE), or the 320-row kernel's own norm epilogue (without;
# 6000 rows end in a 240-row tile).
@pytest.mark.parametrize("M,nseg,grid", [(4680, 3, (6, 26, 30)), (4680, 1, None), (520, 3, (2, 10, 26)),
                                         (120, 1, (2, 6, 10)), (6240, 3, (2, 26, 30)),
                                         (4680, 3, (1, 12, 15)), (5120, 1, (5, 32, 32)),
                                         (4680, 1, "per-sample"), (520, 1, "per-sample"),
                                         (6240, 1, (2, 26, 30)), (6240, 1, None), (6000, 1, None)])
def test_linear_qk_norm(dev, M, nseg, grid):
    from wam_ops import ops, synthetic
    K = N = 3072
    H = N // 128
    x = _randn((M, K), dev, 1)
    ws = [_randn((N, K), dev, 10 + i, 0.02) for i in range(nseg)]
    bs = [_randn((N,), dev, 20 + i, 0.02) for i in range(nseg)]
    gs = [_randn((N,), dev, 30 + i, 0.1) + 1 for i in range(min(nseg, 2))] + [None] * (nseg - 2)
    if grid == "per-sample":
        # sample 0: raster ids of a (1, 2, M/4) grid; sample 1: the same grid
        # shifted by 7 frames, so every row of the two samples differs
        ids = synthetic.mesh_grid_ids(1, 2, M // 4)
        shifted = ids.clone()
        shifted[0] += 7
        freq = torch.cat([synthetic.rope_freqs(ids), synthetic.rope_freqs(shifted)]).to(dev)
        assert freq.shape == (2, M // 2, 1, 64) and not torch.equal(freq[0], freq[1])
    else:
        freq = synthetic.rope_freqs(synthetic.mesh_grid_ids(*grid)).to(dev) if grid else None
    plain = ops.linear(x, ws, bs)
    outs, ssqs = ops.linear(x, ws, bs, norm_gamma=gs, norm_freq=freq)
    for i in range(nseg):
        if gs[i] is None:
            assert ssqs[i] is None and torch.equal(outs[i], plain[i]), "segment without norm = plain GEMM"
            continue
        y = plain[i].float()
        ref_ss = (y.double() ** 2).reshape(M, N // 256, 256).sum(-1)
        rel = ((ssqs[i].double() - ref_ss).abs() / ref_ss).max().item()
        print(f"qk-norm {M}x{nseg} seg {i}: sum of squares rel err {rel:.2e}")
        assert rel < 1e-5, rel
        z = y * gs[i].float()
        if freq is not None:
            z = apply_rope(z.reshape(-1, freq.shape[1], H, 128), freq).reshape(M, N)
        ref = z.float()
        same = (outs[i] == ref.to(torch.bfloat16)).float().mean().item()
        assert same > 0.999, f"only {same:.5f} of the outputs equal bf16(rope(y * gamma))"
        assert_close(outs[i], ref, _ulp_bound(ref, 1e-3), 0.99999, f"qk-norm out {M}x{nseg} seg {i}")


@pytest.mark.parametrize("B,Mq,Mk,H", [(2, 100, 37, 2), (1, 4680, 4680, 24), (1, 4680, 512, 24),
                                       (1, 1560, 7800, 24)])
def test_attention_q_ssq(dev, B, Mq, Mk, H):
    """Queries scaled by their 1/rms inside attention (q_ssq) against
    attention over the RMS-normalised queries."""
    from wam_ops import ops
    D = H * 128
    y = _randn((B, Mq, D), dev, 1, 3.0)
    g = _randn((D,), dev, 4, 0.1) + 1
    k = _randn((B, Mk, H, 128), dev, 2)
    v = _randn((B, Mk, H, 128), dev, 3)
    yf = y.float()
    ssq = (yf ** 2).reshape(B * Mq, -1, min(D, 256)).sum(-1).contiguous()
    qg = (yf * g.float()).to(torch.bfloat16).reshape(B, Mq, H, 128)
    o = ops.attention(qg, k, v, q_ssq=ssq, q_eps=1e-6)
    qn = torch.nn.functional.rms_norm(yf, (D,), g.float(), 1e-6).reshape(B, Mq, H, 128)
    assert_close(o, _ref_attn(qn, k, v), 2e-2, 0.9999, f"attention q_ssq {B}x{Mq}x{Mk}x{H}")

def _ref_attn(q, k, v):
    return torch.nn.functional.scaled_dot_product_attention(
        q.float().transpose(1, 2), k.float().transpose(1, 2), v.float().transpose(1, 2)).transpose(1, 2)


@pytest.mark.parametrize("B,Mq,Mk,H", [(1, 1, 1, 1), (1, 100, 37, 2), (2, 129, 200, 3),
                                       (1, 4680, 512, 24), (1, 1560, 1560, 24),
                                       # grids of >= 128 workgroups of 256 queries (the
                                       # pipelined kernel): ragged queries and keys, one
                                       # key, key-range splits (4100 x 4099: 256-query units
                                       # in 3 ranges; 1560 x 7800: 224-query units in 3 ranges)
                                       (2, 1000, 77, 16), (1, 3000, 1, 24), (1, 4100, 4099, 24),
                                       (3, 700, 2500, 24), (1, 4680, 4680, 24), (1, 1560, 7800, 24),
                                       # the ping-pong schedule (16 key tiles or more) on short
                                       # key ranges: 256-query units in 8 ranges of 2 tiles;
                                       # 224-query units in 4 ranges of 4-5 tiles, with a
                                       # wave past the last query of each row
                                       (1, 2688, 1024, 25), (2, 1300, 1030, 26)])
def test_attention_plain(dev, B, Mq, Mk, H):
    from wam_ops import ops
    q = _randn((B, Mq, H, 128), dev, 1)
    k = _randn((B, Mk, H, 128), dev, 2)
    v = _randn((B, Mk, H, 128), dev, 3)
    o = ops.attention(q, k, v)
    assert_close(o, _ref_attn(q, k, v), 2e-2, 0.9999, f"attention {B}x{Mq}x{Mk}x{H}")


@pytest.mark.parametrize("B,Mq,Mk,H,nvalid", [(1, 100, 300, 2, 0), (1, 4680, 4680, 24, 0),
                                              (1, 1560, 7800, 24, 0), (2, 1000, 3000, 24, 1237),
                                              (1, 1560, 1560, 24, 6240)])
def test_attention_rising_scores(dev, B, Mq, Mk, H, nvalid):
    """Scores that rise along the keys, so the running max moves many times.

    Key j is scaled by 1 + 40 j / n (score spread from about 1 to 41 natural
    units).  A block of 64 keys three fifths of the way along is scaled by
    100 on top of that: its scores sit hundreds of log2 units above the max
    of the keys before it, past the range of an fp32 exponential taken
    against that max.  nvalid > 0 puts the first nvalid keys in a pool read
    through a slot list.
    """
    from wam_ops import ops
    n = nvalid + Mk
    ramp = 1 + 40 * torch.arange(n, device=dev, dtype=torch.float32) / n
    j0 = (3 * n) // 5
    ramp[j0:j0 + 64] *= 100
    q = _randn((B, Mq, H, 128), dev, 1)
    kall = (_randn((B, n, H, 128), dev, 2).float() * ramp[None, :, None, None]).bfloat16()
    vall = _randn((B, n, H, 128), dev, 3)
    if nvalid:
        slots = torch.arange(nvalid, dtype=torch.int32, device=dev)
        o = ops.attention(q, kall[:, nvalid:], vall[:, nvalid:], pool_k=kall[:, :nvalid].contiguous(),
                          pool_v=vall[:, :nvalid].contiguous(), slots=slots,
                          n_hist=torch.tensor([nvalid], dtype=torch.int32, device=dev))
    else:
        o = ops.attention(q, kall, vall)
    assert_close(o, _ref_attn(q, kall, vall), 2e-2, 0.9999, f"rising scores {B}x{Mq}x{Mk}+{nvalid}")


def test_attention_strided_and_broadcast(dev):
    from wam_ops import ops
    B, M, H = 2, 70, 2
    qkv = _randn((B, M, 3, H, 128), dev, 1)
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    o = ops.attention(q, k, v)
    assert_close(o, _ref_attn(q, k, v), 2e-2, 0.9999, "strided qkv")
    kc = _randn((1, 33, H, 128), dev, 4)
    vc = _randn((1, 33, H, 128), dev, 5)
    o = ops.attention(q, kc, vc)  # one context row for both samples
    assert_close(o, _ref_attn(q, kc.expand(B, -1, -1, -1), vc.expand(B, -1, -1, -1)), 2e-2, 0.9999, "broadcast")
    rows = torch.tensor([0, 0], dtype=torch.int64, device=dev)
    o = ops.attention(q, k, v, kv_rows=rows)
    assert_close(o, _ref_attn(q, k[:1].expand(B, -1, -1, -1), v[:1].expand(B, -1, -1, -1)), 2e-2, 0.9999, "kv_rows")


@pytest.mark.parametrize("B,Mq,P,nvalid,Bp,candidate", [(1, 50, 300, 170, 1, False),
                                                        (2, 64, 500, 321, 2, False),
                                                        (4, 33, 400, 250, 2, True),
                                                        (4, 1560, 7800, 6240, 1, True),
                                                        (2, 1560, 7800, 5000, 2, False),
                                                        # pipelined kernel: a key block that mixes
                                                        # pool and own keys (n_hist % 4 != 0), a
                                                        # history shorter than one key tile
                                                        (2, 1000, 3000, 1237, 2, False),
                                                        (1, 3000, 100, 3, 1, True)])
def test_attention_history(dev, B, Mq, P, nvalid, Bp, candidate):
    from wam_ops import ops
    H = 2 if Mq < 1000 else 24
    q = _randn((B, Mq, H, 128), dev, 1)
    k = _randn((B, Mq, H, 128), dev, 2)
    v = _randn((B, Mq, H, 128), dev, 3)
    pk = _randn((Bp, P, H, 128), dev, 4)
    pv = _randn((Bp, P, H, 128), dev, 5)
    g = torch.Generator().manual_seed(6)
    slots = torch.randperm(P, generator=g)[:nvalid].sort().values
    slots_d = slots.to(torch.int32).to(dev)
    n = torch.tensor([nvalid], dtype=torch.int32, device=dev)
    rows = torch.tensor([i % Bp for i in range(B)], dtype=torch.int64, device=dev) if candidate else None
    o = ops.attention(q, k, v, pool_k=pk, pool_v=pv, slots=slots_d, n_hist=n, pool_rows=rows)
    r = rows if candidate else torch.arange(B, device=dev)
    hk = pk[:, slots.to(dev)].index_select(0, r)
    hv = pv[:, slots.to(dev)].index_select(0, r)
    ref = _ref_attn(q, torch.cat([hk, k], 1), torch.cat([hv, v], 1))
    assert_close(o, ref, 2e-2, 0.9999, "history attention")


# History in consecutive slots (kv_layout's info[2] >= 0): the pipelined
# kernel reads the pool rows at that base, without the slot list.  Same keys
# in the same order as through the slot list, so the outputs are bitwise
# equal; n_hist % 4 != 0 puts the last pool keys in a block that straddles
# the own keys; a base of 0 and a base inside the pool; the C4a shape.
@pytest.mark.parametrize("B,Mq,P,base,nvalid,Bp", [(4, 1560, 7800, 0, 6240, 1), (2, 1000, 3000, 700, 1237, 2),
                                                   (1, 1560, 7800, 0, 6240, 1), (2, 1300, 2000, 3, 1, 2)])
def test_attention_consecutive_history(dev, B, Mq, P, base, nvalid, Bp):
    from wam_ops import ops
    H = 24
    q = _randn((B, Mq, H, 128), dev, 11)
    k = _randn((B, Mq, H, 128), dev, 12)
    v = _randn((B, Mq, H, 128), dev, 13)
    pk = _randn((Bp, P, H, 128), dev, 14)
    pv = _randn((Bp, P, H, 128), dev, 15)
    slots = torch.arange(base, base + nvalid, dtype=torch.int32, device=dev)
    n = torch.tensor([nvalid], dtype=torch.int32, device=dev)
    rows = torch.tensor([(i + 1) % Bp for i in range(B)], dtype=torch.int64, device=dev)
    via_slots = ops.attention(q, k, v, pool_k=pk, pool_v=pv, slots=slots, n_hist=n, pool_rows=rows)
    hb = torch.tensor([base], dtype=torch.int32, device=dev)
    at_base = ops.attention(q, k, v, pool_k=pk, pool_v=pv, slots=slots, n_hist=n, pool_rows=rows, hist_base=hb)
    assert torch.equal(at_base, via_slots), "consecutive-history path differs from the slot-list path"
    none = torch.tensor([-1], dtype=torch.int32, device=dev)
    assert torch.equal(ops.attention(q, k, v, pool_k=pk, pool_v=pv, slots=slots, n_hist=n, pool_rows=rows,
                                     hist_base=none), via_slots)
    hk = pk[:, base:base + nvalid].index_select(0, rows)
    hv = pv[:, base:base + nvalid].index_select(0, rows)
    ref = _ref_attn(q, torch.cat([hk, k], 1), torch.cat([hv, v], 1))
    assert_close(at_base, ref, 2e-2, 0.9999, "consecutive history attention")


def test_kv_layout_reports_consecutive_history(dev):
    """info[2]: the first history slot when the valid slots form one run,
    else -1."""
    from wam_ops import ops
    P, H = 64, 1
    for valid, expect in (((3, 4, 5, 6), 3), ((0, 1, 2), 0), ((2, 3, 5), -1), ((), -1)):
        cache = {"k": torch.zeros(1, P, H, 128, dtype=torch.bfloat16, device=dev),
                 "v": torch.zeros(1, P, H, 128, dtype=torch.bfloat16, device=dev),
                 "id": torch.full((P,), -1, dtype=torch.int64, device=dev),
                 "mask": torch.zeros(P, dtype=torch.bool, device=dev),
                 "is_pred": torch.zeros(P, dtype=torch.bool, device=dev)}
        for i in valid:
            cache["mask"][i] = True
            cache["id"][i] = 0
        rows = torch.zeros(1, dtype=torch.int64, device=dev)
        res = ops.kv_layout(cache, 4, 0, candidate_rows=rows)
        info = res[-1].cpu()
        assert info[0].item() == len(valid) and info[2].item() == expect, (valid, info.tolist())


def _cache_pair(P, H, seed, dev, prefix_chunks):
    """Identical CPU (oracle) and GPU pools after committing some chunks."""
    c = okv.new_cache(P, H, 128, 1, torch.bfloat16)
    g = torch.Generator().manual_seed(seed)
    for n, upd in prefix_chunks:
        kk = torch.randn(1, n, H, 128, generator=g).bfloat16()
        okv.update_cache(c, kk, kk, is_pred=(upd == 1))
    return c, {k: v.to(dev) for k, v in c.items()}


@pytest.mark.parametrize("P,chunks,tokens,update", [
    (100, [(30, 2), (30, 1)], 20, 0),
    (100, [(30, 2), (30, 1)], 20, 1),
    (100, [(40, 2), (40, 2)], 40, 2),      # evicts 20 of the oldest chunk
    (64, [(32, 2), (32, 1)], 48, 1),       # evicts a whole chunk and part of the next
    (3000, [(1000, 2), (1000, 1), (900, 2)], 1000, 0),
    (12000, [(5000, 2), (4000, 1), (2500, 2)], 1500, 1),   # 12 slots per thread (read per pass), evicts
    (20000, [(9000, 2), (9000, 1)], 3000, 2),               # 20 slots per thread (read per pass), evicts
])
def test_kv_layout_matches_oracle(dev, P, chunks, tokens, update):
    from wam_ops import ops
    H = 1
    cpu, gpu = _cache_pair(P, H, 11, dev, chunks)
    # oracle: slots chosen by update_cache, history = valid minus the new slots
    ref = okv.clone_cache(cpu)
    kk = torch.zeros(1, tokens, H, 128, dtype=torch.bfloat16)
    new = okv.update_cache(ref, kk, kk, is_pred=(update == 1))
    valid_after = okv.valid_slots(ref)
    hist_ref = [s for s in valid_after.tolist() if s not in set(new.tolist())]
    if update == 0:
        okv.restore_cache(ref, new)
    hist, newslots, info = ops.kv_layout(gpu, tokens, update)
    torch.cuda.synchronize()
    n = int(info[0])
    assert int(info[1]) == 0
    assert hist[:n].cpu().tolist() == hist_ref
    assert newslots[:tokens].cpu().tolist() == new.tolist()
    for key in ("mask", "id", "is_pred"):
        assert torch.equal(gpu[key].cpu(), ref[key]), key


def test_kv_layout_candidate_read_only(dev):
    from wam_ops import ops
    cpu, gpu = _cache_pair(50, 1, 3, dev, [(20, 2), (10, 1)])
    before = {k: v.clone() for k, v in gpu.items()}
    rows = torch.tensor([0, 0, 0], dtype=torch.int64, device=dev)
    hist, _, info = ops.kv_layout(gpu, 5, 0, candidate_rows=rows)
    torch.cuda.synchronize()
    assert int(info[1]) == 0 and int(info[0]) == 30
    assert hist[:30].cpu().tolist() == okv.valid_slots(cpu).tolist()
    for k in before:
        assert torch.equal(before[k], gpu[k])
    bad = torch.tensor([0, 1, 0], dtype=torch.int64, device=dev)
    _, _, info = ops.kv_layout(gpu, 5, 0, candidate_rows=bad)
    torch.cuda.synchronize()
    assert int(info[1]) == 2


def test_kv_commit(dev):
    from wam_ops import ops
    P, H, M = 40, 2, 7
    cache = {"k": torch.zeros(2, P, H, 128, dtype=torch.bfloat16, device=dev),
             "v": torch.zeros(2, P, H, 128, dtype=torch.bfloat16, device=dev)}
    k = _randn((2, M, H * 128), dev, 1)
    v = _randn((2, M, H * 128), dev, 2)
    slots = torch.tensor([3, 9, 10, 11, 20, 30, 39], dtype=torch.int32, device=dev)
    ops.kv_commit(cache, k, v, slots)
    s = slots.long()
    assert torch.equal(cache["k"][:, s].flatten(2), k)
    assert torch.equal(cache["v"][:, s].flatten(2), v)
