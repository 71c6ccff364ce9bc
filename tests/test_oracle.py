"""Pin the oracle's building blocks on the CPU against brute force and closed
forms, so that a dropped term, a wrong index or a transposed operand in the
oracle fails here (not only in the GPU comparison)."""
import math

import pytest
import torch

from oracle import kvcache as okv
from oracle import rope as orope
from oracle.block import apply_rope, block_forward, sdpa
from oracle.metrics import compare


def _g(seed):
    return torch.Generator().manual_seed(seed)


def test_layer_norm_brute_force():
    x = torch.randn(3, 5, 40, generator=_g(0), dtype=torch.float64) * 3 + 1
    D = x.shape[-1]
    ref = torch.empty_like(x)
    for i in range(3):
        for j in range(5):
            row = x[i, j]
            mu = sum(row.tolist()) / D
            var = sum((v - mu) ** 2 for v in row.tolist()) / D
            ref[i, j] = (row - mu) / math.sqrt(var + 1e-6)
    got = torch.nn.functional.layer_norm(x.float(), (D,), eps=1e-6)
    assert (got.double() - ref).abs().max() < 1e-5
    # closed form: zero mean, unit variance
    assert got.mean(-1).abs().max() < 1e-5 and (got.var(-1, unbiased=False) - 1).abs().max() < 1e-4


def test_rms_norm_is_across_all_heads():
    H, hd = 3, 8
    x = torch.randn(2, 4, H * hd, generator=_g(1), dtype=torch.float64)
    x[..., :hd] *= 10  # heads of very different scale
    g = 1 + 0.1 * torch.randn(H * hd, generator=_g(2), dtype=torch.float64)
    ref = torch.empty_like(x)
    for i in range(2):
        for j in range(4):
            ms = sum(v * v for v in x[i, j].tolist()) / (H * hd)
            ref[i, j] = x[i, j] / math.sqrt(ms + 1e-6) * g
    got = torch.nn.functional.rms_norm(x.float(), (H * hd,), g.float(), 1e-6)
    assert (got.double() - ref).abs().max() < 1e-5
    per_head = torch.nn.functional.rms_norm(x.float().unflatten(-1, (H, hd)), (hd,), None, 1e-6).flatten(-2)
    assert (per_head.double() * g - ref).abs().max() > 0.1  # a per-head norm would differ


def test_gelu_tanh_closed_form():
    x = torch.linspace(-8, 8, 1001, dtype=torch.float64)
    ref = 0.5 * x * (1 + torch.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))
    got = torch.nn.functional.gelu(x.float(), approximate="tanh").double()
    assert (got - ref).abs().max() < 1e-6
    assert abs(got[500]) < 1e-12 and abs(got[-1] - 8) < 1e-6 and abs(got[0]) < 1e-6


def test_sdpa_brute_force():
    B, L, S, H, d = 2, 5, 7, 2, 8
    q = torch.randn(B, L, H, d, generator=_g(3))
    k = torch.randn(B, S, H, d, generator=_g(4))
    v = torch.randn(B, S, H, d, generator=_g(5))
    got = sdpa(q, k, v)
    ref = torch.zeros(B, L, H, d, dtype=torch.float64)
    for b in range(B):
        for h in range(H):
            for i in range(L):
                s = [sum(q[b, i, h, t].item() * k[b, j, h, t].item() for t in range(d)) / math.sqrt(d)
                     for j in range(S)]
                m = max(s)
                e = [math.exp(x - m) for x in s]
                z = sum(e)
                for j in range(S):
                    ref[b, i, h] += e[j] / z * v[b, j, h].double()
    assert (got.double() - ref).abs().max() < 1e-5
    # a dominant logit selects its value row
    k2 = k.clone()
    k2[:, 3] = q[:, 0:1].expand(-1, 1, -1, -1)[:, 0] * 100
    out = sdpa(q[:, :1], k2, v)
    assert (out[:, 0] - v[:, 3]).abs().max() < 1e-4


def test_rope_properties():
    fb, hb, wb = orope.base_freqs(128)
    assert fb.numel() == 22 and hb.numel() == 21 and wb.numel() == 21
    assert abs(fb[1].item() - 1 / 10000 ** (2 / 44)) < 1e-15
    assert abs(hb[20].item() - 1 / 10000 ** (40 / 42)) < 1e-15
    grid = orope.get_mesh_id(2, 3, 4)
    assert grid.shape == (4, 24)
    assert grid[:3, 13].tolist() == [1.0, 0.0, 1.0]  # raster order (f, h, w)
    freqs = orope.rope_freqs(grid[None])
    assert freqs.shape == (1, 24, 1, 64) and freqs.dtype == torch.complex64
    x = torch.randn(1, 24, 2, 128, generator=_g(6))
    y = apply_rope(x, freqs)
    # identity at the origin, pairwise norm preserved everywhere
    assert torch.allclose(y[:, 0], x[:, 0], atol=1e-6)
    n_in = x.reshape(1, 24, 2, 64, 2).pow(2).sum(-1)
    n_out = y.reshape(1, 24, 2, 64, 2).pow(2).sum(-1)
    assert torch.allclose(n_in, n_out, rtol=1e-5, atol=1e-5)
    # explicit cos/sin rotation of pair j at token t
    t, j = 17, 30
    ang = torch.angle(freqs[0, t, 0, j]).item()
    a, b = x[0, t, 1, 2 * j].item(), x[0, t, 1, 2 * j + 1].item()
    assert abs(y[0, t, 1, 2 * j].item() - (a * math.cos(ang) - b * math.sin(ang))) < 1e-5
    assert abs(y[0, t, 1, 2 * j + 1].item() - (a * math.sin(ang) + b * math.cos(ang))) < 1e-5
    # relative-position invariance along the frame axis
    q = torch.randn(1, 1, 1, 128, generator=_g(7))
    k = torch.randn(1, 1, 1, 128, generator=_g(8))

    def at(frame):
        g = torch.tensor([[[float(frame)], [0.0], [0.0]]])
        return orope.rope_freqs(g)
    d1 = (apply_rope(q, at(5)) * apply_rope(k, at(2))).sum()
    d2 = (apply_rope(q, at(9)) * apply_rope(k, at(6))).sum()
    assert abs(d1 - d2) < 1e-4


def test_product_rope_generator_matches_oracle():
    from wam_ops import synthetic
    grid = (3, 4, 5)
    prod = synthetic.rope_freqs(synthetic.mesh_grid_ids(*grid))
    ref = orope.rope_freqs(orope.get_mesh_id(*grid)[None])
    assert torch.equal(prod, ref)


def test_kvcache_protocol_by_hand():
    c = okv.new_cache(6, 1, 2)
    kv = lambda n, val: torch.full((1, n, 1, 2), float(val))
    s = okv.update_cache(c, kv(2, 1), kv(2, 1), is_pred=False)       # id 0 -> slots 0,1
    assert s.tolist() == [0, 1] and c["id"].tolist() == [0, 0, -1, -1, -1, -1]
    s = okv.update_cache(c, kv(3, 2), kv(3, 2), is_pred=True)        # id 1 -> slots 2,3,4
    assert s.tolist() == [2, 3, 4] and c["is_pred"].tolist() == [False, False, True, True, True, False]
    s = okv.update_cache(c, kv(3, 3), kv(3, 3), is_pred=False)       # 1 free, evict 2 oldest (id 0)
    assert s.tolist() == [0, 1, 5] and c["id"].tolist() == [2, 2, 1, 1, 1, 2]
    okv.restore_cache(c, s)
    assert c["mask"].tolist() == [False, False, True, True, True, False]
    okv.clear_pred_cache(c)
    assert not c["mask"].any()
    assert okv.next_cache_id(c) == 0


def test_metrics_special_values():
    a = torch.tensor([0.0, 1.0])
    b = torch.tensor([-0.0, 1.0])
    m = compare(a, b)
    assert m["max_abs"] == 0 and m["finite"]
    m = compare(torch.tensor([float("nan"), 1.0]), b)
    assert not m["finite"]


def test_bf16_reference_vs_fp32_calibration():
    """The reference's own bf16 precision (emulated) against fp32 at a tiny shape:
    how much of the 2e-2 budget bf16 rounding alone uses (recorded, cos bound)."""
    from wam_ops import synthetic
    shape = synthetic.BlockShape(256, 2, 512)
    params = synthetic.block_params(shape, seed=5)
    x, ctx, temb, freqs = synthetic.block_inputs(shape, 1, 60, (3, 4, 5), context_len=16, seed=6)
    ref32 = block_forward(params, x, ctx, temb, freqs, shape.heads, shape.eps)
    ref16 = block_forward(params, x, ctx, temb, freqs, shape.heads, shape.eps, dtype=torch.bfloat16)
    m = compare(ref16, ref32)
    assert m["cosine"] > 0.99999 and m["max_abs"] < 0.05


def test_fp8_quantization_pinned():
    """The oracle's e4m3 quantization against values decoded by hand from the
    OCP E4M3 bit layout, exact round-to-nearest-even cases and the per-row
    scale's closed form."""
    from oracle import fp8
    # every finite e4m3 byte decodes to a value that the cast maps back to itself
    for b in range(256):
        v = fp8.e4m3_decode(b)
        if v != v:  # NaN codes 0x7f, 0xff
            continue
        t = torch.tensor([v], dtype=torch.float32).to(fp8.E4M3)
        assert t.view(torch.uint8).item() in (b, 0x00 if b == 0x80 else b), (b, v)
        assert t.float().item() == v
    assert fp8.e4m3_decode(0x7E) == 448.0 and fp8.e4m3_decode(0x38) == 1.0
    assert fp8.e4m3_decode(0x01) == 2.0 ** -9  # smallest subnormal
    # round to nearest even between neighbours 1.0 (0x38) and 1.125 (0x39)
    cases = {1.0625: 0x38, 1.0625 + 1e-3: 0x39, 1.1875: 0x3A, 1.1875 - 1e-3: 0x39, 447.0: 0x7E}
    for v, b in cases.items():
        assert torch.tensor([v]).to(fp8.E4M3).view(torch.uint8).item() == b, v
    # per-row scale: the row max maps to 448 exactly, zero rows get scale 1
    w = torch.tensor([[0.5, -2.0, 1.0, 0.0], [0.0, 0.0, 0.0, 0.0], [3e-3, -1e-3, 2e-3, 7e-4]])
    q, s = fp8.quantize_rows(w)
    assert torch.allclose(s, torch.tensor([2.0 / 448, 1.0, 3e-3 / 448]))
    assert q.float()[0, 1].item() == -448.0 and q.float()[2, 0].item() == 448.0
    assert q.float()[1].abs().sum().item() == 0.0
    deq = fp8.dequantize_rows(q, s)
    # relative error of a normal e4m3 value is at most 2^-4 (3 mantissa bits, RNE)
    nz = w.abs() > 0
    assert ((deq - w).abs()[nz] <= w.abs()[nz] * 2 ** -4 + 1e-12).all()
    # the factor 448 / max is one correctly rounded fp32 division, and the
    # product is rounded to fp32 before the e4m3 rounding: -0.017578125 *
    # fp32(448 / 3) is exactly -2.625 in fp32, a tie that goes to the even
    # code -2.5 (with fp32(448 * fp32(1 / 3)) it would land on -2.75)
    q, s = fp8.quantize_rows(torch.tensor([[-0.017578125, 3.0]]))
    assert q.float()[0, 0].item() == -2.5 and q.float()[0, 1].item() == 448.0
    amax = torch.rand(2000, generator=torch.Generator().manual_seed(3)) * 100 + 1e-3
    w = torch.stack([amax, -amax / 3], dim=1)
    q, s = fp8.quantize_rows(w)
    f = (448.0 / amax.double()).float()
    assert torch.equal(q.view(torch.uint8), (w * f[:, None]).to(fp8.E4M3).view(torch.uint8))
    assert torch.equal(s, (amax.double() / 448.0).float())


def test_ffn_gated_pinned():
    """oracle.fp8.ffn_gated (the FFN unit with its gated residual) against a
    float64 loop over the definition, with the tanh GELU written out, on
    shapes where no two dimensions agree (a transposed operand cannot even
    broadcast), and against the block oracle's own FFN stage (pinned by the
    reference's golden vectors) for one block of the tiny shape."""
    from oracle import fp8
    g = _g(11)
    M, K, F_, N = 3, 5, 7, 4
    x = torch.randn(M, K, generator=g)
    w1, b1 = torch.randn(F_, K, generator=g), torch.randn(F_, generator=g)
    w2, b2 = torch.randn(N, F_, generator=g), torch.randn(N, generator=g)
    res, gate = torch.randn(M, N, generator=g), torch.randn(N, generator=g)
    got = fp8.ffn_gated(x, w1, b1, w2, b2, res, gate).double()
    c = math.sqrt(2 / math.pi)
    for m in range(M):
        h = []
        for j in range(F_):
            u = sum(float(x[m, k]) * float(w1[j, k]) for k in range(K)) + float(b1[j])
            h.append(0.5 * u * (1 + math.tanh(c * (u + 0.044715 * u ** 3))))
        for n in range(N):
            y = sum(h[j] * float(w2[n, j]) for j in range(F_)) + float(b2[n])
            want = float(res[m, n]) + float(gate[n]) * y
            assert abs(float(got[m, n]) - want) <= 1e-5 * (1 + abs(want)), (m, n)
    # the FFN stage of the block oracle (fp32): output = residual2 + ffn2 * c_gate
    from wam_ops import synthetic
    shape = synthetic.BlockShape(256, 2, 512)
    params = synthetic.block_params(shape, seed=7)
    xb, ctx, temb, freqs = synthetic.block_inputs(shape, 1, 24, (2, 3, 4), context_len=8, seed=8)
    keep = {}
    out = block_forward(params, xb, ctx, temb, freqs, shape.heads, shape.eps, intermediates=keep)
    c_gate = keep["modulation"][:, :, 5]
    unit = fp8.ffn_gated(keep["modulated3"][0], params["ffn.net.0.proj.weight"], params["ffn.net.0.proj.bias"],
                         params["ffn.net.2.weight"], params["ffn.net.2.bias"], keep["residual2"][0],
                         c_gate[0, 0])
    assert (unit - out[0].float()).abs().max() < 1e-4
    assert (unit - out[0].float()).abs().max() < (out[0].float() - keep["residual2"][0]).abs().max() * 1e-3


def test_mx32_quantization_pinned():
    """The oracle's MX (32-value block, e8m0 exponent) quantization: the
    exponent's closed form at the boundaries (448 * 2^X is the largest block
    max that keeps X), brute force over a range of exponents that it is the
    smallest one with no value above 448, and the round trip."""
    from oracle import fp8
    cases = {448.0: 0, 448.0 * 1.0001: 1, 256.0: 0, 255.99: 0, 224.0: -1, 223.9: -1, 112.01: -1, 1.0: -8, 1.75: -8,
             1.7501: -7, 3.5: -7, 0.0: -127, 2.0 ** -140: -127, 448.0 * 2 ** 20: 20}
    for v, x in cases.items():
        assert fp8.mx_exponent(torch.tensor([v], dtype=torch.float32)).item() == x, v
    g = torch.Generator().manual_seed(5)
    amax = torch.rand(4000, generator=g) * torch.pow(2.0, torch.randint(-30, 30, (4000,), generator=g).float())
    X = fp8.mx_exponent(amax).double()
    assert (amax.double() <= 448 * torch.pow(2.0, X)).all()
    assert (amax.double() > 448 * torch.pow(2.0, X - 1)).all()
    y = torch.randn(6, 128, generator=g) * torch.pow(2.0, torch.randint(-8, 8, (6, 1), generator=g).float())
    y[1, 32:64] = 0
    q, e = fp8.quantize_mx32(y)
    assert e.shape == (6, 4) and e[1, 1].item() == 0 and not q.float()[1, 32:64].any()
    blockmax = q.float().reshape(6, 4, 32).abs().amax(dim=2)
    nz = blockmax > 0
    assert (blockmax[nz] >= 224).all() and (blockmax <= 448).all()
    d = fp8.dequantize_mx32(q, e)
    # e4m3 keeps 3 mantissa bits: 2^-4 relative, or half the subnormal step 2^-10 at the block's scale
    step = torch.pow(2.0, (e.double() - 127 - 10)).float().repeat_interleave(32, dim=1)
    assert ((d - y).abs() <= torch.maximum(y.abs() * 2 ** -4, step) + 1e-30).all()
