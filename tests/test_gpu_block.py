"""Whole-block parity: the HIP block (one wam_block_forward call) against the
CPU fp32 oracle on identical seeded inputs.

Bound (the stated target): max |out - ref| <= 2e-2 and cosine >= 0.9999 for
the bf16 block against the fp32 reference.
"""
import pytest
import torch

from oracle import kvcache as okv
from oracle.block import block_forward
from oracle.metrics import assert_close, compare

pytestmark = pytest.mark.gpu

TINY = dict(dim=256, heads=2, ffn=512)


def _shape(dim, heads, ffn):
    from wam_ops.synthetic import BlockShape
    return BlockShape(dim, heads, ffn)


def native_block(params, shape, dev):
    from wam_ops.block import TransformerBlock
    blk = TransformerBlock(shape.dim, shape.ffn, shape.heads, cross_attn_norm=True, eps=shape.eps)
    sd = blk.state_dict()
    for name, t in params.items():
        assert name in sd, name
    with torch.no_grad():
        for name, mod_param in blk.named_parameters():
            mod_param.data = params[name].to(dev)
    return blk.to(dev)


def _inputs(shape, B, grid, Lc, seed, per_token=False):
    from wam_ops import synthetic
    M = grid[0] * grid[1] * grid[2]
    return synthetic.block_inputs(shape, B, M, grid, context_len=Lc, context_batch=B, seed=seed,
                                  per_token_temb=per_token)


@pytest.mark.parametrize("cfg,B,grid,Lc,per_token", [
    (TINY, 1, (3, 4, 5), 16, False),
    (TINY, 2, (2, 5, 7), 24, True),
    (dict(dim=3072, heads=24, ffn=14336), 1, (4, 8, 8), 512, False),
    # the Wan-1.3B-shaped block of the CPU reference case: 1024 tokens on a
    # (4, 16, 16) grid, dim 1536, 12 heads, FFN 8960, 512 context tokens
    (dict(dim=1536, heads=12, ffn=8960), 1, (4, 16, 16), 512, False),
])
def test_block_vs_fp32_oracle(dev, cfg, B, grid, Lc, per_token):
    from wam_ops import synthetic
    shape = _shape(**cfg)
    params = synthetic.block_params(shape, seed=5)
    x, ctx, temb, freqs = _inputs(shape, B, grid, Lc, 6, per_token)
    ref = block_forward(params, x, ctx, temb, freqs, shape.heads, shape.eps)
    blk = native_block(params, shape, dev)
    with torch.no_grad():
        out = blk(x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev))
    torch.cuda.synchronize()
    m = assert_close(out.cpu(), ref, max_abs=2e-2, min_cos=0.9999, what=f"block {cfg} B{B} {grid}")
    print("block parity", cfg, grid, m)


def test_block_l4680_headline(dev):
    """The measured workload itself: one Wan2.2-5B block, B=1, 4680 tokens
    (RoPE grid 6x26x30), 512 text tokens with precomputed cross K/V, against
    the fp32 oracle at the block bound."""
    from wam_ops import synthetic
    from wam_ops.whole_layer import WholeLayerBlock
    shape = synthetic.WAN22_5B
    params = synthetic.block_params(shape, seed=1)
    x, ctx, temb, freqs = synthetic.block_inputs(shape, 1, 4680, (6, 26, 30), context_len=512, seed=1)
    wl = WholeLayerBlock(native_block(params, shape, dev))
    with torch.no_grad():
        wl.prepare_context(ctx.to(dev), precompute=True)
        out = wl(x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev))
    torch.cuda.synchronize()
    ref = block_forward(params, x, ctx, temb, freqs, shape.heads, shape.eps)
    m = assert_close(out.cpu(), ref, max_abs=2e-2, min_cos=0.9999, what="L4680 block")
    print("L4680 parity", m)


def test_verify_layer_full_size(dev):
    """The verify layer at its real size: 4 candidates x 1560 tokens, each over
    the shared 6240-token committed prefix (pool row 0 of a 7800-slot pool)
    plus its own tokens, read-only cache, against the fp32 oracle."""
    from wam_ops import synthetic
    shape = synthetic.WAN22_5B
    params = synthetic.block_params(shape, seed=2)
    B, M, prefix = 4, 1560, 6240
    x, ctx, temb, freqs = synthetic.block_inputs(shape, B, M, (2, 26, 30), context_len=512, seed=3)
    blk = native_block(params, shape, dev)
    cache = synthetic.kv_pool(shape, prefix + M, prefix, batch=1, seed=4, device=dev)
    blk.attn1.attn_caches["pos"] = cache
    ocache = {k: (v.float().cpu() if v.dtype == torch.bfloat16 else v.cpu()) for k, v in cache.items()}
    rows = torch.zeros(B, dtype=torch.int64)
    with torch.no_grad():
        out = blk(x.to(dev), ctx[:1].to(dev), temb.to(dev), freqs.to(dev), update_cache=0,
                  candidate_cache_rows=rows.to(dev))
    torch.cuda.synchronize()
    ref = block_forward(params, x, ctx[:1], temb, freqs, shape.heads, shape.eps, cache=ocache, update_cache=0,
                        candidate_rows=rows)
    m = assert_close(out.cpu(), ref, max_abs=2e-2, min_cos=0.9999, what="verify layer 4x1560 over 6240")
    assert torch.equal(blk.attn1.attn_caches["pos"]["mask"].cpu(), ocache["mask"])
    print("verify parity", m)


def test_block_debug_intermediates(dev):
    from wam_ops import synthetic
    shape = _shape(**TINY)
    params = synthetic.block_params(shape, seed=7)
    x, ctx, temb, freqs = _inputs(shape, 1, (3, 4, 5), 16, 8)
    inter = {}
    block_forward(params, x, ctx, temb, freqs, shape.heads, shape.eps, intermediates=inter)
    from wam_ops.native import NativeBlock
    blk = native_block(params, shape, dev)
    with torch.no_grad():
        dbg = NativeBlock(blk)(x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev), debug=True)
    from wam_ops import _lib
    # all 28 named intermediates of the reference (whole_layer.cu:1203-1209)
    assert set(dbg) == set(_lib.DEBUG_NAMES) and len(_lib.DEBUG_NAMES) == 28
    for name in _lib.DEBUG_NAMES:
        ref = inter[name].float()
        got = dbg[name].reshape(ref.shape).float().cpu()
        # bf16 outputs: half an ulp of the largest value plus accumulation noise;
        # the modulation table is an fp32 sum
        bound = 1e-5 if name == "modulation" else max(2e-2, 2.0 ** -8 * ref.abs().max().item() + 2e-3)
        assert_close(got, ref, max_abs=bound, min_cos=0.9999, what=f"debug {name}")


def test_block_debug_l4680_runs_the_same_kernels(dev):
    """At L4680 the cross-attention queries are normalised in the projection's
    epilogue and attention applies their 1/rms.  A debug call runs those same
    kernels (the debug copies come from extra launches), so its output equals
    a normal call's bit for bit; its cross-q intermediates (the projection
    before the norm, the normalised queries) and the cross-attention output
    match the oracle's."""
    from wam_ops import synthetic
    from wam_ops.native import NativeBlock
    shape = synthetic.WAN22_5B
    params = synthetic.block_params(shape, seed=11)
    x, ctx, temb, freqs = synthetic.block_inputs(shape, 1, 4680, (6, 26, 30), context_len=512, seed=12)
    inter = {}
    block_forward(params, x, ctx, temb, freqs, shape.heads, shape.eps, intermediates=inter)
    blk = native_block(params, shape, dev)
    with torch.no_grad():
        out = blk(x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev))
        dbg = NativeBlock(blk)(x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev), debug=True)
    torch.cuda.synchronize()
    assert torch.equal(dbg["output"], out), "a debug call changed the block output"
    for name in ("cross_q_linear", "cross_q", "cross_attention", "output"):
        ref = inter[name].float()
        got = dbg[name].reshape(ref.shape).float().cpu()
        # half an ulp of the largest value plus accumulation noise; the
        # normalised queries are formed from the rounded projection (whose
        # own error is that bound) and rounded again: two half-ulps
        ulps = 2 if name == "cross_q" else 1
        bound = max(2e-2, ulps * 2.0 ** -8 * ref.abs().max().item() + 2e-3)
        m = assert_close(got, ref, max_abs=bound, min_cos=0.9999, what=f"L4680 debug {name}")
        print(f"L4680 debug {name}: {m['max_abs']:.5f} (bound {bound:.4f})")


def test_cache_protocol_sequence(dev):
    """update 2 -> 1 -> 0 -> candidate rows, outputs and pool state vs the oracle."""
    from wam_ops import synthetic
    shape = _shape(**TINY)
    params = synthetic.block_params(shape, seed=9)
    blk = native_block(params, shape, dev)
    P = 150
    blk.attn1.init_kv_cache("pos", P, shape.heads, shape.head_dim, dev, torch.bfloat16, 1)
    gcache = blk.attn1.attn_caches["pos"]
    ocache = okv.new_cache(P, shape.heads, shape.head_dim, 1, torch.float32)
    grid = (2, 5, 6)
    for step, upd in enumerate((2, 1, 0, 2, 1)):
        x, ctx, temb, freqs = _inputs(shape, 1, grid, 16, 20 + step)
        ref = block_forward(params, x, ctx, temb, freqs, shape.heads, shape.eps, cache=ocache,
                            update_cache=upd)
        with torch.no_grad():
            out = blk(x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev), update_cache=upd)
        torch.cuda.synchronize()
        assert_close(out.cpu(), ref, 2e-2, 0.9999, f"cache step {step} update {upd}")
        for key in ("mask", "id", "is_pred"):
            assert torch.equal(gcache[key].cpu(), ocache[key]), (step, key)
        valid = okv.valid_slots(ocache)
        assert_close(gcache["k"][:, valid.to(dev)].cpu(), ocache["k"][:, valid], 2e-2, 0.9999, "pool k")
        assert_close(gcache["v"][:, valid.to(dev)].cpu(), ocache["v"][:, valid], 2e-2, 0.9999, "pool v")
    # candidate verification: 3 candidates over pool row 0, read only
    before = {k: v.clone() for k, v in gcache.items()}
    x, ctx, temb, freqs = _inputs(shape, 3, grid, 16, 40)
    rows = torch.zeros(3, dtype=torch.int64)
    ref = block_forward(params, x, ctx, temb, freqs, shape.heads, shape.eps, cache=ocache,
                        update_cache=0, candidate_rows=rows)
    with torch.no_grad():
        out = blk(x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev), update_cache=0,
                  candidate_cache_rows=rows.to(dev))
    torch.cuda.synchronize()
    assert_close(out.cpu(), ref, 2e-2, 0.9999, "candidate verify")
    for k in before:
        assert torch.equal(before[k], gcache[k]), k
    with pytest.raises(ValueError):
        with torch.no_grad():
            blk(x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev), update_cache=0,
                candidate_cache_rows=torch.tensor([0, 1, 0], device=dev))


def test_candidates_isolated(dev):
    """Changing one candidate's tokens leaves every other candidate's output bitwise equal."""
    from wam_ops import synthetic
    shape = _shape(**TINY)
    params = synthetic.block_params(shape, seed=12)
    blk = native_block(params, shape, dev)
    blk.attn1.attn_caches["pos"] = synthetic.kv_pool(shape, 120, 90, batch=1, device=dev)
    x, ctx, temb, freqs = _inputs(shape, 3, (2, 4, 5), 16, 13)
    x, ctx, temb, freqs = x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev)
    rows = torch.zeros(3, dtype=torch.int64, device=dev)
    with torch.no_grad():
        a = blk(x, ctx, temb, freqs, candidate_cache_rows=rows)
        x2 = x.clone()
        x2[1] = -x2[1]
        b = blk(x2, ctx, temb, freqs, candidate_cache_rows=rows)
    assert torch.equal(a[0], b[0]) and torch.equal(a[2], b[2])
    assert not torch.equal(a[1], b[1])


def test_whole_layer_precomputed_context(dev):
    from wam_ops import synthetic
    from wam_ops.whole_layer import WholeLayerBlock
    shape = _shape(**TINY)
    params = synthetic.block_params(shape, seed=14)
    blk = native_block(params, shape, dev)
    x, ctx, temb, freqs = _inputs(shape, 2, (2, 3, 5), 24, 15)
    ctx = ctx[:1].expand(2, -1, -1).contiguous()  # CFG-style identical rows
    x, ctx, temb, freqs = x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev)
    wl = WholeLayerBlock(blk)
    with torch.no_grad():
        base = blk(x, ctx, temb, freqs)
        wl.prepare_context(ctx, precompute=False)
        grouped = wl(x, ctx, temb, freqs)
        wl.prepare_context(ctx, precompute=True)
        pre = wl(x, ctx, temb, freqs)
    assert wl.context_rows is not None and wl.context_rows.tolist() == [0, 0]
    assert torch.equal(base, grouped)
    assert torch.equal(base, pre)


def test_grad_mode_rejected(dev):
    from wam_ops import synthetic
    shape = _shape(**TINY)
    blk = native_block(synthetic.block_params(shape, seed=1), shape, dev)
    x, ctx, temb, freqs = _inputs(shape, 1, (1, 2, 3), 8, 2)
    with pytest.raises(RuntimeError, match="inference-only"):
        blk(x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev))


def test_inputs_and_weights_unchanged(dev):
    """A block call never writes its inputs or parameters (the reference's
    harness asserts inputs_unchanged and weights_unchanged on every native
    call, 算子研究/tools/verify_native.py:130-134): x, context, temb, the
    RoPE table and all 27 parameters are byte-identical after calls with
    update_cache 2, 1 and 0, with debug output, and through WholeLayerBlock
    with precomputed cross K/V."""
    from wam_ops import synthetic
    from wam_ops.native import NativeBlock
    from wam_ops.whole_layer import WholeLayerBlock
    shape = _shape(**TINY)
    params = synthetic.block_params(shape, seed=21)
    blk = native_block(params, shape, dev)
    blk.attn1.init_kv_cache("pos", 150, shape.heads, shape.head_dim, dev, torch.bfloat16, 1)
    x, ctx, temb, freqs = (t.to(dev) for t in _inputs(shape, 1, (2, 5, 6), 16, 22))
    inputs = {"x": x, "context": ctx, "temb": temb, "freqs": freqs}
    before = {k: v.clone() for k, v in inputs.items()}
    wbefore = {n: p.detach().clone() for n, p in blk.named_parameters()}
    rng_cpu, rng_gpu = torch.get_rng_state(), torch.cuda.get_rng_state(dev)
    with torch.no_grad():
        for upd in (2, 1, 0):
            blk(x, ctx, temb, freqs, update_cache=upd)
        NativeBlock(blk)(x, ctx, temb, freqs, update_cache=0, debug=True)
        wl = WholeLayerBlock(blk)
        wl.prepare_context(ctx, precompute=True)
        wl(x, ctx, temb, freqs, update_cache=0)
    torch.cuda.synchronize()
    for k, v in inputs.items():
        assert torch.equal(v, before[k]), f"input {k} changed"
    for n, p in blk.named_parameters():
        assert torch.equal(p.detach(), wbefore[n]), f"parameter {n} changed"
    assert torch.equal(torch.get_rng_state(), rng_cpu) and torch.equal(torch.cuda.get_rng_state(dev), rng_gpu)


def test_prepared_context_batch_checked(dev):
    """A prepared context fixes the batch: a call with another batch is refused
    before anything launches."""
    from wam_ops import synthetic
    from wam_ops.whole_layer import WholeLayerBlock
    shape = _shape(**TINY)
    blk = native_block(synthetic.block_params(shape, seed=23), shape, dev)
    x, ctx, temb, freqs = (t.to(dev) for t in _inputs(shape, 2, (2, 3, 5), 16, 24))
    ctx2 = ctx[:1].expand(2, -1, -1).contiguous()
    wl = WholeLayerBlock(blk)
    with torch.no_grad():
        wl.prepare_context(ctx2, precompute=True)
        wl(x, ctx2, temb, freqs)
        x3 = torch.cat([x, x[:1]])
        temb3 = torch.cat([temb, temb[:1]])
        with pytest.raises(RuntimeError, match="prepared"):
            wl(x3, ctx2, temb3, freqs)
        with pytest.raises(RuntimeError, match="prepared"):
            wl(x, ctx2[:1], temb, freqs)
