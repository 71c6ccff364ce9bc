"""HIP-graph capture and replay of the block and of the block stack.

The reference's published block times are warm CUDA-graph replays
(算子研究/wam_ops/optimized/prepared.py:1-4).  A block call here is a chain of
kernel launches on the caller's stream with no host synchronisation, no
device allocation inside the library and no memset, so torch.cuda.graph can
capture it.  Each test captures once, then replays several times with the
program's own eager work and synchronisations in between, and checks every
replay byte for byte against the eager output of the same inputs, including
after the static inputs have been overwritten with new values (the replay
computes, it does not return a cached result).

* WholeLayerBlock at dim 3072 / 24 heads / FFN 14336 with 256 tokens over a
  1024-slot read-only pool (candidate rows, validated before the capture) and
  512 precomputed context rows; also in the fp8 FFN variant with e4m3
  weights and activations (FFN1 and FFN2 on the fp8 MFMA, the hidden layer
  as MX e4m3).
* BlockStack of three small layers with candidate rows (the one host
  read-back per forward happens before the capture, so the captured forward
  reads nothing back).
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def _check_replays(g, out, eager, static_x, new_x, noise):
    ref = eager()
    torch.cuda.synchronize()
    for i in range(3):
        g.replay()
        noise()  # unrelated eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i} differs from the eager output"
    static_x.copy_(new_x)
    ref2 = eager()
    torch.cuda.synchronize()
    assert not torch.equal(ref2, ref)
    for i in range(2):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref2), f"replay {i} after new inputs differs from the eager output"


@pytest.mark.parametrize("variant", ["bf16", "fp8_act"])
def test_whole_layer_graph_replay(dev, variant):
    from wam_ops import synthetic
    from wam_ops.block import TransformerBlock
    from wam_ops.whole_layer import WholeLayerBlock
    print(f"graph replay: whole layer {variant}", flush=True)
    shape = synthetic.BlockShape(3072, 24, 14336)
    params = synthetic.block_params(shape, seed=61)
    blk = TransformerBlock(shape.dim, shape.ffn, shape.heads, cross_attn_norm=True, eps=shape.eps)
    with torch.no_grad():
        for name, prm in blk.named_parameters():
            prm.data = params[name].to(dev)
    blk = blk.to(dev)
    blk.attn1.attn_caches["pos"] = synthetic.kv_pool(shape, 1024, 768, batch=1, seed=62, device=dev)
    M = 4 * 8 * 8
    x, ctx, temb, freqs = synthetic.block_inputs(shape, 2, M, (4, 8, 8), context_len=512, seed=63,
                                                 device=dev)
    x2, *_ = synthetic.block_inputs(shape, 2, M, (4, 8, 8), context_len=512, seed=64, device=dev)
    rows = torch.zeros(2, dtype=torch.int64, device=dev)
    opts = dict(ffn_fp8=True, ffn_act_fp8=2) if variant == "fp8_act" else {}
    wl = WholeLayerBlock(blk, **opts)
    junk = torch.randn(1 << 20, device=dev)
    with torch.no_grad():
        wl.prepare_context(ctx, precompute=True)

        def fn():
            return wl(x, ctx, temb, freqs, candidate_cache_rows=rows)
        fn()  # validates the rows once (host read-back) before the capture
        g, out = _capture(fn)
        _check_replays(g, out, lambda: fn().clone(), x, x2, lambda: junk.mul_(1.0001))


def test_block_stack_graph_replay(dev):
    from wam_ops import BlockStack, synthetic
    from wam_ops.block import TransformerBlock
    print("graph replay: block stack", flush=True)
    shape = synthetic.BlockShape(256, 2, 512)
    blocks = []
    for i in range(3):
        p = synthetic.block_params(shape, seed=70 + i)
        blk = TransformerBlock(shape.dim, shape.ffn, shape.heads, cross_attn_norm=True, eps=shape.eps)
        with torch.no_grad():
            for name, prm in blk.named_parameters():
                prm.data = p[name].to(dev)
        blk = blk.to(dev)
        blk.attn1.attn_caches["pos"] = synthetic.kv_pool(shape, 120, 90, batch=2, seed=80 + i, device=dev)
        blocks.append(blk)
    x, ctx, temb, freqs = synthetic.block_inputs(shape, 3, 60, (2, 5, 6), context_len=16, seed=90,
                                                 per_token_temb=True, device=dev)
    x2, *_ = synthetic.block_inputs(shape, 3, 60, (2, 5, 6), context_len=16, seed=91,
                                    per_token_temb=True, device=dev)
    rows = torch.tensor([1, 0, 1], dtype=torch.int64, device=dev)
    stack = BlockStack(blocks)
    junk = torch.randn(1 << 16, device=dev)
    with torch.no_grad():
        stack.prepare_context(ctx)

        def fn():
            # rows validated by the warm-up calls: the captured forward reads nothing back
            return stack(x, ctx, temb, freqs, candidate_cache_rows=rows)
        g, out = _capture(fn)
        _check_replays(g, out, lambda: fn().clone(), x, x2, lambda: junk.add_(1.0))
