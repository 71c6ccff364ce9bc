"""Multi-layer speculative verify (BlockStack) against the fp32 oracle.

Each layer is checked at the block bound (max |out - ref| <= 2e-2, cosine >=
0.9999) with the oracle fed the HIP path's previous-layer output, so that
every layer is pinned at the stated tolerance; the end-to-end drift of the
whole stack against the oracle's own composition is bounded at 5e-2 / 0.9999.
The stack must equal calling each WholeLayerBlock in turn bit for bit.
"""
import pytest
import torch

from oracle.block import block_forward
from oracle.metrics import assert_close

pytestmark = pytest.mark.gpu

TINY = dict(dim=256, heads=2, ffn=512)


def _setup(dev, n_layers=3, B=3, grid=(2, 5, 6), Lc=16, pool=120, prefix=90, cfg_rows=2, seed=30):
    from wam_ops import synthetic
    from wam_ops.block import TransformerBlock
    shape = synthetic.BlockShape(**TINY)
    params, blocks, ocaches = [], [], []
    for i in range(n_layers):
        p = synthetic.block_params(shape, seed=seed + i)
        blk = TransformerBlock(shape.dim, shape.ffn, shape.heads, cross_attn_norm=True, eps=shape.eps)
        with torch.no_grad():
            for name, prm in blk.named_parameters():
                prm.data = p[name].to(dev)
        blk = blk.to(dev)
        cache = synthetic.kv_pool(shape, pool, prefix, batch=cfg_rows, seed=seed + 100 + i, device=dev)
        blk.attn1.attn_caches["pos"] = cache
        params.append(p)
        blocks.append(blk)
        ocaches.append({k: (v.float().cpu() if v.dtype == torch.bfloat16 else v.cpu()) for k, v in cache.items()})
    M = grid[0] * grid[1] * grid[2]
    x, ctx, temb, freqs = synthetic.block_inputs(shape, B, M, grid, context_len=Lc, seed=seed + 50,
                                                 per_token_temb=True)
    return shape, params, blocks, ocaches, (x, ctx, temb, freqs)


def test_stack_layers_vs_oracle(dev):
    from wam_ops import BlockStack, WholeLayerBlock
    shape, params, blocks, ocaches, (x, ctx, temb, freqs) = _setup(dev)
    rows = torch.tensor([1, 0, 1], dtype=torch.int64)
    stack = BlockStack(blocks)
    with torch.no_grad():
        stack.prepare_context(ctx.to(dev))
        out = stack(x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev), candidate_cache_rows=rows.to(dev))
        # the same layers one by one
        h = x.to(dev)
        per_layer = []
        for layer in stack.layers:
            h = layer(h, ctx.to(dev), temb.to(dev), freqs.to(dev), candidate_cache_rows=rows.to(dev))
            per_layer.append(h)
    torch.cuda.synchronize()
    assert torch.equal(out, per_layer[-1])
    # each layer at the block bound, oracle fed the previous HIP layer output
    prev = x
    for i, (p, oc) in enumerate(zip(params, ocaches)):
        ref = block_forward(p, prev, ctx, temb, freqs, shape.heads, shape.eps, cache=oc,
                            update_cache=0, candidate_rows=rows)
        assert_close(per_layer[i].cpu(), ref, 2e-2, 0.9999, f"verify layer {i}")
        prev = per_layer[i].cpu()
    # whole-stack drift against the oracle's own composition
    ref = x
    for p, oc in zip(params, ocaches):
        ref = block_forward(p, ref, ctx, temb, freqs, shape.heads, shape.eps, cache=oc,
                            update_cache=0, candidate_rows=rows)
    assert_close(out.cpu(), ref, 5e-2, 0.9999, "verify stack end to end")
    # caches are read only
    for blk, oc in zip(blocks, ocaches):
        c = blk.attn1.attn_caches["pos"]
        for key in ("mask", "id", "is_pred"):
            assert torch.equal(c[key].cpu(), oc[key])


def test_stack_contract_errors(dev):
    from wam_ops import BlockStack
    shape, params, blocks, ocaches, (x, ctx, temb, freqs) = _setup(dev, n_layers=2, B=2)
    stack = BlockStack(blocks)
    args = (x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev))
    with torch.no_grad():
        with pytest.raises(ValueError):
            stack(*args, candidate_cache_rows=torch.tensor([0, 2], device=dev))  # row 2 >= 2 CFG rows
        with pytest.raises(ValueError):
            stack(*args, update_cache=1, candidate_cache_rows=torch.tensor([0, 1], device=dev))
        with pytest.raises(ValueError):
            stack(*args, candidate_cache_rows=torch.tensor([0, 1], device=dev, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="inference-only"):
        stack(*args, candidate_cache_rows=torch.tensor([0, 1], device=dev))


def test_stack_under_inference_mode(dev):
    """The verify forward under torch.inference_mode (inference tensors carry
    no version counter) gives the same output as under no_grad."""
    from wam_ops import BlockStack
    shape, params, blocks, ocaches, (x, ctx, temb, freqs) = _setup(dev, n_layers=2, B=3)
    stack = BlockStack(blocks)
    args = (x.to(dev), ctx.to(dev), temb.to(dev), freqs.to(dev))
    with torch.no_grad():
        stack.prepare_context(args[1])
        ref = stack(*args, candidate_cache_rows=torch.tensor([1, 0, 1], device=dev))
    with torch.inference_mode():
        rows = torch.tensor([1, 0, 1], device=dev)
        assert rows.is_inference()
        out = stack(*args, candidate_cache_rows=rows)
        out2 = stack(*args, candidate_cache_rows=rows)
        with pytest.raises(ValueError):
            stack(*args, candidate_cache_rows=torch.tensor([0, 2, 0], device=dev))
    assert torch.equal(out, ref) and torch.equal(out2, ref)
