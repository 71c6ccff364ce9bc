"""The 30-layer speculative verify forward at its real size.

Workload: 30 Wan2.2-5B-shaped blocks, each with its own 7800-slot KV pool
holding 6240 committed prefix rows (pool row 0), 4 candidates x 1560 tokens,
a 512-token text context with precomputed cross K/V, per-sample temb.  This is
the block loop of WanTransformer3DModel.forward for a verify call
(投机采样/wam-p0-worktree/wan_va/modules/model.py:1091-1098, caller
wan_va_server.py:1904-1935).  The reference's replay harness gates the full
30-layer model the same way (算子研究/tools/replay.py:116-189) and checks that
inputs, weights and RNG are untouched by a native call
(算子研究/tools/verify_native.py:130-134).

Checked here, on the GPU:
* the output is finite; two runs are bitwise equal; the BlockStack output is
  bitwise equal to calling each WholeLayerBlock in turn;
* every layer's pool (k, v, id, mask, is_pred) is bitwise unchanged
  (candidate verification is read-only);
* negating one candidate's tokens leaves the other candidates bitwise equal;
* hidden states, context, temb, RoPE table and all 30 x 27 parameters are
  byte-identical afterwards;
* the whole run happens under torch.inference_mode (inference tensors, no
  version counters);
* a 2-layer stack at the same size against the fp32 oracle: each layer at the
  block bound (2e-2 / 0.9999) with the oracle fed the previous HIP layer's
  output, and end to end at the stack bound (5e-2 / 0.9999).
"""
import pytest
import torch

from oracle.block import block_forward
from oracle.metrics import assert_close

pytestmark = pytest.mark.gpu

B, M, PREFIX, LC = 4, 1560, 6240, 512
GRID = (2, 26, 30)


def _block(shape, dev, seed):
    from wam_ops import synthetic
    from wam_ops.block import TransformerBlock
    params = synthetic.block_params(shape, seed=seed, device=dev)
    with torch.device("meta"):
        blk = TransformerBlock(shape.dim, shape.ffn, shape.heads, cross_attn_norm=True, eps=shape.eps)
    blk.load_state_dict(params, assign=True)
    return blk, params


def _stack_setup(dev, layers, seed0=100):
    from wam_ops import synthetic
    shape = synthetic.WAN22_5B
    blocks, params = [], []
    for i in range(layers):
        blk, p = _block(shape, dev, seed0 + i)
        blk.attn1.attn_caches["pos"] = synthetic.kv_pool(shape, PREFIX + M, PREFIX, batch=1,
                                                         seed=seed0 + 300 + i, device=dev)
        blocks.append(blk)
        params.append(p)
    x, ctx, temb, freqs = synthetic.block_inputs(shape, B, M, GRID, context_len=LC, seed=seed0 + 7,
                                                 device=dev)
    return shape, blocks, params, (x, ctx, temb, freqs)


def test_verify_stack30_full_size(dev):
    from wam_ops import BlockStack
    shape, blocks, params, (x, ctx, temb, freqs) = _stack_setup(dev, 30)
    print(f"C5 stack: 30 layers, {B} x {M} tokens over {PREFIX} cached rows, {LC} text tokens", flush=True)
    weights_before = [{k: v.clone() for k, v in p.items()} for p in params]
    caches_before = [{k: v.clone() for k, v in b.attn1.attn_caches["pos"].items()} for b in blocks]
    inputs_before = [t.clone() for t in (x, ctx, temb, freqs)]
    stack = BlockStack(blocks)
    with torch.inference_mode():
        rows = torch.zeros(B, dtype=torch.int64, device=dev)
        stack.prepare_context(ctx, precompute=True)
        out1 = stack(x, ctx, temb, freqs, candidate_cache_rows=rows)
        out2 = stack(x, ctx, temb, freqs, candidate_cache_rows=rows)
        h = x
        for layer in stack.layers:
            h = layer(h, ctx, temb, freqs, candidate_cache_rows=rows)
        xn = x.clone()
        xn[2] = -xn[2]
        out3 = stack(xn, ctx, temb, freqs, candidate_cache_rows=rows)
    torch.cuda.synchronize()
    assert out1.shape == x.shape and out1.dtype == torch.bfloat16
    assert bool(torch.isfinite(out1.float()).all()), "30-layer verify output is not finite"
    assert torch.equal(out1, out2), "two runs differ"
    assert torch.equal(out1, h), "BlockStack differs from the per-layer WholeLayerBlock calls"
    for c in (0, 1, 3):
        assert torch.equal(out3[c], out1[c]), f"candidate {c} changed when candidate 2 changed"
    assert not torch.equal(out3[2], out1[2])
    for i, (blk, before) in enumerate(zip(blocks, caches_before)):
        after = blk.attn1.attn_caches["pos"]
        for key in ("k", "v", "id", "mask", "is_pred"):
            assert torch.equal(after[key], before[key]), f"layer {i} cache {key} changed"
    for name, t0, t1 in zip(("x", "context", "temb", "freqs"), inputs_before, (x, ctx, temb, freqs)):
        assert torch.equal(t0, t1), f"input {name} changed"
    for i, (p, before) in enumerate(zip(params, weights_before)):
        for k in p:
            assert torch.equal(p[k], before[k]), f"layer {i} parameter {k} changed"
    print(f"C5 stack: out std {out1.float().std().item():.4f}, max |out| {out1.float().abs().max().item():.3f}",
          flush=True)


def test_verify_stack_full_size_vs_oracle(dev):
    from wam_ops import BlockStack
    shape, blocks, params, (x, ctx, temb, freqs) = _stack_setup(dev, 2, seed0=140)
    ocaches = [{k: (v.float().cpu() if v.dtype == torch.bfloat16 else v.cpu())
                for k, v in b.attn1.attn_caches["pos"].items()} for b in blocks]
    stack = BlockStack(blocks)
    rows = torch.zeros(B, dtype=torch.int64, device=dev)
    with torch.no_grad():
        stack.prepare_context(ctx, precompute=True)
        per_layer = []
        h = x
        for layer in stack.layers:
            h = layer(h, ctx, temb, freqs, candidate_cache_rows=rows)
            per_layer.append(h.cpu())
        out = stack(x, ctx, temb, freqs, candidate_cache_rows=rows)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), per_layer[-1])
    xc, cc, tc, fc, rc = x.cpu(), ctx.cpu(), temb.cpu(), freqs.cpu(), rows.cpu()
    pc = [{k: v.cpu() for k, v in p.items()} for p in params]
    prev = xc
    refs = []
    for i in range(2):
        ref = block_forward(pc[i], prev, cc, tc, fc, shape.heads, shape.eps, cache=ocaches[i],
                            update_cache=0, candidate_rows=rc)
        refs.append(ref)
        assert_close(per_layer[i], ref, 2e-2, 0.9999, f"C5 full-size layer {i} (oracle fed HIP input)")
        prev = per_layer[i]
    # end to end: the oracle's own composition (layer 0 is the same call as above)
    ref = block_forward(pc[1], refs[0], cc, tc, fc, shape.heads, shape.eps, cache=ocaches[1],
                        update_cache=0, candidate_rows=rc)
    assert_close(out.cpu(), ref, 5e-2, 0.9999, "C5 full-size 2-layer stack end to end")
