"""The whole WanTransformer3DModel forward (WholeModel) at the speculative
verify size: latents [4, 48, 2, 52, 60] (4 candidates x 1560 tokens), text
[4, 512, 4096], per-frame timesteps [4, 2], every layer reading a 6240-row
committed prefix from its own read-only KV pool (candidate rows 0).  This is
the call of 投机采样/wam-p0-worktree/wan_va/wan_va_server.py:1904-1935 into
model.py:1033-1116; the reference's replay harness gates the full model the
same way (算子研究/tools/replay.py:116-189).

* 30 layers: the output is finite, two forwards are bitwise equal, the
  prepared text (embedder + every layer's cross K/V once per prompt) gives
  the bitwise output of the per-call text path, changing one candidate's
  latents leaves the other candidates bitwise equal, and every pool is
  bitwise unchanged.
* one full-size layer plus the model I/O (4096 -> 3072 text embedder, patch
  embedding, RoPE from grid ids, condition embedder, norm_out + modulation,
  proj_out and unpatchify) against the oracle's model_forward at the model
  bound (5e-2 / 0.9999; the block bound is 2e-2 per layer).
"""
import pytest
import torch

from oracle import model as om
from oracle.metrics import assert_close

pytestmark = pytest.mark.gpu

B, FRAMES, HP, WP, PREFIX, LC = 4, 2, 26, 30, 6240, 512
M = FRAMES * HP * WP


def _model(dev, layers, seed0):
    from wam_ops import TransformerModel, synthetic
    from wam_ops.block import TransformerBlock
    shape = synthetic.WAN22_5B
    with torch.device("meta"):
        model = TransformerModel(num_attention_heads=shape.heads, attention_head_dim=shape.head_dim,
                                 ffn_dim=shape.ffn, num_layers=0)
    model.load_state_dict(synthetic.model_io_params(model, seed=seed0, device=dev), assign=True)
    blocks = []
    for i in range(layers):
        with torch.device("meta"):
            blk = TransformerBlock(shape.dim, shape.ffn, shape.heads, cross_attn_norm=True, eps=shape.eps)
        blk.load_state_dict(synthetic.block_params(shape, seed=seed0 + 1 + i, device=dev), assign=True)
        blk.attn1.attn_caches["pos"] = synthetic.kv_pool(shape, PREFIX + M, PREFIX, batch=1,
                                                         seed=seed0 + 200 + i, device=dev)
        blocks.append(blk)
    model.blocks = torch.nn.ModuleList(blocks)
    return model.requires_grad_(False), shape


def _inputs(dev, seed):
    from wam_ops import synthetic
    g = torch.Generator(device=dev).manual_seed(seed)
    lat = torch.randn(B, 48, FRAMES, 2 * HP, 2 * WP, generator=g, device=dev).to(torch.bfloat16)
    text = torch.randn(B, LC, 4096, generator=g, device=dev).to(torch.bfloat16)
    grid = synthetic.mesh_grid_ids(FRAMES, HP, WP).to(torch.int64)
    grid = torch.cat([grid, torch.zeros_like(grid[:1])])[None].repeat(B, 1, 1).to(dev)
    ts = torch.tensor([[0.0, 500.0 + 50 * k] for k in range(B)], device=dev)
    return {"noisy_latents": lat, "text_emb": text, "grid_id": grid, "timesteps": ts}


def test_model30_full_size_properties(dev):
    from wam_ops import WholeModel
    model, _ = _model(dev, 30, 700)
    inp = _inputs(dev, 701)
    print(f"model30: latents {list(inp['noisy_latents'].shape)}, text {list(inp['text_emb'].shape)}, "
          f"30 layers over {PREFIX} cached rows", flush=True)
    pools = [{k: v.clone() for k, v in b.attn1.attn_caches["pos"].items()} for b in model.blocks]
    rows = torch.zeros(B, dtype=torch.int64, device=dev)
    whole = WholeModel(model)
    with torch.no_grad():
        plain = whole(inp, candidate_cache_rows=rows)
        whole.prepare_text(inp["text_emb"])
        out1 = whole(inp, candidate_cache_rows=rows)
        out2 = whole(inp, candidate_cache_rows=rows)
        changed = dict(inp, noisy_latents=inp["noisy_latents"].clone())
        changed["noisy_latents"][1] = -changed["noisy_latents"][1]
        out3 = whole(changed, candidate_cache_rows=rows)
    torch.cuda.synchronize()
    # unpatchified as 'b l (n c) -> b (l n) c' (model.py:1110-1112): [4, 1560 x 4, 48]
    assert out1.shape == (B, M * 4, 48) and out1.dtype == torch.bfloat16
    assert bool(torch.isfinite(out1.float()).all()), "model output is not finite"
    assert torch.equal(out1, out2), "two forwards differ"
    assert torch.equal(out1, plain), "prepared text differs from the per-call text path"
    for c in (0, 2, 3):
        assert torch.equal(out3[c], out1[c]), f"candidate {c} changed with candidate 1's latents"
    assert not torch.equal(out3[1], out1[1])
    for i, (blk, before) in enumerate(zip(model.blocks, pools)):
        after = blk.attn1.attn_caches["pos"]
        for key in ("k", "v", "id", "mask", "is_pred"):
            assert torch.equal(after[key], before[key]), f"layer {i} pool {key} changed"
    print(f"model30: out std {out1.float().std().item():.4f}", flush=True)


def test_model_full_size_one_layer_vs_oracle(dev):
    model, shape = _model(dev, 1, 800)
    inp = _inputs(dev, 801)
    print("model full size, 1 layer + I/O vs oracle", flush=True)
    rows = torch.zeros(B, dtype=torch.int64, device=dev)
    ocaches = [{k: (v.float().cpu() if v.dtype == torch.bfloat16 else v.cpu())
                for k, v in b.attn1.attn_caches["pos"].items()} for b in model.blocks]
    with torch.no_grad():
        out = model(inp, candidate_cache_rows=rows)
    torch.cuda.synchronize()
    P = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    cfg = dict(patch_size=(1, 2, 2), num_attention_heads=shape.heads, attention_head_dim=shape.head_dim,
               num_layers=1, eps=shape.eps, freq_dim=256)
    cpu_inp = {k: v.cpu() for k, v in inp.items()}
    ref = om.model_forward(P, cpu_inp, cfg, caches=ocaches, candidate_rows=rows.cpu())
    m = assert_close(out.cpu(), ref, 5e-2, 0.9999, "full-size model (1 layer + I/O) vs oracle")
    print("full-size model vs oracle", m)
