"""Model input/output kernels and the whole WanTransformer3DModel forward
(WholeModel) against the oracle (oracle/model.py, pinned by the reference
fixture reference_model_tiny.safetensors).

Bounds:
* patchify is a gather: bit-exact, padding columns exactly zero.
* timestep sinusoid: both sides form the same fp32 frequency and argument;
  exp/sin/cos may differ in the last place, and one ulp of the frequency moves
  an argument of ~1000 by ~6e-5, so max |err| <= 2e-4.
* RoPE frequencies: identical fp32 angles, cos/sin within 2 ulp (<= 2.4e-7).
* rows_linear: fp32 weights vs a float64 reference, relative 1e-5 of the
  row's |x||w|; bf16 outputs within one bf16 ulp of the exact value.
* head_norm (norm_out + modulation): the bf16 ulp bound of the output.
* whole model, bf16 vs the fp32 oracle: max |err| <= 5e-2, cosine >= 0.9999
  (two layers plus the head; the block bound is 2e-2 per layer).
"""
import sys
from pathlib import Path

import pytest
import torch
from safetensors import safe_open
from safetensors.torch import load_file

from oracle import model as om
from oracle import rope as orope
from oracle.metrics import assert_close, compare

GOLD = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLD))
import tiny_model  # noqa: E402

pytestmark = pytest.mark.gpu


def _randn(shape, seed, std=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(dtype)


def test_patchify_bit_exact(dev):
    from wam_ops import ops
    lat = _randn((2, 48, 2, 8, 10), 1, dtype=torch.bfloat16)
    y = ops.patchify(lat.to(dev), (1, 2, 2))
    assert torch.equal(y.cpu(), om.patchify(lat, (1, 2, 2)))
    act = _randn((3, 30, 2, 4, 1), 2, dtype=torch.bfloat16)
    y = ops.patchify(act.to(dev), (1, 1, 1), k_pad=64).cpu()
    assert torch.equal(y[..., :30], om.patchify(act, (1, 1, 1)))
    assert torch.equal(y[..., 30:], torch.zeros_like(y[..., 30:]))
    # an odd patch and shape
    odd = _randn((1, 3, 6, 3, 8), 3, dtype=torch.bfloat16)
    assert torch.equal(ops.patchify(odd.to(dev), (2, 3, 4)).cpu(), om.patchify(odd, (2, 3, 4)))


def test_timestep_embedding(dev):
    from wam_ops import ops
    t = torch.tensor([0.0, 1.0, 37.0, 377.25, 640.0, 812.5, 999.0, 0.5])
    y = ops.timestep_embedding(t.to(dev), 256).cpu()
    ref = om.timestep_sinusoid(t, 256)
    m = compare(y, ref)
    assert m["max_abs"] <= 2e-4, m
    # t = 0 is exact: cos half 1, sin half 0
    assert torch.equal(y[0, :128], torch.ones(128)) and torch.equal(y[0, 128:], torch.zeros(128))
    yb = ops.timestep_embedding(t.to(dev), 256, out_dtype=torch.bfloat16).cpu()
    assert (yb.float() - ref).abs().max() <= 2 ** -8 + 2e-4
    ys = ops.timestep_embedding(t.to(dev), 256, flip_sin_to_cos=False).cpu()
    assert torch.equal(ys[:, :128], y[:, 128:]) and torch.equal(ys[:, 128:], y[:, :128])


def test_rope_freqs(dev):
    from wam_ops import ops
    g = orope.get_mesh_id(3, 26, 30, 0, 1, 5)[None].repeat(2, 1, 1)
    for grid in (g.to(torch.int64), g.to(torch.float32), g.to(torch.float64)):
        y = ops.rope_freqs(grid.to(dev)).cpu()
        ref = orope.rope_freqs(grid)
        assert y.shape == ref.shape
        assert (torch.view_as_real(y) - torch.view_as_real(ref)).abs().max() <= 2.4e-7
    a = orope.get_mesh_id(2, 4, 1, 1, 1, 3, action=True)[None]
    y = ops.rope_freqs(a.to(dev)).cpu()
    assert (torch.view_as_real(y) - torch.view_as_real(orope.rope_freqs(a))).abs().max() <= 2.4e-7
    # a strided view (one sample of a larger batch)
    big = g.to(torch.int64).to(dev)
    y = ops.rope_freqs(big[1:2]).cpu()
    assert (torch.view_as_real(y) - torch.view_as_real(orope.rope_freqs(g[1:2]))).abs().max() <= 2.4e-7


def _rows_ref(x, w, b, act_in, act_out, x_dtype, out_dtype):
    xd = x.double()
    if act_in:
        xd = torch.nn.functional.silu(xd).to(x_dtype).double()
    y = xd @ w.double().t() + (b.double() if b is not None else 0)
    if act_out:
        y = torch.nn.functional.silu(y.to(out_dtype).double())
    return y


@pytest.mark.parametrize("R,N,K", [(8, 3072, 256), (3, 200, 3072), (20, 30, 3072), (5, 64, 30)])
@pytest.mark.parametrize("dtypes", [("f32", "f32", "f32"), ("bf16", "bf16", "bf16"), ("f32", "f32", "bf16"),
                                    ("bf16", "f32", "f32")])
def test_rows_linear(dev, R, N, K, dtypes):
    from wam_ops import ops
    dt = {"f32": torch.float32, "bf16": torch.bfloat16}
    xd, wd, od = (dt[d] for d in dtypes)
    x = _randn((R, K), 10 + R, 1.0, xd)
    w = _randn((N, K), 11 + N, 0.02, wd)
    b = _randn((N,), 12, 0.02, wd)
    scale = (x.double().abs() @ w.double().abs().t()).max().item() + 1e-3
    for act_in, act_out in ((None, None), ("silu", None), (None, "silu")):
        y = ops.rows_linear(x.to(dev), w.to(dev), b.to(dev), act_in=act_in, act_out=act_out, out_dtype=od)
        ref = _rows_ref(x, w, b, act_in, act_out, xd, od)
        err = (y.cpu().double() - ref).abs().max().item()
        bound = 1e-5 * scale + (2 ** -8 * ref.abs().max().item() if od == torch.bfloat16 else 0.0)
        if act_out and od == torch.bfloat16:
            bound += 2 ** -8 * ref.abs().max().item()  # the pre-activation rounding
        assert err <= bound, (act_in, act_out, err, bound)


def test_head_norm(dev):
    from wam_ops import ops
    B, M, D, Fr = 2, 60, 256, 3
    x = _randn((B, M, D), 20, 1.0, torch.bfloat16)
    table = _randn((1, 2, D), 21, 1.0 / 16)
    temb = _randn((B, Fr, D), 22, 0.1, torch.bfloat16)
    y = ops.head_norm(x.to(dev), table.to(dev), temb.to(dev)).cpu()
    tt = torch.repeat_interleave(temb, M // Fr, dim=1)
    mod = table[None] + tt.float()[:, :, None]
    ref = torch.nn.functional.layer_norm(x.float(), (D,), eps=1e-6) * (1 + mod[:, :, 1]) + mod[:, :, 0]
    assert_close(y, ref, 2 ** -8 * ref.abs().max().item() + 1e-3, 0.99999, "head_norm")
    # per-sample and per-token temb lengths
    for L in (1, M):
        tl = _randn((B, L, D), 23 + L, 0.1, torch.bfloat16)
        y = ops.head_norm(x.to(dev), table.to(dev), tl.to(dev)).cpu()
        mod = table[None] + tl.float().expand(B, M, D)[:, :, None]
        ref = torch.nn.functional.layer_norm(x.float(), (D,), eps=1e-6) * (1 + mod[:, :, 1]) + mod[:, :, 0]
        assert_close(y, ref, 2 ** -8 * ref.abs().max().item() + 1e-3, 0.99999, f"head_norm L={L}")


# ------------------------------------------------------------- whole model
@pytest.fixture(scope="module")
def tiny(dev):
    from wam_ops import TransformerModel
    path = str(GOLD / "reference_model_tiny.safetensors")
    with safe_open(path, "pt") as f:
        meta = f.metadata()
    shapes = {}
    for item in meta["params"].split(";"):
        name, shape = item.split(":")
        shapes[name] = tuple(int(s) for s in shape.split("x"))
    P = tiny_model.make_params(shapes)
    model = TransformerModel(**tiny_model.CONFIG)
    fp32 = ("scale_shift_table", "norm2.weight", "norm2.bias", "time_embedder")
    with torch.no_grad():
        for n, p in model.named_parameters():
            keep32 = any(k in n for k in fp32)
            p.data = P[n].to(torch.float32 if keep32 else torch.bfloat16)
    model = model.to(dev).requires_grad_(False)
    return model, P, load_file(path)


def _dev_inputs(t, mode, dev):
    inp = {k: t[f"{mode}.{k}"] for k in ("noisy_latents", "text_emb", "grid_id", "timesteps")}
    d = {k: v.to(dev) for k, v in inp.items()}
    d["noisy_latents"] = d["noisy_latents"].bfloat16()
    d["text_emb"] = d["text_emb"].bfloat16()
    return inp, d


@pytest.mark.parametrize("mode", ["video", "action"])
def test_model_vs_oracle(dev, tiny, mode):
    model, P, t = tiny
    inp, d = _dev_inputs(t, mode, dev)
    with torch.no_grad():
        out = model(d, action_mode=mode == "action")
    torch.cuda.synchronize()
    gold = t[f"{mode}.out"]
    assert out.shape == gold.shape and out.dtype == torch.bfloat16
    ref = om.model_forward(P, inp, tiny_model.CONFIG, action_mode=mode == "action")
    m = assert_close(out.cpu(), ref, 5e-2, 0.9999, f"model {mode} vs oracle")
    m2 = assert_close(out.cpu(), gold, 5e-2, 0.9999, f"model {mode} vs reference fixture")
    print(mode, m, m2)


def test_model_prepared_text_matches(dev, tiny):
    from wam_ops import WholeModel
    model, P, t = tiny
    _, d = _dev_inputs(t, "video", dev)
    whole = WholeModel(model)
    with torch.no_grad():
        plain = whole(d)
        whole.prepare_text(d["text_emb"])
        prepared = whole(d)
        again = whole(d)
    torch.cuda.synchronize()
    assert torch.equal(prepared, again)
    assert_close(prepared.cpu(), plain.cpu(), 1e-2, 0.99999, "prepared text vs per-call text")


def test_model_verify_with_caches(dev, tiny):
    """Candidate verification through the whole model: read-only caches,
    candidate rows into the CFG batch, against the oracle with the same caches."""
    from wam_ops import synthetic
    model, P, t = tiny
    inp, d = _dev_inputs(t, "video", dev)
    shape = synthetic.BlockShape(tiny_model.DIM, tiny_model.CONFIG["num_attention_heads"],
                                 tiny_model.CONFIG["ffn_dim"])
    ocaches = []
    for i, blk in enumerate(model.blocks):
        c = synthetic.kv_pool(shape, 96, 70, batch=2, seed=40 + i, device=dev)
        blk.attn1.attn_caches["pos"] = c
        ocaches.append({k: (v.float().cpu() if v.dtype == torch.bfloat16 else v.cpu()) for k, v in c.items()})
    rows = torch.tensor([1, 0], dtype=torch.int64)
    try:
        with torch.no_grad():
            out = model(d, candidate_cache_rows=rows.to(dev))
        torch.cuda.synchronize()
        ref = om.model_forward(P, inp, tiny_model.CONFIG, caches=ocaches, candidate_rows=rows)
        assert_close(out.cpu(), ref, 5e-2, 0.9999, "model verify vs oracle")
        for blk, oc in zip(model.blocks, ocaches):
            assert torch.equal(blk.attn1.attn_caches["pos"]["mask"].cpu(), oc["mask"])
        with pytest.raises(ValueError):
            with torch.no_grad():
                model(d, update_cache=1, candidate_cache_rows=rows.to(dev))
    finally:
        for blk in model.blocks:
            blk.attn1.attn_caches.pop("pos", None)


def test_model_contract_errors(dev, tiny):
    model, P, t = tiny
    _, d = _dev_inputs(t, "video", dev)
    with pytest.raises(RuntimeError, match="inference-only"):
        model(d)
    with torch.no_grad():
        bad = dict(d, noisy_latents=d["noisy_latents"].float())
        with pytest.raises(RuntimeError, match="bfloat16"):
            model(bad)
        bad = dict(d, timesteps=d["timesteps"][:, :1].repeat(1, 3))
        with pytest.raises(ValueError, match="timesteps"):
            model(bad)
        with pytest.raises(NotImplementedError):
            model(d, train_mode=True)
