"""The model-level oracle (oracle/model.py) against golden vectors written from
the reference's own WanTransformer3DModel.forward
(tests/golden/make_model_vectors.py), plus the closed forms that pin the
timestep sinusoid and the patch rearranges.  CPU only; the fixture holds
inputs and outputs, parameters are regenerated from tests/golden/tiny_model.py."""
import math
import sys
from pathlib import Path

import pytest
import torch
from einops import rearrange
from safetensors import safe_open
from safetensors.torch import load_file

from oracle import model as om
from oracle import rope as orope
from oracle.metrics import compare

GOLD = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLD))
import tiny_model  # noqa: E402


@pytest.fixture(scope="module")
def model_gold():
    path = str(GOLD / "reference_model_tiny.safetensors")
    with safe_open(path, "pt") as f:
        meta = f.metadata()
    shapes = {}
    for item in meta["params"].split(";"):
        name, shape = item.split(":")
        shapes[name] = tuple(int(s) for s in shape.split("x"))
    return load_file(path), tiny_model.make_params(shapes)


def _inputs(t, mode):
    return {k: t[f"{mode}.{k}"] for k in ("noisy_latents", "text_emb", "grid_id", "timesteps")}


@pytest.mark.parametrize("mode", ["video", "action"])
def test_oracle_model_matches_reference(model_gold, mode):
    t, P = model_gold
    out = om.model_forward(P, _inputs(t, mode), tiny_model.CONFIG, action_mode=mode == "action")
    m = compare(out, t[f"{mode}.out"])
    assert out.shape == t[f"{mode}.out"].shape
    assert m["max_abs"] < 2e-5 and m["cosine"] > 0.9999999, m


def test_planted_mistakes_fail_the_golden(model_gold, monkeypatch):
    """Plausible mistakes in the oracle's model-level composition must fail the
    golden comparison by a wide margin."""
    t, P = model_gold
    inp, gold = _inputs(t, "video"), t["video.out"]

    def err():
        return compare(om.model_forward(P, inp, tiny_model.CONFIG), gold)["max_abs"]

    good_head, good_sin, good_patch = om.head, om.timestep_sinusoid, om.patchify

    def swapped_head(P_, x, temb, eps=1e-6, proj="proj_out"):  # shift and scale exchanged
        P2 = dict(P_)
        P2["scale_shift_table"] = P_["scale_shift_table"].flip(1)
        return good_head(P2, x, temb, eps, proj)
    monkeypatch.setattr(om, "head", swapped_head)
    assert err() > 1e-2
    monkeypatch.setattr(om, "head", good_head)
    monkeypatch.setattr(om, "timestep_sinusoid",
                        lambda t_, dim=256, **kw: good_sin(t_, dim, flip_sin_to_cos=False))
    assert err() > 1e-3
    monkeypatch.setattr(om, "timestep_sinusoid", good_sin)
    monkeypatch.setattr(om, "patchify",  # channel-last feature order
                        lambda lat, patch: rearrange(lat, "b c (f p1) (h p2) (w p3) -> b (f h w) (p1 p2 p3 c)",
                                                     p1=patch[0], p2=patch[1], p3=patch[2]))
    assert err() > 1e-2
    monkeypatch.setattr(om, "patchify", good_patch)
    assert err() < 2e-5


def test_timestep_sinusoid_closed_forms():
    t = torch.tensor([0.0, 1.0, 812.5, 37.0])
    e = om.timestep_sinusoid(t, 256).double()
    assert e.shape == (4, 256)
    # t = 0: cos half is 1, sin half is 0 (flip_sin_to_cos puts cos first)
    assert torch.equal(e[0, :128], torch.ones(128, dtype=torch.float64))
    assert torch.equal(e[0, 128:], torch.zeros(128, dtype=torch.float64))
    # frequency i is 10000^(-i/128): column 0 is cos(t), column 128 sin(t)
    for j, tv in enumerate(t.tolist()):
        assert abs(e[j, 0] - math.cos(tv)) < 1e-6 and abs(e[j, 128] - math.sin(tv)) < 1e-6
        f127 = 10000 ** (-127 / 128)
        assert abs(e[j, 127] - math.cos(tv * f127)) < 1e-5
        assert abs(e[j, 255] - math.sin(tv * f127)) < 1e-5
        f64 = 10000 ** (-64 / 128)
        assert abs(e[j, 64] - math.cos(tv * f64)) < 2e-4
    # each (cos, sin) pair lies on the unit circle
    assert ((e[:, :128] ** 2 + e[:, 128:] ** 2) - 1).abs().max() < 1e-6


def test_patchify_matches_einops_and_loop():
    g = torch.Generator().manual_seed(5)
    lat = torch.randn(2, 3, 4, 6, 8, generator=g)
    p = (1, 2, 2)
    x = om.patchify(lat, p)
    ref = rearrange(lat, "b c (f p1) (h p2) (w p3) -> b (f h w) (c p1 p2 p3)", p1=1, p2=2, p3=2)
    assert torch.equal(x, ref)
    # brute force on one token
    b, fi, hi, wi = 1, 2, 1, 3
    tok = (fi * 3 + hi) * 4 + wi
    want = [lat[b, c, fi, 2 * hi + a, 2 * wi + d] for c in range(3) for a in range(2) for d in range(2)]
    assert torch.equal(x[b, tok], torch.stack(want))
    assert torch.equal(om.patchify(lat, (1, 1, 1)), rearrange(lat, "b c f h w -> b (f h w) c"))
    y = torch.randn(2, 5, 4 * 7, generator=g)
    assert torch.equal(om.unpatchify(y, p), rearrange(y, "b l (n c) -> b (l n) c", n=4))


def test_mesh_ids_match_reference_fixture(model_gold):
    t, _ = model_gold
    g = orope.get_mesh_id(2, 4, 5, 0, 1, 3)
    assert torch.equal(g, t["video.grid_id"][0].to(g.dtype))
    a = orope.get_mesh_id(2, 4, 1, 1, 1, 3, action=True)
    assert torch.equal(a, t["action.grid_id"][0])
