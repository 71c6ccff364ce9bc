"""The oracle against golden vectors written from the reference's own
WanTransformerBlock / WanAttention (tests/golden/make_reference_vectors.py).
CPU only; the fixtures hold data, no reference code."""
from pathlib import Path

import pytest
import torch
from safetensors.torch import load_file

from oracle import kvcache as okv
from oracle.block import block_forward
from oracle.metrics import compare

GOLD = Path(__file__).resolve().parent / "golden"
HEADS = 2


def _params(t):
    return {k[len("param."):]: v for k, v in t.items() if k.startswith("param.")}


def _freqs(t):
    return torch.view_as_complex(t.contiguous())


@pytest.fixture(scope="module")
def block_gold():
    return load_file(str(GOLD / "reference_block_tiny.safetensors"))


@pytest.fixture(scope="module")
def cache_gold():
    return load_file(str(GOLD / "reference_cache_tiny.safetensors"))


def test_oracle_fp32_matches_reference(block_gold):
    t = block_gold
    out = block_forward(_params(t), t["x"], t["context"], t["temb"], _freqs(t["freqs"]), HEADS, 1e-6)
    m = compare(out, t["out_fp32"])
    assert m["max_abs"] < 2e-5 and m["cosine"] > 0.9999999, m


def test_oracle_bf16_emulation_matches_reference(block_gold):
    t = block_gold
    out = block_forward(_params(t), t["x"], t["context"], t["temb"], _freqs(t["freqs"]), HEADS, 1e-6,
                        dtype=torch.bfloat16)
    assert out.dtype == torch.bfloat16
    m = compare(out, t["out_bf16"])
    assert m["max_abs"] <= 2 ** -6, m  # at most one bf16 ulp apart


def test_rope_construction_matches_reference(block_gold):
    from oracle import rope as orope
    t = block_gold
    freqs = orope.rope_freqs(orope.get_mesh_id(3, 4, 5)[None])
    assert torch.equal(torch.view_as_real(freqs), t["freqs"])


def test_oracle_cache_protocol_matches_reference(cache_gold):
    t = cache_gold
    params = _params(load_file(str(GOLD / "reference_block_tiny.safetensors")))
    cache = okv.new_cache(100, HEADS, 128, 1, torch.float32)
    for i in range(5):
        upd = [2, 1, 0, 2, 1][i]
        # the fixture was written on the CPU, so its eviction order is CPU torch.argsort's
        out = block_forward(params, t[f"s{i}.x"], t[f"s{i}.context"], t[f"s{i}.temb"],
                            _freqs(t[f"s{i}.freqs"]), HEADS, 1e-6, cache=cache, update_cache=upd,
                            evict_order="torch")
        m = compare(out, t[f"s{i}.out"])
        assert m["max_abs"] < 2e-5, (i, m)
        for key in ("mask", "id", "is_pred"):
            assert torch.equal(cache[key], t[f"s{i}.{key}"]), (i, key)
    valid = okv.valid_slots(cache)
    assert torch.allclose(cache["k"][:, valid], t["final.k"][:, valid], atol=1e-5)
    assert torch.allclose(cache["v"][:, valid], t["final.v"][:, valid], atol=1e-5)
    out = block_forward(params, t["cand.x"], t["cand.context"], t["cand.temb"], _freqs(t["cand.freqs"]),
                        HEADS, 1e-6, cache=cache, update_cache=0, candidate_rows=t["cand.rows"])
    m = compare(out, t["cand.out"])
    assert m["max_abs"] < 2e-5, m


def test_stable_eviction_differs_only_in_tie_order(cache_gold):
    """With the stable tie order (the HIP kernel's and CUDA's), the eviction step
    evicts the same number of slots, all of the oldest id, lowest slots first."""
    t = cache_gold
    params = _params(load_file(str(GOLD / "reference_block_tiny.safetensors")))
    cache = okv.new_cache(100, HEADS, 128, 1, torch.float32)
    for i in range(4):
        upd = [2, 1, 0, 2][i]
        before = okv.clone_cache(cache)
        block_forward(params, t[f"s{i}.x"], t[f"s{i}.context"], t[f"s{i}.temb"],
                      _freqs(t[f"s{i}.freqs"]), HEADS, 1e-6, cache=cache, update_cache=upd)
    ref_evicted = set((before["mask"] & (t["s3.id"] != before["id"])).nonzero().flatten().tolist())
    ours = set((before["mask"] & (cache["id"] != before["id"])).nonzero().flatten().tolist())
    assert len(ours) == len(ref_evicted) == 20
    assert all(int(before["id"][s]) == 0 for s in ours | ref_evicted)
    assert sorted(ours) == list(range(20))
    assert torch.equal(cache["mask"], t["s3.mask"]) and torch.equal(cache["is_pred"], t["s3.is_pred"])
