"""Host-side behaviour of the operator surface that needs no GPU: class
swapping by install_block, its refusals, the grad-mode guard, the parameter
order and context grouping."""
import pytest
import torch

from wam_ops import install_block, install_model
from wam_ops.block import TransformerBlock
from wam_ops.native import NativeBlock, block_eps, block_parameters
from wam_ops.parameters import Attention
from wam_ops.whole_layer import WholeLayerBlock


class RefLikeAttention(torch.nn.Module):
    """A module with WanAttention's attribute layout (model.py:289-346)."""

    def __init__(self, dim, heads):
        super().__init__()
        self.heads = heads
        self.to_q, self.to_k, self.to_v = (torch.nn.Linear(dim, dim) for _ in range(3))
        self.to_out = torch.nn.ModuleList([torch.nn.Linear(dim, dim), torch.nn.Dropout(0.0)])
        self.norm_q = torch.nn.RMSNorm(dim, eps=1e-6)
        self.norm_k = torch.nn.RMSNorm(dim, eps=1e-6)
        self.attn_caches = {}
        self.cache_mode = "original"


class RefLikeBlock(torch.nn.Module):
    def __init__(self, dim=256, ffn=512, heads=2):
        super().__init__()
        ref = TransformerBlock(dim, ffn, heads, cross_attn_norm=True)
        self.attn_mode = "torch"
        self.norm1, self.norm2, self.norm3 = ref.norm1, ref.norm2, ref.norm3
        self.attn1, self.attn2 = RefLikeAttention(dim, heads), RefLikeAttention(dim, heads)
        self.attn2.attn_caches = None
        self.ffn = ref.ffn
        self.scale_shift_table = ref.scale_shift_table

    def forward(self, *a, **k):
        return "original"


def test_install_block_swaps_and_restores():
    blk = RefLikeBlock()
    classes = (type(blk), type(blk.attn1), type(blk.attn2))
    with install_block(blk, "optimized") as b:
        assert type(b) is TransformerBlock and type(b.attn1) is Attention
        assert isinstance(b.__dict__["_native_block"], NativeBlock)
    assert (type(blk), type(blk.attn1), type(blk.attn2)) == classes
    assert "_native_block" not in blk.__dict__
    assert blk() == "original"


def test_install_refusals():
    blk = RefLikeBlock()
    blk.attn_mode = "flashattn"
    with pytest.raises(ValueError):
        with install_block(blk):
            pass
    blk = RefLikeBlock()
    blk.attn1.cache_mode = "lifecycle"
    with pytest.raises(ValueError):
        with install_block(blk):
            pass
    blk = RefLikeBlock()
    blk.forward = lambda *a: None
    with pytest.raises(ValueError):
        with install_block(blk):
            pass
    blk = RefLikeBlock()
    with pytest.raises(ValueError):
        with install_block(blk, "baseline", execution_mode="tiled"):
            pass
    with pytest.raises(ValueError):
        with install_block(RefLikeBlock(), "triton"):
            pass


def test_install_model_all_blocks():
    class M(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.blocks = torch.nn.ModuleList([RefLikeBlock(), RefLikeBlock()])
    m = M()
    with install_model(m, "optimized", execution_mode="persistent"):
        assert all(type(b) is TransformerBlock for b in m.blocks)
        assert m.blocks[0]._native_block.mode == "persistent"
    assert all(type(b) is RefLikeBlock for b in m.blocks)


def test_parameter_order_and_eps():
    blk = TransformerBlock(256, 512, 2, cross_attn_norm=True, eps=1e-6)
    w = block_parameters(blk)
    assert len(w) == 27
    assert w[0] is not None and w[0].shape == (1, 6, 256)
    assert w[1].shape == (256,) and w[23].shape == (512, 256) and w[25].shape == (256, 512)
    assert w[3].data_ptr() == blk.attn1.to_q.weight.data_ptr()
    assert w[21].data_ptr() == blk.attn2.norm_q.weight.data_ptr()
    assert not any(t.requires_grad for t in w)
    assert blk.attn1.to_q.weight.requires_grad  # aliases, flags untouched
    assert block_eps(blk) == [1e-6] * 7
    blk2 = TransformerBlock(256, 512, 2, cross_attn_norm=False)
    w2 = block_parameters(blk2)
    assert w2[1].numel() == 0 and w2[2].numel() == 0


def test_native_block_guards():
    blk = TransformerBlock(256, 512, 2, cross_attn_norm=True)
    nb = NativeBlock(blk)
    x = torch.zeros(1, 4, 256, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="inference-only"):
        nb(x, x, torch.zeros(1, 1, 6, 256), None)
    with torch.no_grad():
        with pytest.raises(RuntimeError, match="GPU"):
            nb(x, x, torch.zeros(1, 1, 6, 256), None)
    with pytest.raises(ValueError):
        NativeBlock(blk, mode="graph")


def test_state_dict_keys_match_reference_layout():
    keys = set(TransformerBlock(256, 512, 2, cross_attn_norm=True).state_dict())
    for k in ("scale_shift_table", "norm2.weight", "norm2.bias", "attn1.to_out.0.weight",
              "attn2.norm_k.weight", "ffn.net.0.proj.weight", "ffn.net.2.bias"):
        assert k in keys


def test_prepare_context_groups_identical_rows():
    blk = TransformerBlock(256, 512, 2, cross_attn_norm=True)
    wl = WholeLayerBlock(blk)
    ctx = torch.randn(4, 8, 256).bfloat16()
    ctx[2] = ctx[0]
    wl.prepare_context(ctx, precompute=False)
    assert wl.context_rows.tolist() == [0, 1, 0, 2]
    assert wl.context_roots.tolist() == [0, 1, 3]
    wl.prepare_context(ctx[:2].clone(), precompute=False)
    assert wl.context_rows is None


def test_block_stack_contract_on_host():
    """The verify stack refuses a writing update with candidate rows and a
    missing read-only cache before any native call (model.py:1056-1057, :628-629)."""
    from wam_ops import BlockStack
    blocks = [TransformerBlock(64, 128, 2, cross_attn_norm=True) for _ in range(2)]
    stack = BlockStack(blocks)
    assert len(stack) == 2
    x = torch.zeros(2, 4, 64, dtype=torch.bfloat16)
    rows = torch.zeros(2, dtype=torch.int64)
    with torch.no_grad():
        with pytest.raises(ValueError, match="update_cache=0"):
            stack(x, x, None, None, update_cache=1, candidate_cache_rows=rows)
        with pytest.raises(ValueError, match="read-only KV"):
            stack(x, x, None, None, candidate_cache_rows=rows)
    with pytest.raises(ValueError):
        BlockStack([])


def test_candidate_rows_validation_reuse():
    """The rows check (model.py:639-647) reads the rows back once per tensor;
    the same unmodified tensor passes again without a read, and any in-place
    write, another tensor, or another pool size is checked afresh."""
    from wam_ops.native import validate_candidate_rows
    dev = torch.device("cpu")
    rows = torch.tensor([0, 1, 1, 0], dtype=torch.long)
    validate_candidate_rows(rows, 4, 2, dev)
    validate_candidate_rows(rows, 4, 2, dev)          # cached
    rows[2] = 2                                       # in-place write: out of range now
    with pytest.raises(ValueError, match="candidate_cache_rows"):
        validate_candidate_rows(rows, 4, 2, dev)
    validate_candidate_rows(rows, 4, 3, dev)          # a larger pool admits it
    with pytest.raises(ValueError, match="candidate_cache_rows"):
        validate_candidate_rows(rows, 4, 2, dev)      # the cache is keyed by pool size
    bad = torch.tensor([0, -1, 0, 0], dtype=torch.long)
    with pytest.raises(ValueError, match="candidate_cache_rows"):
        validate_candidate_rows(bad, 4, 2, dev)
    with pytest.raises(ValueError, match="candidate_cache_rows"):
        validate_candidate_rows(rows, 3, 3, dev)      # wrong batch
