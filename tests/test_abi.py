"""The C-ABI library: loads, exports every symbol include/wam_block.h declares,
agrees with the ctypes struct layouts, and rejects contract violations on the
host before launching anything (these calls never reach the GPU)."""
import ctypes
import re
from pathlib import Path

import pytest

from wam_ops import _lib

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "wam_block.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(wam_[a-z_0-9]+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    h = _lib.lib()
    declared = declared_symbols()
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)
    for name in declared:
        assert hasattr(h, name), name
    assert h.wam_abi_version() == _lib.ABI_VERSION


def test_struct_layouts_match():
    assert _lib.check_abi() == {}


def _err(rc):
    assert rc == _lib.WAM_ERR_ARG
    return _lib.lib().wam_last_error().decode()


def test_linear_host_validation():
    h = _lib.lib()
    a = _lib.LinearArgs()
    a.a, a.lda, a.M, a.K, a.n_seg, a.seg_n, a.ldw, a.ldo = 16, 100, 8, 100, 1, 128, 100, 128
    a.w[0], a.out[0] = 16, 16
    assert "multiple of 64" in _err(h.wam_linear(ctypes.byref(a), None))
    a.K = a.lda = a.ldw = 128
    a.seg_n = 100
    assert "multiple of 8" in _err(h.wam_linear(ctypes.byref(a), None))
    a.seg_n, a.n_seg = 192, 2  # a partial last tile is fine for one segment only
    assert "of 128 with several segments" in _err(h.wam_linear(ctypes.byref(a), None))
    a.seg_n, a.n_seg = 128, 4
    assert "n_seg" in _err(h.wam_linear(ctypes.byref(a), None))
    a.n_seg, a.epilogue = 1, _lib.EPI_BIAS_GATE_RES
    assert "residual" in _err(h.wam_linear(ctypes.byref(a), None))
    # the epilogue addresses rows of one tile in 32 bits: strides of 2^21
    # elements (8 MiB fp32 rows) and more are refused
    a.epilogue, a.ldo = _lib.EPI_BIAS, 1 << 21
    assert "2^21" in _err(h.wam_linear(ctypes.byref(a), None))
    a.ldo, a.ldr = 128, 1 << 21
    assert "2^21" in _err(h.wam_linear(ctypes.byref(a), None))



def test_norm_epilogue_host_validation():
    """The q/k-norm epilogue of wam_linear and the query RMS factor of
    wam_attention reject bad arguments before any launch."""
    h = _lib.lib()
    a = _lib.LinearArgs()
    a.a, a.lda, a.M, a.K, a.n_seg, a.seg_n, a.ldw, a.ldo = 16, 128, 8, 128, 1, 128, 128, 128
    a.w[0], a.out[0] = 16, 16
    a.norm_ssq[0] = 16
    a.epilogue = _lib.EPI_BIAS_GELU
    assert "needs WAM_EPI_BIAS" in _err(h.wam_linear(ctypes.byref(a), None))
    a.epilogue = _lib.EPI_BIAS
    assert "needs a gamma" in _err(h.wam_linear(ctypes.byref(a), None))
    a.norm_gamma[0] = 16
    a.norm_ssq[1] = 16  # a segment that the launch does not have
    assert "norm segment 1" in _err(h.wam_linear(ctypes.byref(a), None))
    a.norm_ssq[1] = None
    a.norm_freq, a.norm_head_dim, a.norm_tokens, a.norm_freq_batch = 16, 96, 8, 1
    assert "head_dim 96" in _err(h.wam_linear(ctypes.byref(a), None))
    a.norm_head_dim, a.norm_tokens = 128, 3
    assert "freq batch" in _err(h.wam_linear(ctypes.byref(a), None))
    a.norm_tokens, a.norm_freq = 8, 24
    assert "16-byte aligned" in _err(h.wam_linear(ctypes.byref(a), None))
    t = _lib.AttentionArgs()
    t.B, t.Mq, t.H, t.head_dim, t.Mk, t.kv_batch = 1, 4, 1, 128, 4, 1
    t.q = t.o = t.k = t.v = 16
    t.q_ssq, t.q_ssq_n, t.q_norm_dim = 16, 17, 128
    assert "q_ssq needs 1..16 partials" in _err(h.wam_attention(ctypes.byref(t), None))
    t.q_ssq_n, t.q_norm_dim = 1, 0
    assert "q_norm_dim" in _err(h.wam_attention(ctypes.byref(t), None))

def test_attention_host_validation():
    h = _lib.lib()
    a = _lib.AttentionArgs()
    a.B, a.Mq, a.H, a.head_dim, a.Mk, a.kv_batch = 1, 4, 1, 64, 4, 1
    a.q = a.o = a.k = a.v = 16
    assert "head_dim must be 128" in _err(h.wam_attention(ctypes.byref(a), None))
    a.head_dim, a.Mk = 128, 0
    assert "bad shape" in _err(h.wam_attention(ctypes.byref(a), None))


def test_kv_layout_host_validation():
    h = _lib.lib()
    a = _lib.KvLayoutArgs()
    a.mask = a.ids = a.is_pred = a.hist_slots = a.info = a.new_slots = 16
    a.pool, a.tokens, a.update = 10, 11, 1
    assert "do not fit" in _err(h.wam_kv_layout(ctypes.byref(a), None))
    a.tokens, a.update = 5, 3
    assert "update must be" in _err(h.wam_kv_layout(ctypes.byref(a), None))
    a.update, a.candidate = 1, 1
    assert "needs rows" in _err(h.wam_kv_layout(ctypes.byref(a), None))


def test_block_host_validation():
    h = _lib.lib()
    w = _lib.BlockWeights()
    w.dim, w.heads, w.head_dim, w.ffn_dim = 256, 2, 128, 512
    args = _lib.BlockArgs()
    args.weights = ctypes.pointer(w)
    assert "scale_shift_table" in _err(h.wam_block_forward(ctypes.byref(args), None))
    for i in range(27):
        w.w[i] = 256 * (i + 1)
    w.dim = 300
    assert "must equal heads" in _err(h.wam_block_forward(ctypes.byref(args), None))
    w.dim, w.ffn_act_fp8 = 256, 1  # fp8 activations without the fp8 weights
    assert "fp8 FFN activations" in _err(h.wam_block_forward(ctypes.byref(args), None))
    w.ffn_fp8[0] = w.ffn_fp8[1] = w.ffn_scale[0] = w.ffn_scale[1] = 16
    w.ffn_dim = 384  # not whole 256-column tiles
    assert "ffn_dim % 256" in _err(h.wam_block_forward(ctypes.byref(args), None))


def test_workspace_size():
    h = _lib.lib()
    R, D, F, Lc = 4680, 3072, 14336, 512
    n = h.wam_block_workspace_bytes(1, R, D, F, 1, Lc, 0)
    expect = (R * D * 2 + R * 3 * D * 2 + R * D * 2 + 2 * R * D * 4 + 2 * Lc * D * 2 + R * F * 2
              + R * D + R * 4  # e4m3 copy of the LayerNorm-3 rows and their scales
              + R * 4  # new-slot list
              + R * (D // 256) * 4  # per-row query sums of squares per 256-column group
              + (1 + 2) * D * 4)  # zero modulation for the unmodulated LayerNorm debug outputs
    assert expect <= n < expect + 4096
    # 4680 queries over their own 4680 keys fill two dispatch rounds: no split
    assert h.wam_attention_workspace_bytes(1, R, 24, R) == 0


def test_linear_split_k_plan_workspace():
    h = _lib.lib()
    # 6240 x 14336 -> 3072 (FFN2 of 4 x 1560 rows): 250 whole 256x256 tiles,
    # the last 2 tile columns (50 tiles) in 5 k ranges of fp32 partials
    assert h.wam_linear_workspace_bytes(6240, 3072, 1, 14336) == 5 * 6240 * 512 * 4
    # 6240 x 3072 -> 14336 (FFN1): 1275 whole tiles, 125 tail tiles in 2 ranges
    assert h.wam_linear_workspace_bytes(6240, 14336, 1, 3072) == 2 * 6240 * 1280 * 4
    assert h.wam_linear_workspace_bytes(6240, 2816, 1, 3072) == 8 * 6240 * 256 * 4
    assert h.wam_linear_workspace_bytes(3900, 4352, 1, 4160) == 8 * 3900 * 256 * 4
    # short k (3072 -> 3072) keeps the 128x128 tail; 4680 rows leave no
    # partial round worth splitting; QKV (three segments) is never split
    assert h.wam_linear_workspace_bytes(6240, 3072, 1, 3072) == 0
    assert h.wam_linear_workspace_bytes(4680, 14336, 1, 3072) == 0
    assert h.wam_linear_workspace_bytes(4680, 3072, 1, 14336) == 0
    assert h.wam_linear_workspace_bytes(6240, 3072, 3, 3072) == 0


def test_attention_split_plan_workspace():
    h = _lib.lib()
    # 4 x 1560 queries over 1560 own + 7800 pool keys: 512 whole units, the
    # other 160 in 3 key ranges of fp32 partials (256 queries x (128 + 2)).
    assert h.wam_attention_workspace_bytes(4, 1560, 24, 1560 + 7800) == 3 * 160 * 256 * 130 * 4
    # one 1560-query chunk over 7800 keys: all 168 units in 3 ranges
    assert h.wam_attention_workspace_bytes(1, 1560, 24, 7800) == 3 * 168 * 256 * 130 * 4
    # short key lists are never split (cross attention over 512 text tokens)
    assert h.wam_attention_workspace_bytes(4, 1560, 24, 512) == 0
    # the block reserves one region for the largest of its split needs
    B, M, D, F, Lc, P = 4, 1560, 3072, 14336, 512, 7800
    R = B * M
    core = (R * D * 2 + R * D + R * 4  # LayerNorm rows, their e4m3 copy and its scales
            + R * 3 * D * 2 + R * D * 2 + 2 * R * D * 4 + 2 * Lc * D * 2 + R * F * 2
            + P * 4 + M * 4  # slot lists
            + R * (D // 256) * 4  # query sums of squares
            + (B + 2) * D * 4)  # zero modulation (debug LayerNorms)
    need = max(h.wam_attention_workspace_bytes(B, M, 24, M + P), h.wam_linear_workspace_bytes(R, D, 1, F),
               h.wam_linear_workspace_bytes(R, F, 1, D))
    assert need > 0
    n = h.wam_block_workspace_bytes(B, M, D, F, 1, Lc, P)
    assert core + need <= n < core + need + 4096


def test_modulation_host_validation():
    h = _lib.lib()
    a = _lib.LnArgs()
    a.x = a.y = 16
    a.rows, a.D, a.eps = 12, 256, 1e-6
    a.mod.table = a.mod.temb = 16
    a.mod.tokens, a.mod.temb_len = 6, 4  # 4 does not divide 6
    assert "divisor" in _err(h.wam_ln_modulate(ctypes.byref(a), None))
    a.mod.temb_len, a.mod.temb_mods = 3, 2
    assert "mods" in _err(h.wam_ln_modulate(ctypes.byref(a), None))
    a.mod.temb_mods, a.shift_index = 1, 3  # a one-vector temb goes with the [2, D] head table
    assert "shift index" in _err(h.wam_ln_modulate(ctypes.byref(a), None))
    a.mod.tokens = 5
    assert "divisible by tokens" in _err(h.wam_ln_modulate(ctypes.byref(a), None))
    a.mod.tokens, a.shift_index, a.y8 = 6, 0, 16  # e4m3 rows without their scales
    assert "y8_scale" in _err(h.wam_ln_modulate(ctypes.byref(a), None))


def test_model_io_host_validation():
    h = _lib.lib()
    p = _lib.PatchifyArgs()
    p.x = p.out = 16
    p.B, p.C, p.F, p.H, p.W, p.p1, p.p2, p.p3, p.k_pad = 1, 48, 2, 9, 10, 1, 2, 2, 192
    assert "multiples of the patch" in _err(h.wam_patchify(ctypes.byref(p), None))
    p.H, p.k_pad = 8, 100
    assert "k_pad" in _err(h.wam_patchify(ctypes.byref(p), None))
    t = _lib.TimestepArgs()
    t.t = t.out = 16
    t.rows, t.dim, t.max_period, t.out_dtype = 4, 256, 10000.0, 7
    assert "out dtype" in _err(h.wam_timestep_embedding(ctypes.byref(t), None))
    r = _lib.RowsLinearArgs()
    r.x = r.w = r.out = 16
    r.R, r.N, r.K, r.ldx, r.ldw, r.ldo = 8, 30, 64, 64, 64, 30
    r.w_dtype = _lib.WAM_FP8
    assert "dtypes" in _err(h.wam_rows_linear(ctypes.byref(r), None))
    r.w_dtype, r.ldw = _lib.WAM_BF16, 32
    assert "strides" in _err(h.wam_rows_linear(ctypes.byref(r), None))
    r.ldw, r.act_out = 64, 5
    assert "activation" in _err(h.wam_rows_linear(ctypes.byref(r), None))
    f = _lib.RopeFreqArgs()
    f.grid = f.out = 16
    f.grid_dtype, f.B, f.L, f.head_dim, f.theta = _lib.WAM_BF16, 1, 4, 128, 10000.0
    assert "grid dtype" in _err(h.wam_rope_freqs(ctypes.byref(f), None))
    f.grid_dtype, f.head_dim = _lib.WAM_I64, 130
    assert "whole f/h/w pairs" in _err(h.wam_rope_freqs(ctypes.byref(f), None))
