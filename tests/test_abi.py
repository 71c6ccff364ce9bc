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
    assert "multiple of 128" in _err(h.wam_linear(ctypes.byref(a), None))
    a.seg_n, a.n_seg = 128, 4
    assert "n_seg" in _err(h.wam_linear(ctypes.byref(a), None))
    a.n_seg, a.epilogue = 1, _lib.EPI_BIAS_GATE_RES
    assert "residual" in _err(h.wam_linear(ctypes.byref(a), None))


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


def test_workspace_size():
    h = _lib.lib()
    R, D, F, Lc = 4680, 3072, 14336, 512
    n = h.wam_block_workspace_bytes(1, R, D, F, 1, Lc, 0)
    expect = (R * D * 2 + R * 3 * D * 2 + R * D * 2 + 2 * R * D * 4 + 2 * Lc * D * 2 + R * F * 2
              + R * 4)  # new-slot list
    assert expect <= n < expect + 4096
