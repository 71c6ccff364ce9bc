"""ctypes binding of libwam_block.so (the C ABI declared in include/wam_block.h).

The structures below mirror the C structs field for field; ``check_abi()``
compares every ``sizeof`` with the library's own (``wam_abi_struct_size``).
There is no fallback: if the library is missing, every entry point raises.
"""
import ctypes
from ctypes import (POINTER, Structure, c_char_p, c_double, c_float, c_int, c_int32, c_int64,
                    c_size_t, c_uint32, c_void_p)
from functools import lru_cache
from pathlib import Path

LIB_NAME = "libwam_block.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

WAM_OK, WAM_ERR_ARG, WAM_ERR_HIP, WAM_ERR_STATE = 0, -1, -2, -3
WAM_BF16, WAM_F32, WAM_FP8, WAM_I64, WAM_F64, WAM_FP8_MX = 0, 1, 2, 3, 4, 5
WAM_ACT_NONE, WAM_ACT_SILU = 0, 1
EPI_BIAS, EPI_BIAS_GELU, EPI_BIAS_GATE_RES, EPI_BIAS_RES = 0, 1, 2, 3
PEAK_BF16_32, PEAK_BF16_16, PEAK_FP8_32, PEAK_FP8_16 = 0, 1, 2, 3
DEBUG_SLOTS = 28
STAGES = ("ln1", "qkv", "rms_rope", "kv_layout", "self_attn", "self_out", "ln2",
          "cross_q", "cross_kv", "cross_attn", "cross_out", "ln3", "ffn1", "ffn2",
          "kv_commit")
DEBUG_NAMES = ("modulated1", "self_q_rope", "self_k_rope", "self_v", "self_attention",
               "residual1", "norm2", "cross_q", "cross_k", "cross_v", "cross_attention",
               "residual2", "modulated3", "gelu", "output",
               "self_q_linear", "self_k_linear", "self_q_norm", "self_k_norm", "self_out",
               "cross_q_linear", "cross_k_linear", "cross_out", "ffn1", "ffn2", "norm1", "norm3",
               "modulation")


class Modulation(Structure):
    _fields_ = [("table", c_void_p), ("table_dtype", c_int), ("temb", c_void_p),
                ("temb_dtype", c_int), ("temb_len", c_int), ("tokens", c_int),
                ("temb_mods", c_int)]


class LinearArgs(Structure):
    _fields_ = [("a", c_void_p), ("lda", c_int64), ("M", c_int), ("K", c_int),
                ("n_seg", c_int), ("seg_n", c_int), ("w", c_void_p * 3), ("ldw", c_int64),
                ("bias", c_void_p * 3), ("out", c_void_p * 3), ("ldo", c_int64),
                ("epilogue", c_int), ("res", c_void_p), ("ldr", c_int64),
                ("res_dtype", c_int), ("out_dtype", c_int),
                ("gate", Modulation), ("gate_index", c_int),
                ("w_dtype", c_int), ("w_scale", c_void_p * 3),
                ("workspace", c_void_p), ("workspace_bytes", c_int64),
                ("norm_ssq", c_void_p * 3), ("norm_gamma", c_void_p * 3), ("norm_freq", c_void_p),
                ("norm_freq_batch", c_int), ("norm_tokens", c_int), ("norm_head_dim", c_int),
                ("a_dtype", c_int), ("a_scale", c_void_p), ("a_block_scale", c_void_p),
                ("out_block_scale", c_void_p)]


class LnArgs(Structure):
    _fields_ = [("x", c_void_p), ("y", c_void_p), ("rows", c_int), ("D", c_int),
                ("x_dtype", c_int), ("eps", c_float), ("affine", c_int), ("gamma", c_void_p),
                ("beta", c_void_p), ("gb_dtype", c_int), ("mod", Modulation), ("shift_index", c_int),
                ("y8", c_void_p), ("y8_scale", c_void_p)]


class RmsRopeArgs(Structure):
    _fields_ = [("x", c_void_p * 2), ("y", c_void_p * 2), ("gamma", c_void_p * 2),
                ("eps", c_float * 2), ("ldx", c_int64), ("ldy", c_int64),
                ("n_tensors", c_int), ("rows", c_int), ("D", c_int), ("head_dim", c_int),
                ("freq", c_void_p), ("freq_batch", c_int), ("tokens", c_int)]


class AttentionArgs(Structure):
    _fields_ = [("q", c_void_p), ("q_bstride", c_int64), ("q_rstride", c_int64),
                ("o", c_void_p), ("o_bstride", c_int64), ("o_rstride", c_int64),
                ("B", c_int), ("Mq", c_int), ("H", c_int), ("head_dim", c_int),
                ("pool_k", c_void_p), ("pool_v", c_void_p), ("pool_bstride", c_int64),
                ("pool_rstride", c_int64), ("pool_batch", c_int), ("slots", c_void_p),
                ("n_hist_dev", c_void_p), ("pool_rows", c_void_p), ("k", c_void_p),
                ("v", c_void_p), ("kv_bstride", c_int64), ("kv_rstride", c_int64),
                ("Mk", c_int), ("kv_rows", c_void_p), ("kv_batch", c_int), ("scale", c_float),
                ("workspace", c_void_p), ("workspace_bytes", c_int64), ("max_keys", c_int),
                ("q_ssq", c_void_p), ("q_ssq_n", c_int), ("q_norm_dim", c_int), ("q_eps", c_float),
                ("hist_base_dev", c_void_p)]


class KvLayoutArgs(Structure):
    _fields_ = [("mask", c_void_p), ("ids", c_void_p), ("is_pred", c_void_p), ("pool", c_int),
                ("tokens", c_int), ("update", c_int), ("candidate", c_int), ("rows", c_void_p),
                ("batch", c_int), ("pool_batch", c_int), ("hist_slots", c_void_p),
                ("new_slots", c_void_p), ("info", c_void_p)]


class KvCommitArgs(Structure):
    _fields_ = [("k", c_void_p), ("v", c_void_p), ("ld", c_int64), ("pool_k", c_void_p),
                ("pool_v", c_void_p), ("pool_bstride", c_int64), ("pool_rstride", c_int64),
                ("new_slots", c_void_p), ("B", c_int), ("tokens", c_int), ("D", c_int)]


class BlockWeights(Structure):
    _fields_ = [("w", c_void_p * 27), ("table_dtype", c_int), ("norm2_dtype", c_int),
                ("dim", c_int), ("heads", c_int), ("head_dim", c_int), ("ffn_dim", c_int),
                ("eps", c_float * 7), ("ffn_fp8", c_void_p * 2), ("ffn_scale", c_void_p * 2),
                ("ffn_act_fp8", c_int)]


class BlockArgs(Structure):
    _fields_ = [("weights", POINTER(BlockWeights)), ("B", c_int), ("M", c_int),
                ("x", c_void_p), ("context", c_void_p), ("context_batch", c_int),
                ("context_len", c_int), ("context_rows", c_void_p), ("mod", Modulation),
                ("freq", c_void_p), ("freq_batch", c_int), ("cache_k", c_void_p),
                ("cache_v", c_void_p), ("cache_id", c_void_p), ("cache_mask", c_void_p),
                ("cache_is_pred", c_void_p), ("cache_batch", c_int), ("pool", c_int),
                ("candidate_rows", c_void_p), ("update", c_int), ("cross_k", c_void_p),
                ("cross_v", c_void_p), ("out", c_void_p), ("workspace", c_void_p),
                ("workspace_bytes", c_size_t), ("debug", c_void_p), ("timer", c_void_p),
                ("out_dtype", c_int)]


class PatchifyArgs(Structure):
    _fields_ = [("x", c_void_p), ("out", c_void_p), ("B", c_int), ("C", c_int), ("F", c_int),
                ("H", c_int), ("W", c_int), ("p1", c_int), ("p2", c_int), ("p3", c_int),
                ("k_pad", c_int)]


class TimestepArgs(Structure):
    _fields_ = [("t", c_void_p), ("rows", c_int), ("dim", c_int), ("flip_sin_to_cos", c_int),
                ("shift", c_float), ("max_period", c_float), ("out", c_void_p), ("out_dtype", c_int)]


class RowsLinearArgs(Structure):
    _fields_ = [("x", c_void_p), ("x_dtype", c_int), ("ldx", c_int64), ("w", c_void_p),
                ("w_dtype", c_int), ("ldw", c_int64), ("bias", c_void_p), ("bias_dtype", c_int),
                ("out", c_void_p), ("out_dtype", c_int), ("ldo", c_int64), ("R", c_int), ("N", c_int),
                ("K", c_int), ("act_in", c_int), ("act_out", c_int)]


class RopeFreqArgs(Structure):
    _fields_ = [("grid", c_void_p), ("grid_dtype", c_int), ("grid_bstride", c_int64),
                ("grid_rstride", c_int64), ("grid_lstride", c_int64), ("B", c_int), ("L", c_int),
                ("head_dim", c_int), ("theta", c_double), ("out", c_void_p)]


STRUCTS = {
    "wam_modulation": Modulation, "wam_linear_args": LinearArgs, "wam_ln_args": LnArgs,
    "wam_rms_rope_args": RmsRopeArgs, "wam_attention_args": AttentionArgs,
    "wam_kv_layout_args": KvLayoutArgs, "wam_kv_commit_args": KvCommitArgs,
    "wam_block_weights": BlockWeights, "wam_block_args": BlockArgs,
    "wam_patchify_args": PatchifyArgs, "wam_timestep_args": TimestepArgs,
    "wam_rows_linear_args": RowsLinearArgs, "wam_rope_freq_args": RopeFreqArgs,
}

# Every symbol include/wam_block.h declares, with its ctypes signature.
SIGNATURES = {
    "wam_linear": (c_int, [POINTER(LinearArgs), c_void_p]),
    "wam_attention_workspace_bytes": (c_int64, [c_int, c_int, c_int, c_int]),
    "wam_linear_workspace_bytes": (c_int64, [c_int, c_int, c_int, c_int]),
    "wam_quantize_fp8_rows": (c_int, [c_void_p, c_int, c_int, c_int64, c_void_p, c_void_p, c_void_p]),
    "wam_ln_modulate": (c_int, [POINTER(LnArgs), c_void_p]),
    "wam_rms_rope": (c_int, [POINTER(RmsRopeArgs), c_void_p]),
    "wam_attention": (c_int, [POINTER(AttentionArgs), c_void_p]),
    "wam_attention_noalloc": (c_int, [POINTER(AttentionArgs), c_void_p]),
    "wam_kv_layout": (c_int, [POINTER(KvLayoutArgs), c_void_p]),
    "wam_kv_commit": (c_int, [POINTER(KvCommitArgs), c_void_p]),
    "wam_block_workspace_bytes": (c_size_t, [c_int] * 7),
    "wam_block_forward": (c_int, [POINTER(BlockArgs), c_void_p]),
    "wam_prepare_context": (c_int, [POINTER(BlockWeights), c_void_p, c_int, c_void_p, c_void_p,
                                    c_void_p]),
    "wam_patchify": (c_int, [POINTER(PatchifyArgs), c_void_p]),
    "wam_timestep_embedding": (c_int, [POINTER(TimestepArgs), c_void_p]),
    "wam_rows_linear": (c_int, [POINTER(RowsLinearArgs), c_void_p]),
    "wam_rope_freqs": (c_int, [POINTER(RopeFreqArgs), c_void_p]),
    "wam_mfma_peak": (c_int, [c_int, c_int, c_void_p, c_int64, POINTER(c_double), c_void_p]),
    "wam_timer_create": (c_void_p, [c_int, c_uint32]),
    "wam_timer_reset": (None, [c_void_p]),
    "wam_timer_read": (c_int, [c_void_p, POINTER(c_int32), POINTER(c_float), c_int]),
    "wam_timer_destroy": (None, [c_void_p]),
    "wam_last_error": (c_char_p, []),
    "wam_abi_version": (c_int, []),
    "wam_abi_struct_size": (c_size_t, [c_char_p]),
}
ABI_VERSION = 1


class NativeLibraryMissing(RuntimeError):
    pass


@lru_cache(None)
def lib():
    """Load the in-tree HIP library; raise if it has not been built."""
    path = LIB_PATH
    if not path.exists():
        raise NativeLibraryMissing(
            f"{path} is missing: build the HIP library first (python -c "
            "'import __graft_entry__ as g; g.build()' at the repository root)")
    handle = ctypes.CDLL(str(path))
    for name, (res, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = argtypes
    if handle.wam_abi_version() != ABI_VERSION:
        raise RuntimeError(f"libwam_block ABI {handle.wam_abi_version()} != {ABI_VERSION}")
    return handle


def check_abi():
    """Return {struct: (python size, library size)} for every mismatching struct."""
    h = lib()
    bad = {}
    for name, cls in STRUCTS.items():
        n = h.wam_abi_struct_size(name.encode())
        if n != ctypes.sizeof(cls):
            bad[name] = (ctypes.sizeof(cls), n)
    return bad


def check(rc, what):
    if rc != WAM_OK:
        msg = lib().wam_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {msg} (code {rc})")
