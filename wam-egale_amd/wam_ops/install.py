"""Swap a live block's classes to the native ones for the duration of a context.

Same contract as 算子研究/wam_ops/install.py:6-61: only the given model instance
is touched; its parameters and caches are left as they are; the original
classes are restored on exit.  Refuses non-torch attention modes, existing
forward overrides and non-original cache modes.  Both implementation names of
the reference are accepted and run the same HIP kernels: "baseline" and
"optimized" differ only in the flags the reference exposed for its CUDA
experiments (execution_mode, fused_ffn1), which are validated and recorded.
"""
from contextlib import ExitStack, contextmanager

from .block import TransformerBlock
from .native import NativeBlock
from .parameters import Attention


@contextmanager
def install_block(block, implementation="baseline", *, execution_mode=None, fused_ffn1=None):
    if implementation not in ("baseline", "optimized"):
        raise ValueError("implementation must be baseline or optimized")
    if getattr(block, "attn_mode", "torch") != "torch":
        raise ValueError("the original torch model is required as the matching baseline")
    modules = (block, block.attn1, block.attn2)
    if any("forward" in module.__dict__ for module in modules):
        raise ValueError("the model carries an experimental forward override; refusing to mix")
    if any(getattr(attention, "cache_mode", "original") != "original" for attention in modules[1:]):
        raise ValueError("only the original KV protocol is supported")
    if implementation == "baseline" and (execution_mode is not None or fused_ffn1 is not None):
        raise ValueError("baseline is frozen; optimization flags are invalid")
    classes = tuple(type(module) for module in modules)
    previous_native = block.__dict__.get("_native_block")
    try:
        for module, kind in zip(modules, (TransformerBlock, Attention, Attention)):
            module.__class__ = kind
        native = NativeBlock(block,
                             fused_ffn1=bool(fused_ffn1) if fused_ffn1 is not None else False,
                             mode=execution_mode or "sequential")
        object.__setattr__(block, "_native_block", native)
        yield block
    finally:
        for module, kind in zip(modules, classes):
            module.__class__ = kind
        if previous_native is None:
            block.__dict__.pop("_native_block", None)
        else:
            object.__setattr__(block, "_native_block", previous_native)


@contextmanager
def install_model(model, implementation="baseline", **options):
    with ExitStack() as stack:
        for block in model.blocks:
            stack.enter_context(install_block(block, implementation, **options))
        yield model
