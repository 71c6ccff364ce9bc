"""MI355X-native Wan DiT block operators (HIP kernels behind a C ABI).

Public surface mirrors the reference's wam_ops package:
install_block / install_model, NativeBlock, WholeLayerBlock, the
TransformerBlock / Attention parameter containers, and per-stage operators in
``wam_ops.ops``.
"""
from .install import install_block, install_model
from .native import NativeBlock
from .whole_layer import WholeLayerBlock
from .verify import BlockStack
from .block import TransformerBlock
from .parameters import Attention
from .model import TransformerModel, WholeModel

__all__ = ["install_block", "install_model", "NativeBlock", "WholeLayerBlock", "BlockStack",
           "TransformerBlock", "Attention", "TransformerModel", "WholeModel"]
