"""Drop-in quantized linear modules."""
from .linear_w4a4 import W4A4Linear
from .linear_w4a16 import W4A16Linear, fuse_w4a16, tl_dequant_matmul_w4a16

__all__ = ["W4A4Linear", "W4A16Linear", "fuse_w4a16", "tl_dequant_matmul_w4a16"]
