"""nv4: MI355X-native quantized linears of Nano-vLLM-INT4.

The W4A4 path (RHT + group-128 INT4 activation quantization, grouped INT4 GEMM)
and the W4A16 GPTQ path, as hand-written gfx950 HIP kernels in libnv4.so behind
the reference's Python operator and module interfaces.
"""
from . import _lib
from .kernels import (Config, GroupedConfig, best_config, best_grouped_config, compile_grouped_gemm,
                      compile_kernel, dequant_matmul_w4a16, rht_quant_pack, tile_weights,
                      untile_weights, w4a4_grouped_gemm, w4a4_linear, weights_to_f6)
from .layers import W4A4Linear, W4A16Linear

__version__ = "0.1.0"

__all__ = ["Config", "GroupedConfig", "best_config", "best_grouped_config", "compile_grouped_gemm",
           "compile_kernel", "dequant_matmul_w4a16", "rht_quant_pack", "w4a4_grouped_gemm",
           "w4a4_linear", "tile_weights", "untile_weights", "weights_to_f6",
           "W4A4Linear", "W4A16Linear"]
