"""MI355X kernels of the quantized-linear path (HIP, via libnv4.so)."""
from .rht_a4 import Config, best_config, compile_kernel, rht_quant_pack
from .w4a4_grouped import (GroupedConfig, best_grouped_config, compile_grouped_gemm, tile_weights, untile_weights,
                           w4a4_grouped_gemm, weights_to_f6)
from .w4a16 import dequant_matmul_w4a16, dequant_w4a16
from .w4a4_linear import w4a4_linear

__all__ = ["Config", "best_config", "compile_kernel", "rht_quant_pack", "GroupedConfig",
           "best_grouped_config", "compile_grouped_gemm", "w4a4_grouped_gemm", "dequant_matmul_w4a16", "dequant_w4a16",
           "w4a4_linear", "tile_weights", "untile_weights", "weights_to_f6"]
