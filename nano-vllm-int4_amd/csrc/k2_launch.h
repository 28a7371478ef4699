// Internal launchers shared between the grouped INT4 GEMM translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nv4 {

// Prefill-sized grouped W4A4 GEMM (M > 64): LDS-staged 128x128 tiles,
// v_mfma_i32_32x32x32_i8.  Same arguments and numerical contract as
// nv4_w4a4_gemm; w is in the MFMA-tiled layout when w_tiled (N % 16 == 0);
// arguments are already validated.
hipError_t k2_prefill_launch(const int8_t* a, const int8_t* w, const void* sa, const void* sw,
                             bool sw_grouped, void* out, bool out_fp32, bool w_tiled, int M, int N, int K,
                             hipStream_t st);

}  // namespace nv4
