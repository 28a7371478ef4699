// Shared device helpers for the nv4 HIP kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/nv4.h"

namespace nv4 {

typedef int v4i __attribute__((ext_vector_type(4)));
// Native 16-byte vector: copies are single loads/stores (HIP's uint4 is a
// struct whose copies become memcpy, which can pin an array in scratch).
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// Compute units of the current device (host side, cached per device): the
// launchers size their grids and choose kernel forms by it.
inline int device_cu_count() {
    static int cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
    if (dev < 64 && cache[dev] > 0) return cache[dev];
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    if (dev < 64) cache[dev] = v;
    return v;
}

constexpr int ilog2c(int v) { return v <= 1 ? 0 : 1 + ilog2c(v / 2); }

// Calls f(std::integral_constant<int, I>{}) for I = B .. E-1: indices into
// register arrays stay compile-time constants whatever the unroller decides.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 bits, round to nearest even, in integer arithmetic (NaN kept
// as a quiet NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_rne_int(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// fp32 -> bf16 bits, round to nearest even, by the hardware conversion
// (v_cvt_pk_bf16_f32, one instruction): the bits of f32_to_bf16_rne_int for
// every non-NaN input, denormals included (nv4_probe_bf16_rne checks all 2^32
// inputs on the device); a NaN gives a quiet NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// Two packed signed nibbles per byte, even k in the low nibble.  Returns the
// nibbles as int8 lanes scaled by 16 (the nibble in the high half of each
// byte): lo16 = low nibbles of the 4 bytes, hi16 = high nibbles.  Both
// operands of a product scaled this way give 256 * the true integer dot.
__device__ __forceinline__ uint32_t nib_lo16(uint32_t w) { return (w << 4) & 0xF0F0F0F0u; }
__device__ __forceinline__ uint32_t nib_hi16(uint32_t w) { return w & 0xF0F0F0F0u; }

// 8 packed bytes (16 nibbles) -> one 16-lane int8 MFMA operand, scaled by 16.
// Nibble order inside the operand: lo(b0..b3), hi(b0..b3), lo(b4..b7), hi(b4..b7).
// A and B operands built by the same function pair element for element, so
// the product sums exactly the same 16 k values on both sides.
__device__ __forceinline__ v4i unpack8_x16(uint32_t d0, uint32_t d1) {
    v4i r;
    r[0] = (int)nib_lo16(d0);
    r[1] = (int)nib_hi16(d0);
    r[2] = (int)nib_lo16(d1);
    r[3] = (int)nib_hi16(d1);
    return r;
}

}  // namespace nv4
