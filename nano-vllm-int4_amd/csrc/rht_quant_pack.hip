// K1: fused randomized Hadamard transform + group-128 INT4 quantization +
// nibble packing, for gfx950.  The reference-layout row transforms live in
// k1_row.h; this file holds the kernels and the C ABI entry point.
#include "k1_row.h"

namespace nv4 {
namespace {

// K = 12288: one workgroup of 1024 threads per row.
__global__ void __launch_bounds__(K12_THREADS)
k1_k12288(const uint16_t* __restrict__ x, const int8_t* __restrict__ signs,
          int8_t* __restrict__ packed, uint16_t* __restrict__ scale) {
    __shared__ float buf[K12_LDS];
    const int64_t row = blockIdx.x;
    k1_row12288(x + row * 12288, signs, packed + row * 6144, scale + row * 96, buf);
}

// K = 4096: one workgroup of 256 threads per row.
__global__ void __launch_bounds__(256)
k1_k4096(const uint16_t* __restrict__ x, const int8_t* __restrict__ signs,
         int8_t* __restrict__ packed, uint16_t* __restrict__ scale) {
    __shared__ float buf[K4_LDS];
    const int64_t row = blockIdx.x;
    k1_row4096(x + row * 4096, signs, packed + row * 2048, scale + row * 32, buf);
}

// block128 layout: every aligned 128-block gets its own 128-point Sylvester
// transform, then x RN(1/sqrt 128).  Each thread owns 16 contiguous values
// (butterfly bits 0-3 in registers); bits 4-6 are lanes xor 1, 2, 4.
__global__ void __launch_bounds__(256)
k1_block128(const uint16_t* __restrict__ x, const int8_t* __restrict__ signs,
            int8_t* __restrict__ packed, uint16_t* __restrict__ scale, int64_t units, int K) {
    const int64_t uu = (int64_t)blockIdx.x * 256 + threadIdx.x;
    // units is a multiple of 8, so the 8-lane groups that exchange values
    // below are either wholly in range or wholly out.
    if (uu >= units) return;
    const int kcol = (int)((uu * 16) % K);
    float a[16];
    {
        const uint4 xv = *reinterpret_cast<const uint4*>(x + uu * 16);
        const uint4 xv2 = *reinterpret_cast<const uint4*>(x + uu * 16 + 8);
        const uint4 sv = *reinterpret_cast<const uint4*>(signs + kcol);
        const uint32_t xw[8] = {xv.x, xv.y, xv.z, xv.w, xv2.x, xv2.y, xv2.z, xv2.w};
        const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t h = (xw[i >> 1] >> (16 * (i & 1))) & 0xffffu;
            const int sg = (int)(int8_t)((sw[i >> 2] >> (8 * (i & 3))) & 0xffu);
            a[i] = bf16_to_f32(h) * (float)sg;
        }
    }
#pragma unroll
    for (int rb = 1; rb < 16; rb <<= 1)
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if ((r & rb) == 0) {
                const float lo = a[r], hi = a[r + rb];
                a[r] = lo + hi;
                a[r + rb] = lo - hi;
            }
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int lb = 1; lb < 8; lb <<= 1) {
        const bool upper = (lane & lb) != 0;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float other = __shfl_xor(a[r], lb);
            a[r] = upper ? (other - a[r]) : (a[r] + other);
        }
    }
    const float norm = 0x1.6a09e6p-4f;  // RN(1/sqrt 128)
#pragma unroll
    for (int i = 0; i < 16; ++i) a[i] = a[i] * norm;
    quantize16_store(a, packed + uu * 8, scale + (uu >> 3), (lane & 7) == 0);
}

}  // namespace
}  // namespace nv4

extern "C" int nv4_rht_quant_pack(const void* x, const int8_t* signs, int8_t* packed, void* scale,
                                  int64_t M, int64_t K, int layout, void* stream) {
    using namespace nv4;
    if (!x || !signs || !packed || !scale) return NV4_E_NULL;
    if (M < 1 || M > 0x7fffffffLL) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(packed) % 8 ||
        reinterpret_cast<uintptr_t>(scale) % 2 || reinterpret_cast<uintptr_t>(signs) % 16)
        return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (layout == NV4_LAYOUT_REFERENCE) {
        const auto* xp = static_cast<const uint16_t*>(x);
        auto* sp = static_cast<uint16_t*>(scale);
        if (K == 4096) {
            hipLaunchKernelGGL(k1_k4096, dim3((unsigned)M), dim3(256), 0, st, xp, signs, packed, sp);
            return (int)hipGetLastError();
        }
        if (K == 12288) {
            hipLaunchKernelGGL(k1_k12288, dim3((unsigned)M), dim3(K12_THREADS), 0, st, xp, signs, packed, sp);
            return (int)hipGetLastError();
        }
        return NV4_E_SHAPE;
    }
    if (layout == NV4_LAYOUT_BLOCK128) {
        if (K < 128 || K % 128 || K > 65536) return NV4_E_SHAPE;
        const int64_t units = M * (K / 16);
        const int64_t blocks = (units + 255) / 256;
        if (blocks > 0x7fffffffLL) return NV4_E_SHAPE;
        hipLaunchKernelGGL(k1_block128, dim3((unsigned)blocks), dim3(256), 0, st,
                           static_cast<const uint16_t*>(x), signs, packed, static_cast<uint16_t*>(scale),
                           units, (int)K);
        return (int)hipGetLastError();
    }
    return NV4_E_LAYOUT;
}
