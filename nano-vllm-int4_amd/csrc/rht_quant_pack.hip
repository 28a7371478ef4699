// K1: fused randomized Hadamard transform + group-128 INT4 quantization +
// nibble packing, for gfx950.  The reference-layout row transform lives in
// k1_row.h (shared with the fused decode linear kernel); this file holds the
// standalone kernels and the C ABI entry point.
#include "k1_row.h"

namespace nv4 {
namespace {

// One workgroup of T threads per row.
template <int C, int F, int T>
__global__ void __launch_bounds__(T)
k1_reference(const uint16_t* __restrict__ x, const int8_t* __restrict__ signs,
             int8_t* __restrict__ packed, uint16_t* __restrict__ scale) {
    using S = Shape<C, F, T>;
    __shared__ float buf[S::LDS];
    const int64_t row = blockIdx.x;
    k1_row<C, F, T>(x + row * S::K, signs, packed + row * (S::K / 2), scale + row * (S::K / 128), buf,
                    threadIdx.x, true);
}

// block128 layout: every aligned 128-block gets its own 128-point Sylvester
// transform, then x RN(1/sqrt 128).  Each thread owns 16 contiguous values
// (butterfly bits 0-3 in registers); bits 4-6 are lanes xor 1, 2, 4.
__global__ void __launch_bounds__(256)
k1_block128(const uint16_t* __restrict__ x, const int8_t* __restrict__ signs,
            int8_t* __restrict__ packed, uint16_t* __restrict__ scale, int64_t units, int K) {
    const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
    // Out-of-range lanes recompute unit 0 so every shuffle partner exists;
    // their results are never stored.
    const bool live = u < units;
    const int64_t uu = live ? u : 0;
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
    // Every lane runs the shuffles; only live lanes store.
    quantize16_store(a, packed + uu * 8, scale + (uu >> 3), (lane & 7) == 0, live);
}

template <int C, int F, int T>
hipError_t launch_reference(const void* x, const int8_t* signs, int8_t* packed, void* scale,
                            int64_t M, hipStream_t stream) {
    hipLaunchKernelGGL((k1_reference<C, F, T>), dim3((unsigned)M), dim3(T), 0, stream,
                       static_cast<const uint16_t*>(x), signs, packed, static_cast<uint16_t*>(scale));
    return hipGetLastError();
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
        if (K == 4096) return (int)launch_reference<1, 4096, 256>(x, signs, packed, scale, M, st);
        if (K == 12288) return (int)launch_reference<12, 1024, 256>(x, signs, packed, scale, M, st);
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
