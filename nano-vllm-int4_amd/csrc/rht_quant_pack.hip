// K1: fused randomized Hadamard transform + group-128 INT4 quantization +
// nibble packing, for gfx950.  The reference-layout row transforms live in
// k1_row.h; this file holds the kernels and the C ABI entry points,
// including K1 with the producer of its input fused in front (add+RMSNorm
// for the qkv and gate_up inputs, SiLU-mul for the down input): the row is
// computed, rounded to bf16 as the separate op would store it, and fed to the
// transform without the round trip through memory.
#include "k1_row.h"
#include "norm_ops.h"

namespace nv4 {
namespace {

// K = 12288: one workgroup of 1024 threads per row.
__global__ void __launch_bounds__(K12_THREADS)
k1_k12288(const uint16_t* __restrict__ x, const int8_t* __restrict__ signs,
          int8_t* __restrict__ packed, uint16_t* __restrict__ scale) {
    __shared__ float buf[K12_LDS];
    const int64_t row = blockIdx.x;
    const uint16_t* xr = x + row * 12288;
    k1_row12288([&](int c0, float (&v)[16]) { load_bf16x16(xr + c0, v); }, signs, packed + row * 6144,
                scale + row * 96, buf);
}

// K = 4096: one workgroup of 256 threads per row.
__global__ void __launch_bounds__(256)
k1_k4096(const uint16_t* __restrict__ x, const int8_t* __restrict__ signs,
         int8_t* __restrict__ packed, uint16_t* __restrict__ scale) {
    __shared__ float buf[K4_LDS];
    const int64_t row = blockIdx.x;
    const uint16_t* xr = x + row * 4096;
    k1_row4096([&](int c0, float (&v)[16]) { load_bf16x16(xr + c0, v); }, signs, packed + row * 2048,
               scale + row * 32, buf);
}

// K = 4096 behind add+RMSNorm (same bits as nv4_rmsnorm followed by K1):
// thread t's prologue unit is columns 16t..16t+15, the unit nv4_rmsnorm's
// thread t owns for a 4096-wide row.
template <bool RESID>
__global__ void __launch_bounds__(256)
k1_k4096_rmsnorm(const uint16_t* x, const uint16_t* res_in, uint16_t* res_out, const uint16_t* __restrict__ nw,
                 float eps, const int8_t* __restrict__ signs, int8_t* __restrict__ packed,
                 uint16_t* __restrict__ scale) {
    __shared__ float buf[K4_LDS];
    __shared__ float red[4];
    const int64_t off = (int64_t)blockIdx.x * 4096;
    k1_row4096(
        [&](int c0, float (&v)[16]) {
            // The norm weights are loaded ahead of the row (one round trip).
            const v4u w0 = *reinterpret_cast<const v4u*>(nw + c0);
            const v4u w1 = *reinterpret_cast<const v4u*>(nw + c0 + 8);
            float h[16], ss = 0.0f;
            rms_load16<RESID>(x + off + c0, RESID ? res_in + off + c0 : nullptr,
                              RESID ? res_out + off + c0 : nullptr, h, ss);
            const float r = rms_rsqrt256(ss, red, 4096, eps);
            rms_apply16(h, r, w0, w1, v);
        },
        signs, packed + (int64_t)blockIdx.x * 2048, scale + (int64_t)blockIdx.x * 32, buf);
}

// K1 behind SiLU-and-mul of a [M, 2K] gate/up row (same bits as nv4_silu_mul
// followed by K1).
__global__ void __launch_bounds__(256)
k1_k4096_silu(const uint16_t* __restrict__ gu, const int8_t* __restrict__ signs, int8_t* __restrict__ packed,
              uint16_t* __restrict__ scale) {
    __shared__ float buf[K4_LDS];
    const uint16_t* g = gu + (int64_t)blockIdx.x * 8192;
    k1_row4096([&](int c0, float (&v)[16]) { silu_mul16(g + c0, g + 4096 + c0, v); }, signs,
               packed + (int64_t)blockIdx.x * 2048, scale + (int64_t)blockIdx.x * 32, buf);
}

__global__ void __launch_bounds__(K12_THREADS)
k1_k12288_silu(const uint16_t* __restrict__ gu, const int8_t* __restrict__ signs, int8_t* __restrict__ packed,
               uint16_t* __restrict__ scale) {
    __shared__ float buf[K12_LDS];
    const uint16_t* g = gu + (int64_t)blockIdx.x * 24576;
    k1_row12288([&](int c0, float (&v)[16]) { silu_mul16(g + c0, g + 12288 + c0, v); }, signs,
                packed + (int64_t)blockIdx.x * 6144, scale + (int64_t)blockIdx.x * 96, buf);
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

extern "C" int nv4_rmsnorm_rht_quant_pack(const void* x, const void* residual_in, void* residual_out,
                                          const void* norm_weight, float eps, const int8_t* signs, int8_t* packed,
                                          void* scale, int64_t M, int64_t K, void* stream) {
    using namespace nv4;
    if (!x || !norm_weight || !signs || !packed || !scale || (!residual_in) != (!residual_out)) return NV4_E_NULL;
    if (M < 1 || M > 0x7fffffffLL || K != 4096) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(residual_in) % 16 ||
        reinterpret_cast<uintptr_t>(residual_out) % 16 || reinterpret_cast<uintptr_t>(norm_weight) % 16 ||
        reinterpret_cast<uintptr_t>(packed) % 8 || reinterpret_cast<uintptr_t>(scale) % 2 ||
        reinterpret_cast<uintptr_t>(signs) % 16)
        return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const auto* xp = static_cast<const uint16_t*>(x);
    const auto* wp = static_cast<const uint16_t*>(norm_weight);
    auto* sp = static_cast<uint16_t*>(scale);
    if (residual_in)
        hipLaunchKernelGGL(k1_k4096_rmsnorm<true>, dim3((unsigned)M), dim3(256), 0, st, xp,
                           static_cast<const uint16_t*>(residual_in), static_cast<uint16_t*>(residual_out), wp, eps,
                           signs, packed, sp);
    else
        hipLaunchKernelGGL(k1_k4096_rmsnorm<false>, dim3((unsigned)M), dim3(256), 0, st, xp, nullptr, nullptr, wp,
                           eps, signs, packed, sp);
    return (int)hipGetLastError();
}

extern "C" int nv4_silu_mul_rht_quant_pack(const void* gate_up, const int8_t* signs, int8_t* packed, void* scale,
                                           int64_t M, int64_t K, void* stream) {
    using namespace nv4;
    if (!gate_up || !signs || !packed || !scale) return NV4_E_NULL;
    if (M < 1 || M > 0x7fffffffLL || (K != 4096 && K != 12288)) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(gate_up) % 16 || reinterpret_cast<uintptr_t>(packed) % 8 ||
        reinterpret_cast<uintptr_t>(scale) % 2 || reinterpret_cast<uintptr_t>(signs) % 16)
        return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const auto* gp = static_cast<const uint16_t*>(gate_up);
    auto* sp = static_cast<uint16_t*>(scale);
    if (K == 4096)
        hipLaunchKernelGGL(k1_k4096_silu, dim3((unsigned)M), dim3(256), 0, st, gp, signs, packed, sp);
    else
        hipLaunchKernelGGL(k1_k12288_silu, dim3((unsigned)M), dim3(K12_THREADS), 0, st, gp, signs, packed, sp);
    return (int)hipGetLastError();
}
