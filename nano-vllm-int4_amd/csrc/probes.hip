// Measurement probes: the sustained int8 / fp8 / fp6 matrix-core rate and the HBM
// streaming-read rate of the device they run on.  bench.py reports the
// published MI355X peaks as the roofline's `peak` and these measured figures
// beside them.  No counterpart in the reference.
#include "nv4_common.h"

namespace nv4 {
namespace {

typedef int v8i __attribute__((ext_vector_type(8)));

// Every wave runs `iters` (rounded up to even) rounds of four independent matrix-core products
// (no dependency between consecutive instructions of a round), so the
// matrix pipe of each SIMD stays busy.  The results are folded into one word
// per workgroup, stored only if it equals a value it practically never takes
// (keeps the products live without a store per launch).
template <int KIND>
__global__ void __launch_bounds__(256)
probe_mfma(int64_t iters, int* __restrict__ sink) {
    const int lane = threadIdx.x & 63;
    int acc_i = 0;
    float acc_f = 0.0f;
    if constexpr (KIND == 0) {
        const v4i a = {lane, lane + 1, lane + 2, lane + 3};
        const v4i b0 = {3 * lane, 5, 7, lane}, b1 = {lane, 9, 3, 1}, b2 = {2, lane, 11, 4}, b3 = {6, 8, lane, 13};
        v4i c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (int64_t i = 0; i < iters; i += 2) {  // two rounds per trip (iters is rounded up to even)
            c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b0, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b1, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b2, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b3, c3, 0, 0, 0);
            c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b1, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b2, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b3, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b0, c3, 0, 0, 0);
        }
        acc_i = c0[0] ^ c1[1] ^ c2[2] ^ c3[3];
    } else {
        // KIND 1: fp8 (e4m3) operands; KIND 2: fp6 (e3m2), six registers per operand.
        constexpr int F = KIND == 1 ? 0 : 3;
        const v8i a = {lane, 1, 2, 3, 4, 5, 6, 7};
        const v8i b0 = {7, lane, 5, 4, 3, 2, 1, 0}, b1 = {lane, 6, 5, 4, 3, 2, 1, 0}, b2 = {1, 2, lane, 4, 5, 6, 7, 8},
                  b3 = {9, 8, 7, lane, 5, 4, 3, 2};
        v16f c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (int64_t i = 0; i < iters; i += 2) {  // two rounds per trip (iters is rounded up to even)
            c0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b1, c0, F, F, 0, 127, 0, 127);
            c1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b2, c1, F, F, 0, 127, 0, 127);
            c2 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b3, c2, F, F, 0, 127, 0, 127);
            c3 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b0, c3, F, F, 0, 127, 0, 127);
            c0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b0, c0, F, F, 0, 127, 0, 127);
            c1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b1, c1, F, F, 0, 127, 0, 127);
            c2 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b2, c2, F, F, 0, 127, 0, 127);
            c3 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b3, c3, F, F, 0, 127, 0, 127);
        }
        acc_f = c0[0] + c1[1] + c2[2] + c3[3];
    }
    const int v = acc_i ^ __float_as_int(acc_f);
    if (v == 0x1234567) sink[blockIdx.x] = v;
}

// Streaming read: each thread issues 16 nontemporal 16-byte loads of one
// 64 KiB-per-workgroup chunk before using any, folds them, and stores one
// word only on a practically impossible value.
__global__ void __launch_bounds__(256)
probe_read(const v4u* __restrict__ p, int* __restrict__ sink) {
    const v4u* b = p + (int64_t)blockIdx.x * 4096 + threadIdx.x;
    v4u r[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) r[i] = __builtin_nontemporal_load(b + i * 256);
    v4u x = r[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) x ^= r[i];
    const unsigned v = x[0] ^ x[1] ^ x[2] ^ x[3];
    if (v == 0x89abcdefu) sink[blockIdx.x & 1023] = (int)v;
}

// Every fp32 bit pattern (two per thread and step, grid-stride): the
// library's hardware bf16 conversion against the integer round-to-nearest-
// even, NaN inputs skipped; mismatches are counted into *bad.
__global__ void __launch_bounds__(256)
probe_bf16_rne(unsigned long long* __restrict__ bad) {
    const uint64_t n = (uint64_t)gridDim.x * 256;
    unsigned long long nbad = 0;
    for (uint64_t i = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 2; i < (1ull << 32); i += 2 * n) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t u = (uint32_t)(i + k);
            const float f = __uint_as_float(u);
            if ((u & 0x7fffffffu) <= 0x7f800000u && f32_to_bf16_rne(f) != f32_to_bf16_rne_int(f)) ++nbad;
        }
    }
    if (nbad) atomicAdd(bad, nbad);
}

}  // namespace
}  // namespace nv4

extern "C" int nv4_probe_bf16_rne(unsigned long long* mismatches, void* stream) {
    using namespace nv4;
    if (!mismatches) return NV4_E_NULL;
    hipLaunchKernelGGL(probe_bf16_rne, dim3(8192), dim3(256), 0, static_cast<hipStream_t>(stream), mismatches);
    return (int)hipGetLastError();
}

extern "C" int nv4_probe_mfma(int kind, int64_t iters, int64_t workgroups, int* sink, void* stream) {
    using namespace nv4;
    if (!sink) return NV4_E_NULL;
    if (kind < 0 || kind > 2 || iters < 1 || iters > (1LL << 30) || workgroups < 1 || workgroups > (1 << 20))
        return NV4_E_SHAPE;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (kind == 0)
        hipLaunchKernelGGL(probe_mfma<0>, dim3((unsigned)workgroups), dim3(256), 0, st, iters, sink);
    else if (kind == 1)
        hipLaunchKernelGGL(probe_mfma<1>, dim3((unsigned)workgroups), dim3(256), 0, st, iters, sink);
    else
        hipLaunchKernelGGL(probe_mfma<2>, dim3((unsigned)workgroups), dim3(256), 0, st, iters, sink);
    return (int)hipGetLastError();
}

extern "C" int nv4_probe_read(const void* buf, int64_t bytes, int* sink, void* stream) {
    using namespace nv4;
    if (!buf || !sink) return NV4_E_NULL;
    if (bytes < 65536 || bytes % 65536 || bytes / 65536 > 0x7fffffffLL) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(buf) % 16) return NV4_E_ALIGN;
    hipLaunchKernelGGL(probe_read, dim3((unsigned)(bytes / 65536)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const v4u*>(buf), sink);
    return (int)hipGetLastError();
}
