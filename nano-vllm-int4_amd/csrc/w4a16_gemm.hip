// K3: W4A16 GEMM with GPTQ-packed INT4 weights, for gfx950.
//
// Reference: nanovllm/layers/linear_w4a16.py:11-59 (TileLang dequant GEMM,
// split-K = 8 with BF16 atomics).  Dequantization as the reference does it
// (:45-55, GPTQ zero convention w = (q - z - 1) * s):
//   bf16 activations: deq = bf16_rne(float(q - z - 1) * float(bf16(s)))
//   fp16 activations: deq = fp16_rne(float(q - z - 1) * float(s))
// (q - z - 1 is a small integer and the product is exact in fp32, so each
// dequantized weight is rounded once.)  Products are summed in fp32 by
// v_mfma_f32_16x16x32_{bf16,f16} over the whole K; there are no atomics and
// the result does not depend on scheduling.
//
// Layout: one workgroup per 16 output columns and up to 64 rows (4 m-blocks
// of 16).  The four waves split K into interleaved 32-deep steps and their
// fp32 partial tiles are added in LDS in wave order at the end (fixed
// order, deterministic).  Each lane's B operand is exactly one qweight word
// (8 consecutive k of one column), dequantized in registers.
#include "nv4_common.h"

namespace nv4 {
namespace {

template <bool FP16>
struct W16Traits;
template <>
struct W16Traits<false> {
    typedef v8bf vec;
    typedef __bf16 elem;
    __device__ static inline uint16_t cvt(float f) { return (uint16_t)f32_to_bf16_rne(f); }
    __device__ static inline float scale_of(uint16_t s_f16) {
        // fp16 -> fp32 (exact) -> bf16 (rne), as the reference copies fp16
        // scales into a bf16 buffer.
        return bf16_to_f32(f32_to_bf16_rne((float)__builtin_bit_cast(_Float16, s_f16)));
    }
};
template <>
struct W16Traits<true> {
    typedef v8h vec;
    typedef _Float16 elem;
    __device__ static inline uint16_t cvt(float f) {
        return __builtin_bit_cast(uint16_t, (_Float16)f);
    }
    __device__ static inline float scale_of(uint16_t s_f16) {
        return (float)__builtin_bit_cast(_Float16, s_f16);
    }
};

template <int MB, bool XF16, bool OF16>
__global__ void __launch_bounds__(256)
k3_w4a16(const uint16_t* __restrict__ x, const int32_t* __restrict__ qweight,
         const int32_t* __restrict__ qzeros, const uint16_t* __restrict__ scales,
         void* __restrict__ out, int M, int N, int K) {
    using TR = W16Traits<XF16>;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * 16;
    const int m0 = blockIdx.y * 64;
    const int rc = lane & 15, kq = lane >> 4;  // row/column in block, k-octet within a step
    const int col = min(n0 + rc, N - 1);
    __shared__ float part[4][MB][256];

    const uint16_t* xp[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int r = min(m0 + mb * 16 + rc, M - 1);
        xp[mb] = x + (int64_t)r * K + kq * 8;
    }
    v4f acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = v4f{0.f, 0.f, 0.f, 0.f};

    const int steps = K >> 5;  // 32-deep k steps
    for (int st = wave; st < steps; st += 4) {
        const int k0 = st * 32;
        const int g = k0 >> 7;
        const uint32_t qw = (uint32_t)qweight[(int64_t)(k0 / 8 + kq) * N + col];
        const uint32_t zw = (uint32_t)qzeros[(int64_t)g * (N / 8) + col / 8];
        const int zp1 = (int)((zw >> (4 * (col & 7))) & 15u) + 1;
        const float s = TR::scale_of(scales[(int64_t)g * N + col]);
        typename TR::vec bop;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int q = (int)((qw >> (4 * j)) & 15u);
            const float v = (float)(q - zp1) * s;
            bop[j] = __builtin_bit_cast(typename TR::elem, TR::cvt(v));
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const uint4 xv = *reinterpret_cast<const uint4*>(xp[mb] + k0);
            typename TR::vec aop = __builtin_bit_cast(typename TR::vec, xv);
            if constexpr (XF16)
                acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, acc[mb], 0, 0, 0);
            else
                acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop, bop, acc[mb], 0, 0, 0);
        }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
        *reinterpret_cast<v4f*>(&part[wave][mb][lane * 4]) = acc[mb];
    __syncthreads();
    // Thread e sums entry e of each m-block over the four waves in order.
    const int e = threadIdx.x;
    const int el = e >> 2, ei = e & 3;
    const int on = n0 + (el & 15);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int om = m0 + mb * 16 + 4 * (el >> 4) + ei;
        float v = part[0][mb][e];
        v = v + part[1][mb][e];
        v = v + part[2][mb][e];
        v = v + part[3][mb][e];
        if (om < M && on < N) {
            const uint16_t h = OF16 ? __builtin_bit_cast(uint16_t, (_Float16)v) : (uint16_t)f32_to_bf16_rne(v);
            static_cast<uint16_t*>(out)[(int64_t)om * N + on] = h;
        }
    }
}

template <int MB, bool XF, bool OF>
hipError_t launch(const void* x, const int32_t* qw, const int32_t* qz, const void* sc, void* out,
                  int M, int N, int K, hipStream_t st) {
    dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + 63) / 64));
    hipLaunchKernelGGL((k3_w4a16<MB, XF, OF>), grid, dim3(256), 0, st, static_cast<const uint16_t*>(x), qw, qz,
                       static_cast<const uint16_t*>(sc), out, M, N, K);
    return hipGetLastError();
}

template <bool XF, bool OF>
hipError_t dispatch(const void* x, const int32_t* qw, const int32_t* qz, const void* sc, void* out,
                    int M, int N, int K, hipStream_t st) {
    if (M <= 16) return launch<1, XF, OF>(x, qw, qz, sc, out, M, N, K, st);
    if (M <= 32) return launch<2, XF, OF>(x, qw, qz, sc, out, M, N, K, st);
    if (M <= 48) return launch<3, XF, OF>(x, qw, qz, sc, out, M, N, K, st);
    return launch<4, XF, OF>(x, qw, qz, sc, out, M, N, K, st);
}

}  // namespace
}  // namespace nv4

extern "C" int nv4_w4a16_gemm(const void* x, int x_dtype, const int32_t* qweight, const int32_t* qzeros,
                              const void* scales, void* out, int out_dtype,
                              int64_t M, int64_t N, int64_t K, int group, void* stream) {
    using namespace nv4;
    if (!x || !qweight || !qzeros || !scales || !out) return NV4_E_NULL;
    if ((x_dtype != NV4_BF16 && x_dtype != NV4_FP16) || (out_dtype != NV4_BF16 && out_dtype != NV4_FP16))
        return NV4_E_DTYPE;
    if (group != 128) return NV4_E_GROUP;
    if (M < 1 || N < 8 || N % 8 || K < 128 || K % 128) return NV4_E_SHAPE;
    if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > (1LL << 24) || (M + 63) / 64 > 65535) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(qweight) % 4 ||
        reinterpret_cast<uintptr_t>(qzeros) % 4 || reinterpret_cast<uintptr_t>(scales) % 2 ||
        reinterpret_cast<uintptr_t>(out) % 2)
        return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int m = (int)M, n = (int)N, k = (int)K;
    hipError_t e;
    if (x_dtype == NV4_FP16)
        e = out_dtype == NV4_FP16 ? dispatch<true, true>(x, qweight, qzeros, scales, out, m, n, k, st)
                                  : dispatch<true, false>(x, qweight, qzeros, scales, out, m, n, k, st);
    else
        e = out_dtype == NV4_FP16 ? dispatch<false, true>(x, qweight, qzeros, scales, out, m, n, k, st)
                                  : dispatch<false, false>(x, qweight, qzeros, scales, out, m, n, k, st);
    return (int)e;
}
