// Elementwise / normalisation pieces shared by the standalone decoder kernels
// (decoder_ops.hip) and the fused prologues of K1 (rht_quant_pack.hip), so
// that "op, then K1" and "op fused into K1" produce the same bits.
//
// RMSNorm (nanovllm/layers/layernorm.py:16-50) in one fixed order: thread t
// of a 256-thread workgroup owns the 16-value units u = t, t + 256, ... of
// the row and accumulates fmaf(h, h, ss) over its values in column order;
// the wave sums by xor-shuffles 32, 16, .., 1; the workgroup adds the four
// wave partials left to right.  r = rsqrtf(ss / H + eps) and
// y = bf16(bf16(h * r) * w).
// SiLU-and-mul (nanovllm/layers/activation.py:8-11): y = bf16(bf16(g /
// (1 + expf(-g))) * u), fp32 arithmetic.
#pragma once

#include "nv4_common.h"

namespace nv4 {
namespace {

// Lane value rotated within its row of 16 lanes (DPP row_ror:n, n = CTRL - 0x120).
template <int CTRL>
__device__ __forceinline__ float row_ror(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over the wave by xor-butterflies 32, 16, 8, 4, 2, 1 (v + partner at each
// step).  After the 32 and 16 steps the partial sums repeat every 16 lanes,
// after the 8 step every 8 and so on, so rotating by 8, 4, 2, 1 inside a row of
// 16 lanes hands each lane the same partner value as xor 8, 4, 2, 1: the same
// additions in the same order, on the VALU instead of the LDS crossbar.
__device__ __forceinline__ float wave_sum(float v) {
    v += __shfl_xor(v, 32);
    v += __shfl_xor(v, 16);
    v += row_ror<0x128>(v);
    v += row_ror<0x124>(v);
    v += row_ror<0x122>(v);
    v += row_ror<0x121>(v);
    return v;
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16_rne(f)); }

// h = float(x) (+ float(res)) for 16 contiguous values given as bf16 pairs
// (x0, x1; r0, r1); with a residual the rounded sum goes to res_out.
// Accumulates the sum of squares into ss.
template <bool RESID>
__device__ __forceinline__ void rms_h16(const v4u x0, const v4u x1, const v4u r0, const v4u r1, uint16_t* res_out,
                                        float (&h)[16], float& ss) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t xw = i < 8 ? x0[(i & 7) >> 1] : x1[(i & 7) >> 1];
        float f = bf16_to_f32((xw >> (16 * (i & 1))) & 0xffffu);
        if constexpr (RESID) {
            const uint32_t rw = i < 8 ? r0[(i & 7) >> 1] : r1[(i & 7) >> 1];
            f = f + bf16_to_f32((rw >> (16 * (i & 1))) & 0xffffu);
        }
        h[i] = f;
        ss = __builtin_fmaf(f, f, ss);
    }
    if constexpr (RESID) {
        v4u o0, o1;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            o0[k] = f32_to_bf16_rne(h[2 * k]) | (f32_to_bf16_rne(h[2 * k + 1]) << 16);
            o1[k] = f32_to_bf16_rne(h[8 + 2 * k]) | (f32_to_bf16_rne(h[8 + 2 * k + 1]) << 16);
        }
        *reinterpret_cast<v4u*>(res_out) = o0;
        *reinterpret_cast<v4u*>(res_out + 8) = o1;
    }
}

// rms_h16 on 16 contiguous values loaded from x (and res).
template <bool RESID>
__device__ __forceinline__ void rms_load16(const uint16_t* __restrict__ x, const uint16_t* res, uint16_t* res_out,
                                           float (&h)[16], float& ss) {
    const v4u x0 = *reinterpret_cast<const v4u*>(x);
    const v4u x1 = *reinterpret_cast<const v4u*>(x + 8);
    v4u r0 = {0u, 0u, 0u, 0u}, r1 = r0;
    if constexpr (RESID) {
        r0 = *reinterpret_cast<const v4u*>(res);
        r1 = *reinterpret_cast<const v4u*>(res + 8);
    }
    rms_h16<RESID>(x0, x1, r0, r1, res_out, h, ss);
}

// Workgroup (256 threads) reduction of the per-thread sums of squares and
// the reciprocal RMS.  red: 4 floats of LDS; ends with a barrier after which
// red may be reused.
__device__ __forceinline__ float rms_rsqrt256(float ss, float* red, int H, float eps) {
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = ((red[0] + red[1]) + red[2]) + red[3];
    return rsqrtf(tot / (float)H + eps);
}

// y = bf16(bf16(h * r) * w) for 16 contiguous values, as fp32 (w0, w1: the
// 16 bf16 weights, loaded by the caller ahead of the row).
__device__ __forceinline__ void rms_apply16(const float (&h)[16], float r, const v4u w0, const v4u w1,
                                            float (&y)[16]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t ww = i < 8 ? w0[(i & 7) >> 1] : w1[(i & 7) >> 1];
        const float wf = bf16_to_f32((ww >> (16 * (i & 1))) & 0xffffu);
        y[i] = round_bf16(round_bf16(h[i] * r) * wf);
    }
}
__device__ __forceinline__ void rms_apply16(const float (&h)[16], float r, const uint16_t* __restrict__ w,
                                            float (&y)[16]) {
    rms_apply16(h, r, *reinterpret_cast<const v4u*>(w), *reinterpret_cast<const v4u*>(w + 8), y);
}

__device__ __forceinline__ float silu_mul1(float g, float u) { return round_bf16(round_bf16(g / (1.0f + expf(-g))) * u); }

// y = silu(g) * u (bf16 rounding points above) for 16 contiguous values
// given as bf16 pairs (g0, g1; u0, u1).
__device__ __forceinline__ void silu_mul16(const v4u g0, const v4u g1, const v4u u0, const v4u u1, float (&y)[16]) {
    float gf[16], uf[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t gw = i < 8 ? g0[(i & 7) >> 1] : g1[(i & 7) >> 1];
        const uint32_t uw = i < 8 ? u0[(i & 7) >> 1] : u1[(i & 7) >> 1];
        gf[i] = bf16_to_f32((gw >> (16 * (i & 1))) & 0xffffu);
        uf[i] = bf16_to_f32((uw >> (16 * (i & 1))) & 0xffffu);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) y[i] = silu_mul1(gf[i], uf[i]);
}

__device__ __forceinline__ void silu_mul16(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                           float (&y)[16]) {
    silu_mul16(*reinterpret_cast<const v4u*>(g), *reinterpret_cast<const v4u*>(g + 8),
               *reinterpret_cast<const v4u*>(u), *reinterpret_cast<const v4u*>(u + 8), y);
}

}  // namespace
}  // namespace nv4
