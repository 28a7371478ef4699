// Per-head q/k RMSNorm + rotary embedding shared by qk_norm_rope_store
// (decoder_ops.hip) and the fused decode attention (paged_attention.hip).
#pragma once

#include "norm_ops.h"

namespace nv4 {
namespace {

// Per-head q/k RMSNorm + rotary embedding of a 128-dim head
// (nanovllm/models/qwen3.py:78-94, layers/rotary_embedding.py:6-48) by
// sixteen lanes, shared by qk_norm_rope_store (decoder_ops.hip) and the fused
// decode attention (paged_attention.hip), so both give the same bits.  Lane
// j of the sixteen holds dims 4j .. 4j+3 (xa: two bf16 pairs) and their rotary
// partners 64 + 4j .. 64 + 4j+3 (xb), the norm weights of those dims (wa, wb)
// and cos / sin of dims 4j .. 4j+3 (c, s).  Sum of squares: each lane from 0
// in order, ss += x1^2 + x2^2, then xor steps 8, 4, 2, 1 over the sixteen;
// r = rsqrtf(ss / 128 + eps); a = bf16(bf16(x * r) * w); y1 = bf16(a1 c -
// a2 s), y2 = bf16(a2 c + a1 s), each product rounded.  o1 = y1 of dims 4j..,
// o2 = y2 of dims 64 + 4j.., as bf16 pairs.  The bf16 -> fp32 widening is a
// byte permute: a shift after a load in a branch would be moved next to the
// load by the compiler, and wait for it there.
__device__ __forceinline__ float bf16_lo_f32(uint32_t w) { return __uint_as_float(__builtin_amdgcn_perm(0u, w, 0x01000c0cu)); }
__device__ __forceinline__ float bf16_hi_f32(uint32_t w) { return __uint_as_float(__builtin_amdgcn_perm(0u, w, 0x03020c0cu)); }

__device__ __forceinline__ void qk_head16(uint2 xa, uint2 xb, uint2 wa, uint2 wb, v4f c, v4f s, float eps, uint2& o1,
                                          uint2& o2) {
    float x1[4], x2[4], w1[4], w2[4];
    const uint32_t xs[4] = {xa.x, xa.y, xb.x, xb.y}, ws[4] = {wa.x, wa.y, wb.x, wb.y};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        x1[2 * i] = bf16_lo_f32(xs[i]);
        x1[2 * i + 1] = bf16_hi_f32(xs[i]);
        x2[2 * i] = bf16_lo_f32(xs[2 + i]);
        x2[2 * i + 1] = bf16_hi_f32(xs[2 + i]);
        w1[2 * i] = bf16_lo_f32(ws[i]);
        w1[2 * i + 1] = bf16_hi_f32(ws[i]);
        w2[2 * i] = bf16_lo_f32(ws[2 + i]);
        w2[2 * i + 1] = bf16_hi_f32(ws[2 + i]);
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) ss += x1[i] * x1[i] + x2[i] * x2[i];
    // xor steps 8, 4, 2, 1 as rotations inside the row of sixteen lanes (the
    // same partners: see wave_sum).
    ss += row_ror<0x128>(ss);
    ss += row_ror<0x124>(ss);
    ss += row_ror<0x122>(ss);
    ss += row_ror<0x121>(ss);
    const float r = rsqrtf(ss / 128.0f + eps);
    uint32_t y1p[2], y2p[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a1 = round_bf16(round_bf16(x1[i] * r) * w1[i]);
        const float a2 = round_bf16(round_bf16(x2[i] * r) * w2[i]);
        const uint32_t y1 = f32_to_bf16_rne(a1 * c[i] - a2 * s[i]);
        const uint32_t y2 = f32_to_bf16_rne(a2 * c[i] + a1 * s[i]);
        if (i & 1) {
            y1p[i >> 1] |= y1 << 16;
            y2p[i >> 1] |= y2 << 16;
        } else {
            y1p[i >> 1] = y1;
            y2p[i >> 1] = y2;
        }
    }
    o1 = make_uint2(y1p[0], y1p[1]);
    o2 = make_uint2(y2p[0], y2p[1]);
}

}  // namespace
}  // namespace nv4
