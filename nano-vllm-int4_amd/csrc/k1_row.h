// Device code of the reference-layout RHT + group-128 quantization + INT4
// pack for one row (shared by the standalone K1 kernel and the fused decode
// linear kernel).
//
// Numerical contract (nanovllm/kernels/rht_a4_tilelang.py:58-135,
// benchmarks/rht_a4_bench_common.py:19-36), reproduced bit for bit:
//   a[k] = fp32(x[k]) * fp32(sign[k])                         (exact)
//   Sylvester butterflies on each F-point chunk, strides 1,2,..,F/2 in
//   increasing order: (lo, hi) -> (lo+hi, lo-hi), all fp32
//   a *= 1/sqrt(F)      (F = 4096 -> 2^-6, F = 1024 -> 2^-5; exact)
//   K = 12288 only: out[d] = RN(1/sqrt 12) * (sum_{s=0..11} +-a[s]), summed in
//   source order (k = s*1024 + c, Paley signs)
//   group-128 scale: mx = max|a|, t = RN(RN(mx*0.9f)*RN(1/7)),
//   scale = mx == 0 ? 1 : bf16_rne(max(t, 2^-126)); q = clamp(rint(a/scale), -7, 7)
//   with IEEE division; byte = (q[2i] & 15) | (q[2i+1] & 15) << 4.
//
// Mapping to the hardware.  A team of T threads owns one row.  Each thread
// keeps L = K/T fp32 values in VGPRs.  Butterfly stages run only on
// register-index bits: the row is passed through LDS between "phases" so
// that the next B = log2(F/T) chunk-index bits become register bits (an LDS
// transpose), and the stages of each phase are plain VALU adds in registers.
// The H12 stage needs all 12 chunks of one column in one thread: every phase
// mapping keeps the chunk index in registers, so it runs in registers too.
// Quantization reads the row back from LDS as 16 contiguous values per
// thread, so one 128-group is 8 adjacent lanes (3 xor-shuffles for the max),
// and each thread emits 8 packed bytes with one store.
#pragma once

#include "nv4_common.h"

namespace nv4 {
namespace {

// One pad float per 16 keeps strided phase accesses bank-conflict free.
__device__ __forceinline__ int lds_idx(int i) { return i + (i >> 4); }

__device__ __forceinline__ bool paley_positive(int s, int d) {
    if (s == 0 || d == 0) return true;
    const int delta = ((d - s) % 11 + 11) % 11;
    return delta == 1 || delta == 3 || delta == 4 || delta == 5 || delta == 9;
}

// Chunk-column index held by thread t in register slot r when the register
// window starts at bit w: low thread bits below w, register bits at w..w+B-1,
// high thread bits above.
template <int B>
__device__ __forceinline__ int col_of(int t, int r, int w) {
    const int low = t & ((1 << w) - 1);
    return low | (r << w) | ((t >> w) << (w + B));
}

// Quantize 16 contiguous values (one eighth of a 128-group, 8 adjacent lanes
// hold the group), write 8 packed bytes and, from the group's first lane, the
// bf16 scale.
__device__ __forceinline__ void quantize16_store(const float (&v)[16], int8_t* __restrict__ dst8,
                                                 uint16_t* __restrict__ scale_dst, bool leader,
                                                 bool live = true) {
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(v[i]));
    mx = fmaxf(mx, __shfl_xor(mx, 1));
    mx = fmaxf(mx, __shfl_xor(mx, 2));
    mx = fmaxf(mx, __shfl_xor(mx, 4));
    uint32_t sb;
    if (mx == 0.0f) {
        sb = 0x3F80u;  // 1.0
    } else {
        float t = mx * 0x1.ccccccp-1f;   // fp32(0.9)
        t = t * 0x1.24924ap-3f;          // RN(1/7)
        t = fmaxf(t, 0x1p-126f);
        sb = f32_to_bf16_rne(t);
    }
    const float s = bf16_to_f32(sb);
    uint32_t word[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        float q = __builtin_rintf(v[i] / s);
        q = fminf(fmaxf(q, -7.0f), 7.0f);
        const uint32_t nib = (uint32_t)((int)q) & 15u;
        word[i >> 3] |= nib << (4 * (i & 7));
    }
    if (live) {
        *reinterpret_cast<uint2*>(dst8) = make_uint2(word[0], word[1]);
        if (leader) *scale_dst = (uint16_t)sb;
    }
}

template <int C, int F, int T>
struct Shape {
    static constexpr int K = C * F;
    static constexpr int LOGF = ilog2c(F);
    static constexpr int LC = F / T;                 // chunk columns per thread
    static constexpr int B = ilog2c(LC);             // register bits per phase
    static constexpr int L = C * LC;                 // values per thread
    static constexpr int NP = (LOGF + B - 1) / B;    // butterfly phases
    static constexpr int LDS = K + K / 16;
    static_assert(LC >= 2 && (LC & (LC - 1)) == 0, "need >= 2 power-of-two columns per thread");
    static_assert(T % 64 == 0 && T <= 1024, "whole waves");
    static_assert(K % (16 * 64) == 0, "quantization units must fill whole waves");
};

__host__ __device__ constexpr int window_of(int p, int B, int LOGF) {
    return (p * B < LOGF - B) ? p * B : LOGF - B;
}

// Workgroup barriers executed by k1_row<C, F, T> (2 per phase after the
// first, 1 before quantization): waves outside the team that must keep the
// workgroup in step call k1_row_shadow, which executes exactly these.
template <int C, int F, int T>
__host__ __device__ constexpr int k1_barriers() { return 2 * (Shape<C, F, T>::NP - 1) + 1; }

template <int C, int F, int T>
__device__ __forceinline__ void k1_row_shadow() {
#pragma unroll
    for (int i = 0; i < k1_barriers<C, F, T>(); ++i) __syncthreads();
}

// The reference-layout transform of one row by a team of T threads (whole
// waves; t = thread index inside the team).  C = 1, F = 4096 (K = 4096) or
// C = 12, F = 1024 (K = 12288).  buf is the team's LDS scratch (S::LDS
// floats).  Every thread of the workgroup must call it (it contains
// workgroup barriers); a team with live == false computes but stores nothing.
template <int C, int F, int T>
__device__ __forceinline__ void k1_row(const uint16_t* __restrict__ xr, const int8_t* __restrict__ signs,
                                       int8_t* __restrict__ prow, uint16_t* __restrict__ srow,
                                       float* __restrict__ buf, int t, bool live) {
    using S = Shape<C, F, T>;
    float a[S::L];  // a[s * LC + r]

    // Phase-0 mapping: column c = t*LC + r (contiguous), loaded straight from HBM.
#pragma unroll
    for (int s = 0; s < C; ++s) {
        const int base = s * F + t * S::LC;
#pragma unroll
        for (int r0 = 0; r0 < S::LC; r0 += 8) {
            uint4 xv;
            uint2 sv;
            if constexpr (S::LC >= 8) {
                xv = *reinterpret_cast<const uint4*>(xr + base + r0);
                sv = *reinterpret_cast<const uint2*>(signs + base + r0);
            } else {  // LC == 4 or 2
                const uint2 h = *reinterpret_cast<const uint2*>(xr + base + r0);
                xv = make_uint4(h.x, h.y, 0u, 0u);
                sv = make_uint2(*reinterpret_cast<const uint32_t*>(signs + base + r0), 0u);
            }
            const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
            const uint32_t sw[2] = {sv.x, sv.y};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (r0 + i < S::LC) {
                    const uint32_t h = (xw[i >> 1] >> (16 * (i & 1))) & 0xffffu;
                    const int sg = (int)(int8_t)((sw[i >> 2] >> (8 * (i & 3))) & 0xffu);
                    a[s * S::LC + r0 + i] = bf16_to_f32(h) * (float)sg;
                }
            }
        }
    }

#pragma unroll
    for (int p = 0; p < S::NP; ++p) {
        const int w = window_of(p, S::B, S::LOGF);
        if (p > 0) {
            const int wp = window_of(p - 1, S::B, S::LOGF);
#pragma unroll
            for (int s = 0; s < C; ++s)
#pragma unroll
                for (int r = 0; r < S::LC; ++r)
                    buf[lds_idx(s * F + col_of<S::B>(t, r, wp))] = a[s * S::LC + r];
            __syncthreads();
#pragma unroll
            for (int s = 0; s < C; ++s)
#pragma unroll
                for (int r = 0; r < S::LC; ++r)
                    a[s * S::LC + r] = buf[lds_idx(s * F + col_of<S::B>(t, r, w))];
            __syncthreads();
        }
        const int first = p * S::B;
        const int last = (first + S::B < S::LOGF) ? first + S::B : S::LOGF;
#pragma unroll
        for (int bit = first; bit < last; ++bit) {
            const int rb = 1 << (bit - w);
#pragma unroll
            for (int s = 0; s < C; ++s)
#pragma unroll
                for (int r = 0; r < S::LC; ++r) {
                    if ((r & rb) == 0) {
                        const float lo = a[s * S::LC + r], hi = a[s * S::LC + r + rb];
                        a[s * S::LC + r] = lo + hi;
                        a[s * S::LC + r + rb] = lo - hi;
                    }
                }
        }
    }

    const float norm = (F == 4096) ? 0x1p-6f : (F == 1024 ? 0x1p-5f : 0.0f);
    static_assert(F == 4096 || F == 1024, "reference chunk sizes");
#pragma unroll
    for (int i = 0; i < S::L; ++i) a[i] = a[i] * norm;

    if constexpr (C == 12) {
        const float inv12 = 0x1.279a74p-2f;  // RN(1/sqrt 12)
#pragma unroll
        for (int r = 0; r < S::LC; ++r) {
            float out[12];
#pragma unroll
            for (int d = 0; d < 12; ++d) {
                float acc = 0.0f;
#pragma unroll
                for (int s = 0; s < 12; ++s) {
                    const float v = a[s * S::LC + r];
                    acc = acc + (paley_positive(s, d) ? v : -v);
                }
                out[d] = acc * inv12;
            }
#pragma unroll
            for (int d = 0; d < 12; ++d) a[d * S::LC + r] = out[d];
        }
    }

    // Back to contiguous units of 16 for quantization.
    {
        const int wl = window_of(S::NP - 1, S::B, S::LOGF);
#pragma unroll
        for (int s = 0; s < C; ++s)
#pragma unroll
            for (int r = 0; r < S::LC; ++r)
                buf[lds_idx(s * F + col_of<S::B>(t, r, wl))] = a[s * S::LC + r];
    }
    __syncthreads();
    // K/16 units of 16 values; when T does not divide them the last pass is
    // taken by whole waves only (units and T are multiples of 64).
    constexpr int UNITS = S::K / 16;
#pragma unroll
    for (int j = 0; j < (UNITS + T - 1) / T; ++j) {
        const int u = t + j * T;
        if (UNITS % T == 0 || u < UNITS) {
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = buf[lds_idx(u * 16 + i)];
            quantize16_store(v, prow + u * 8, srow + (u >> 3), (t & 7) == 0, live);
        }
    }
}

}  // namespace
}  // namespace nv4
