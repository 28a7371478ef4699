// Device code of the reference-layout RHT + group-128 quantization + INT4
// pack (K1) for K = 4096 and K = 12288.
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
// Mapping to the hardware.  A 1024-point chunk is one wave: lane l loads the
// 16 contiguous columns 16l..16l+15, so butterfly bits 0-3 are register
// bits.  A wave-local LDS transpose (no workgroup barrier) then puts bits 4-7
// in registers, with bits 0-3 and 8-9 on the lane index.  K = 4096 spans
// four waves: one workgroup transpose brings bits 8-11 into registers.
// K = 12288 finishes bits 8-9 (lane bits 0-1) with DPP quad permutes, and
// needs all 12 chunks of a column for the H12 stage: one thread per column
// reads them from LDS.  Quantization reads 16 contiguous values per thread
// (8 adjacent lanes hold one 128-group).
//
// LDS layout: column c of a 1024-column chunk sits at lds_pos(c) = c +
// (c >> 4) + 8 (c >> 9) in the chunk's block of K1_BLOCK floats.  Every
// access pattern above is then one base register per thread plus constant
// offsets (no per-access address arithmetic), and the 32 lanes a half-wave
// serves hit 32 distinct banks (the cross-wave transpose of K = 4096 has one
// two-way pair).
#pragma once

#include "nv4_common.h"

namespace nv4 {
namespace {

constexpr int K1_BLOCK = 1096;  // > lds_pos(1023) = 1094
__host__ __device__ constexpr int lds_pos(int c) { return c + (c >> 4) + 8 * (c >> 9); }

// Column of chunk-local index held by lane l in register r after the
// wave-local transpose: bits 0-3 = l >> 2, bits 4-7 = r, bits 8-9 = l & 3.
__device__ __forceinline__ int col_t(int l, int r) { return (l >> 2) | (r << 4) | ((l & 3) << 8); }
// lds_pos(16 l + r) = unit_base(l) + r; lds_pos(col_t(l, r)) = tr_base(l) + 17 r.
__device__ __forceinline__ int unit_base(int l) { return 17 * l + 8 * (l >> 5); }
__device__ __forceinline__ int tr_base(int l) { return (l >> 2) + 272 * (l & 3) + 8 * ((l & 3) >> 1); }

__host__ __device__ constexpr bool paley_positive(int s, int d) {
    if (s == 0 || d == 0) return true;
    const int delta = ((d - s) % 11 + 11) % 11;
    return delta == 1 || delta == 3 || delta == 4 || delta == 5 || delta == 9;
}

// DPP lane permutes (gfx9 dpp_ctrl encodings).
constexpr int DPP_QUAD_XOR1 = 0xB1;    // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;    // quad_perm [2,3,0,1]
constexpr int DPP_HALF_MIRROR = 0x141;  // lane i of each 8 reads lane 7-i

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// Orders the LDS accesses of one wave (executed in order by the LDS unit)
// without a workgroup barrier.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// 16 contiguous bf16 values as fp32.
__device__ __forceinline__ void load_bf16x16(const uint16_t* __restrict__ xp, float (&a)[16]) {
    const v4u x0 = *reinterpret_cast<const v4u*>(xp);
    const v4u x1 = *reinterpret_cast<const v4u*>(xp + 8);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t xw = i < 8 ? x0[(i & 7) >> 1] : x1[(i & 7) >> 1];
        a[i] = bf16_to_f32((xw >> (16 * (i & 1))) & 0xffffu);
    }
}

// a[i] *= sign[i] for 16 contiguous int8 signs sv (exact).  The signs are
// loaded before the row's values: vector loads complete in issue order, so
// the wait for the values then covers them too (loaded after the values,
// they would cost a second round trip to memory).
__device__ __forceinline__ v4u load_signs16(const int8_t* __restrict__ sp) {
    return *reinterpret_cast<const v4u*>(sp);
}
__device__ __forceinline__ void apply_signs16(const v4u sv, float (&a)[16]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int sg = (int)(int8_t)((sv[i >> 2] >> (8 * (i & 3))) & 0xffu);
        a[i] = a[i] * (float)sg;
    }
}

// Butterflies on register-index bits (strides 1, 2, 4, 8 in this order).
template <int N>
__device__ __forceinline__ void reg_butterflies(float (&a)[N]) {
#pragma unroll
    for (int rb = 1; rb < N; rb <<= 1)
#pragma unroll
        for (int r = 0; r < N; ++r)
            if ((r & rb) == 0) {
                const float lo = a[r], hi = a[r + rb];
                a[r] = lo + hi;
                a[r + rb] = lo - hi;
            }
}

// Butterfly across lanes l and l ^ (1 << LB) (LB = 0 or 1) in one fma per
// value, v = RN(partner * sg + v) with sg = -1 on the upper lane: the lower
// lane gets lo + hi, the upper hi - lo = -(lo - hi) (RN is symmetric).  So
// after the stages on bits 0 and 1 the lane holds its value times
// lane_flip(l) = (-1)^(bit 0 + bit 1 of l); the flip of the partners is the
// same at bit 1, and the caller's normalisation multiplies it out exactly.
template <int LB, int N>
__device__ __forceinline__ void lane_butterflies(float (&a)[N], int l) {
    const float sg = (l >> LB) & 1 ? -1.0f : 1.0f;
#pragma unroll
    for (int r = 0; r < N; ++r) a[r] = __builtin_fmaf(dpp<LB == 0 ? DPP_QUAD_XOR1 : DPP_QUAD_XOR2>(a[r]), sg, a[r]);
}
__device__ __forceinline__ float lane_flip(int l) { return ((l ^ (l >> 1)) & 1) ? -1.0f : 1.0f; }

// Quantization of N contiguous values per lane, the 128-group spread over
// 128/N adjacent lanes that must be active together (QLANES = 128 / N).
//
// Codes: q = clamp(rint(v / s)) with the IEEE quotient, computed as
// q + 8 = rint(p) for p = fma(v, rcp(s), 8): v_rcp_f32 is within 1 ulp, so
// |v * rcp(s) - v/s| <= 2^-23 |v/s| < 2^-20 (|v/s| < 8 because s >= ~0.128 *
// max|v|), the fma adds at most ulp(16)/2 = 2^-20, and the IEEE quotient is
// within 2^-21 of v/s: p lies within 2^-18 of v/s + 8 and of RN(v/s) + 8.
// If every |p - rint(p)| of the lane is below 0.5 - 2^-18, each of those
// lies strictly inside the unit interval around rint(p), so rint(RN(v/s)) + 8
// = rint(p).  A lane that fails the test (a value near a half-integer, or s
// outside [2^-126, 2^100]) recomputes its values with the IEEE division.
// Nibbles are assembled exactly in fp32: sum (q_i + 8) * 16^i over four
// values is an integer below 2^16, and (q + 8) ^ 8 == q & 15.
template <int N>
__device__ __forceinline__ uint32_t group_scale_bits(const float (&v)[N], float& s) {
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < N; i += 2) mx = fmaxf(mx, fmaxf(fabsf(v[i]), fabsf(v[i + 1])));
    mx = fmaxf(mx, dpp<DPP_QUAD_XOR1>(mx));
    if constexpr (N <= 32) mx = fmaxf(mx, dpp<DPP_QUAD_XOR2>(mx));
    if constexpr (N == 16) mx = fmaxf(mx, dpp<DPP_HALF_MIRROR>(mx));
    uint32_t sb;
    if (mx == 0.0f) {
        sb = 0x3F80u;  // 1.0
    } else {
        float t = mx * 0x1.ccccccp-1f;   // fp32(0.9)
        t = t * 0x1.24924ap-3f;          // RN(1/7)
        t = fmaxf(t, 0x1p-126f);
        sb = f32_to_bf16_rne(t);
    }
    s = bf16_to_f32(sb);
    return sb;
}

// Packed bytes of N codes: word k holds codes 8k..8k+7, low nibble first.
template <int N>
__device__ __forceinline__ void codes_pack(const float (&v)[N], float s, uint32_t (&words)[N / 8]) {
    const float y = __builtin_amdgcn_rcpf(s);
    float q[N], dev = 0.0f;
#pragma unroll
    for (int i = 0; i < N; i += 2) {
        const float p0 = __builtin_fmaf(v[i], y, 8.0f), p1 = __builtin_fmaf(v[i + 1], y, 8.0f);
        q[i] = __builtin_rintf(p0);
        q[i + 1] = __builtin_rintf(p1);
        dev = fmaxf(dev, fmaxf(fabsf(p0 - q[i]), fabsf(p1 - q[i + 1])));
    }
    if (!(dev < 0x1.ffffp-2f && s <= 0x1p100f)) {
#pragma unroll
        for (int i = 0; i < N; ++i) q[i] = __builtin_rintf(v[i] / s) + 8.0f;
    }
#pragma unroll
    for (int k = 0; k < N / 8; ++k) {
        uint32_t half[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int b = 8 * k + 4 * j;
            float h = __builtin_amdgcn_fmed3f(q[b + 3], 1.0f, 15.0f);
#pragma unroll
            for (int i = 2; i >= 0; --i) h = __builtin_fmaf(h, 16.0f, __builtin_amdgcn_fmed3f(q[b + i], 1.0f, 15.0f));
            half[j] = (uint32_t)h;
        }
        words[k] = (half[0] | (half[1] << 16)) ^ 0x88888888u;
    }
}

// Where the 8 packed bytes of one row's 16-column unit u (columns 16u ..
// 16u+15) go.  Reference layout: [M][K/2], bytes 8u.. of the row.  Row-tiled
// layout (the decode GEMM's activation operand): 1 KiB blocks, one per
// 16-row block rb and group g at (rb*G + g) KiB, lane l = 16*part + r of a
// block holding bytes 16*part .. +15 of the group's 64 for row 16*rb + r:
// unit u is group u/8, part (u/2)%4, half u%2 of that lane's 16 bytes.
template <bool RT>
__device__ __forceinline__ int8_t* packed_dst(int8_t* __restrict__ packed, int64_t row, int u, int K) {
    if constexpr (RT) {
        const int G = K >> 7;
        return packed + ((((row >> 4) * G + (u >> 3)) * 64 + ((u >> 1) & 3) * 16 + (row & 15)) << 4) + 8 * (u & 1);
    } else {
        return packed + row * (K >> 1) + 8 * u;
    }
}

// 16 values per lane, 8 lanes per group: 8 packed bytes and, from the
// group's first lane, the bf16 scale.
__device__ __forceinline__ void quantize16_store(const float (&v)[16], int8_t* __restrict__ dst8,
                                                 uint16_t* __restrict__ scale_dst, bool leader) {
    float s;
    const uint32_t sb = group_scale_bits(v, s);
    uint32_t w[2];
    codes_pack(v, s, w);
    *reinterpret_cast<uint2*>(dst8) = make_uint2(w[0], w[1]);
    if (leader) *scale_dst = (uint16_t)sb;
}

// Butterfly bits 0-9 of the 1024-point chunk whose LDS block is blk, by one
// wave (lane l, columns 16l..16l+15 in a).  On return a holds columns
// col_t(l, r) times lane_flip(l), and blk is free for the caller.
__device__ __forceinline__ void chunk1024_bits0_9(float (&a)[16], float* __restrict__ blk, int l) {
    reg_butterflies(a);
    float* pu = blk + unit_base(l);
#pragma unroll
    for (int r = 0; r < 16; ++r) pu[r] = a[r];
    wave_lds_sync();
    const float* pt = blk + tr_base(l);
#pragma unroll
    for (int r = 0; r < 16; ++r) a[r] = pt[17 * r];
    reg_butterflies(a);
    lane_butterflies<0>(a, l);
    lane_butterflies<1>(a, l);
}

// K = 12288 (12 chunks of 1024) by 1024 threads: waves 0-11 run the
// butterflies of one chunk each, then every thread runs the H12 stage of one
// column, and threads 0-767 quantize one 16-column unit each.
constexpr int K12_THREADS = 1024;
constexpr int K12_LDS = 12 * K1_BLOCK;

// The row's values come from a prologue: prologue(col0, v) fills v[0..15]
// with the fp32 values of columns col0..col0+15 (bf16 x, or the output of a
// fused RMSNorm / SiLU-mul rounded to bf16); they are multiplied by the
// signs sv here (the caller loads them, ahead of the row: k1_signs12288).
// Threads 0-767 (waves 0-11) call it once each, with col0 = 16 t.
__device__ __forceinline__ v4u k1_signs12288(const int8_t* __restrict__ signs) {
    const int w = min((int)threadIdx.x >> 6, 11), l = threadIdx.x & 63;
    return load_signs16(signs + w * 1024 + 16 * l);
}

template <class Prologue>
__device__ __forceinline__ void k1_row12288(Prologue&& prologue, const v4u sv, int8_t* __restrict__ pdst,
                                            uint16_t* __restrict__ srow, float* __restrict__ buf) {
    const int t = threadIdx.x, w = t >> 6, l = t & 63;
    if (w < 12) {
        float a[16];
        prologue(w * 1024 + 16 * l, a);
        apply_signs16(sv, a);
        float* blk = buf + w * K1_BLOCK;
        chunk1024_bits0_9(a, blk, l);
        float* pt = blk + tr_base(l);
        const float norm = lane_flip(l) * 0x1p-5f;
#pragma unroll
        for (int r = 0; r < 16; ++r) pt[17 * r] = a[r] * norm;
    }
    __syncthreads();
    {
        float* pc = buf + lds_pos(t);
        float v[12];
#pragma unroll
        for (int s = 0; s < 12; ++s) v[s] = pc[s * K1_BLOCK];
        const float inv12 = 0x1.279a74p-2f;  // RN(1/sqrt 12)
#pragma unroll
        for (int d = 0; d < 12; ++d) {
            float acc = v[0];
#pragma unroll
            for (int s = 1; s < 12; ++s) acc = paley_positive(s, d) ? acc + v[s] : acc - v[s];
            pc[d * K1_BLOCK] = acc * inv12;
        }
    }
    __syncthreads();
    if (w < 12) {
        const float* pu = buf + w * K1_BLOCK + unit_base(l);
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = pu[i];
        quantize16_store(v, pdst, srow + (t >> 3), (t & 7) == 0);
    }
}

// K = 4096 (one 4096-point chunk) by 256 threads: each wave runs bits 0-7 of
// its 1024-column quarter, one workgroup transpose brings bits 8-11 into
// registers (thread t: columns t + 256 r), a second one the contiguous
// units back for quantization.  Every thread calls the prologue once, with
// col0 = 16 t; sv are its 16 signs (k1_signs4096).  pdst is where the
// thread's 8 packed bytes go (packed_dst of its unit t).
constexpr int K4_THREADS = 256;
constexpr int K4_LDS = 4 * K1_BLOCK;

__device__ __forceinline__ v4u k1_signs4096(const int8_t* __restrict__ signs) {
    return load_signs16(signs + 16 * threadIdx.x);
}

template <class Prologue>
__device__ __forceinline__ void k1_row4096(Prologue&& prologue, const v4u sv, int8_t* __restrict__ pdst,
                                           uint16_t* __restrict__ srow, float* __restrict__ buf) {
    const int t = threadIdx.x, w = t >> 6, l = t & 63;
    float a[16];
    prologue(16 * t, a);
    apply_signs16(sv, a);
    reg_butterflies(a);
    float* pu = buf + w * K1_BLOCK + unit_base(l);
#pragma unroll
    for (int r = 0; r < 16; ++r) pu[r] = a[r];
    wave_lds_sync();
    float* pt = buf + w * K1_BLOCK + tr_base(l);
#pragma unroll
    for (int r = 0; r < 16; ++r) a[r] = pt[17 * r];
    reg_butterflies(a);
#pragma unroll
    for (int r = 0; r < 16; ++r) pt[17 * r] = a[r];
    __syncthreads();
    // Register r holds column t + 256 r: chunk r >> 2, chunk column
    // 256 (r & 3) + t, at lds_pos = t + (t >> 4) + 272 (r & 3) + 8 ((r & 3) >> 1).
    float* pc = buf + t + (t >> 4);
#pragma unroll
    for (int r = 0; r < 16; ++r) a[r] = pc[(r >> 2) * K1_BLOCK + 272 * (r & 3) + 8 * ((r & 3) >> 1)];
    reg_butterflies(a);
#pragma unroll
    for (int r = 0; r < 16; ++r) pc[(r >> 2) * K1_BLOCK + 272 * (r & 3) + 8 * ((r & 3) >> 1)] = a[r] * 0x1p-6f;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; ++i) a[i] = pu[i];
    quantize16_store(a, pdst, srow + (t >> 3), (t & 7) == 0);
}

}  // namespace
}  // namespace nv4
