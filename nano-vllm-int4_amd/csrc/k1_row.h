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
// in registers, with bits 0-3 and 8-9 on the lane index; bits 8-9 sit on
// lane bits 0-1 and are finished with DPP quad permutes.  K = 4096 spans
// four waves: one workgroup transpose brings bits 8-11 into registers.
// K = 12288 needs all 12 chunks of a column for the H12 stage: one thread
// per column reads them from LDS.  Quantization reads 16 contiguous values
// per thread (8 adjacent lanes hold one 128-group).
//
// LDS layout: each 1024-column chunk is stored XOR-swizzled (swz below) so
// that the contiguous, transposed, per-column and per-unit access patterns
// are all free of bank conflicts on 32 or 64 banks.
#pragma once

#include "nv4_common.h"

namespace nv4 {
namespace {

__device__ __forceinline__ int swz(int c) { return c ^ ((c >> 4) & 0x3F) ^ ((c >> 6) & 8); }

// Column of chunk-local index held by lane l in register r after the
// wave-local transpose: bits 0-3 = l >> 2, bits 4-7 = r, bits 8-9 = l & 3.
__device__ __forceinline__ int col_t(int l, int r) { return (l >> 2) | (r << 4) | ((l & 3) << 8); }

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

// Butterfly across lanes l and l ^ (1 << LB) (LB = 0 or 1): the lower lane
// keeps lo + hi, the upper lo - hi; fma(v, -1, t) rounds t - v once.
template <int LB>
__device__ __forceinline__ void lane_butterflies(float (&a)[16], int l) {
    const float sg = (l >> LB) & 1 ? -1.0f : 1.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float other = dpp<LB == 0 ? DPP_QUAD_XOR1 : DPP_QUAD_XOR2>(a[r]);
        a[r] = __builtin_fmaf(a[r], sg, other);
    }
}

// Max over the 8 adjacent lanes that hold one 128-group.
__device__ __forceinline__ float group8_max(float m) {
    m = fmaxf(m, dpp<DPP_QUAD_XOR1>(m));
    m = fmaxf(m, dpp<DPP_QUAD_XOR2>(m));
    return fmaxf(m, dpp<DPP_HALF_MIRROR>(m));
}

// Quantize 16 contiguous values (one eighth of a 128-group; the group's 8
// lanes must be active together), write 8 packed bytes and, from the group's
// first lane, the bf16 scale.
//
// Codes: q = clamp(rint(v / s)) with the IEEE quotient.  Fast path: p =
// v * rcp(s) with v_rcp_f32 (<= 1 ulp), so |p - v/s| <= 1.5 * 2^-23 * |v/s|
// < 2^-20 (|v/s| < 8 because s >= ~0.128 * max|v|).  If |p - rint(p)| <
// 0.5 - 2^-18, then v/s, and its rounded quotient (within 2^-22), lie
// strictly inside the same unit interval around rint(p), so rint of the IEEE
// quotient equals rint(p).  A lane whose values fail the test (near a
// half-integer, or s outside [2^-126, 2^100]) recomputes them with the IEEE
// division.  Nibbles are assembled exactly in fp32: sum (q_i + 8) * 16^i over
// four values is an integer below 2^16, and (q + 8) ^ 8 == q & 15.
__device__ __forceinline__ void quantize16_store(const float (&v)[16], int8_t* __restrict__ dst8,
                                                 uint16_t* __restrict__ scale_dst, bool leader) {
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(v[i]));
    mx = group8_max(mx);
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
    const float y = __builtin_amdgcn_rcpf(s);
    bool exact = s <= 0x1p100f;
    float q[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float p = v[i] * y;
        q[i] = __builtin_rintf(p);
        exact = exact & (fabsf(p - q[i]) < 0x1.ffffp-2f);
    }
    if (!exact) {
#pragma unroll
        for (int i = 0; i < 16; ++i) q[i] = __builtin_rintf(v[i] / s);
    }
    uint32_t half[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float h = __builtin_amdgcn_fmed3f(q[4 * j + 3], -7.0f, 7.0f);
#pragma unroll
        for (int i = 2; i >= 0; --i) h = __builtin_fmaf(h, 16.0f, __builtin_amdgcn_fmed3f(q[4 * j + i], -7.0f, 7.0f));
        half[j] = (uint32_t)(h + 34952.0f);  // + 8 * (1 + 16 + 256 + 4096)
    }
    const uint32_t w0 = (half[0] | (half[1] << 16)) ^ 0x88888888u;
    const uint32_t w1 = (half[2] | (half[3] << 16)) ^ 0x88888888u;
    *reinterpret_cast<uint2*>(dst8) = make_uint2(w0, w1);
    if (leader) *scale_dst = (uint16_t)sb;
}

// Butterfly bits 0-9 of the 1024-point chunk whose LDS block is blk, by one
// wave (lane l, columns 16l..16l+15 in a).  On return a holds columns
// col_t(l, r), and blk is free for the caller.
__device__ __forceinline__ void chunk1024_bits0_9(float (&a)[16], float* __restrict__ blk, int l) {
    reg_butterflies(a);
#pragma unroll
    for (int r = 0; r < 16; ++r) blk[swz(16 * l + r)] = a[r];
    wave_lds_sync();
#pragma unroll
    for (int r = 0; r < 16; ++r) a[r] = blk[swz(col_t(l, r))];
    reg_butterflies(a);
    lane_butterflies<0>(a, l);
    lane_butterflies<1>(a, l);
}

// K = 12288 (12 chunks of 1024) by 1024 threads: waves 0-11 run the
// butterflies of one chunk each, then every thread runs the H12 stage of one
// column, and threads 0-767 quantize one 16-column unit each.
constexpr int K12_THREADS = 1024;
constexpr int K12_LDS = 12 * 1024;

//
// The row's values come from a prologue: prologue(col0, v) fills v[0..15]
// with the fp32 values of columns col0..col0+15 (bf16 x, or the output of a
// fused RMSNorm / SiLU-mul rounded to bf16); they are multiplied by the
// signs here.  Threads 0-767 (waves 0-11) call it once each, with
// col0 = 16 t.
template <class Prologue>
__device__ __forceinline__ void k1_row12288(Prologue&& prologue, const int8_t* __restrict__ signs,
                                            int8_t* __restrict__ prow, uint16_t* __restrict__ srow,
                                            float* __restrict__ buf) {
    const int t = threadIdx.x, w = t >> 6, l = t & 63;
    if (w < 12) {
        float a[16];
        const v4u sv = load_signs16(signs + w * 1024 + 16 * l);
        prologue(w * 1024 + 16 * l, a);
        apply_signs16(sv, a);
        float* blk = buf + w * 1024;
        chunk1024_bits0_9(a, blk, l);
#pragma unroll
        for (int r = 0; r < 16; ++r) blk[swz(col_t(l, r))] = a[r] * 0x1p-5f;
    }
    __syncthreads();
    {
        const int c = swz(t);
        float v[12];
#pragma unroll
        for (int s = 0; s < 12; ++s) v[s] = buf[s * 1024 + c];
        const float inv12 = 0x1.279a74p-2f;  // RN(1/sqrt 12)
#pragma unroll
        for (int d = 0; d < 12; ++d) {
            float acc = v[0];
#pragma unroll
            for (int s = 1; s < 12; ++s) acc = paley_positive(s, d) ? acc + v[s] : acc - v[s];
            buf[d * 1024 + c] = acc * inv12;
        }
    }
    __syncthreads();
    if (w < 12) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = buf[w * 1024 + swz(16 * l + i)];
        quantize16_store(v, prow + 8 * t, srow + (t >> 3), (t & 7) == 0);
    }
}

// K = 4096 (one 4096-point chunk) by 256 threads: each wave runs bits 0-9 of
// its 1024-column quarter, one workgroup transpose brings bits 8-11 into
// registers (thread t: columns t | r << 8).  Every thread calls the
// prologue once, with col0 = 16 t.
constexpr int K4_LDS = 4 * 1024;

template <class Prologue>
__device__ __forceinline__ void k1_row4096(Prologue&& prologue, const int8_t* __restrict__ signs,
                                           int8_t* __restrict__ prow, uint16_t* __restrict__ srow,
                                           float* __restrict__ buf) {
    const int t = threadIdx.x, w = t >> 6, l = t & 63;
    float a[16];
    const v4u sv = load_signs16(signs + w * 1024 + 16 * l);
    prologue(w * 1024 + 16 * l, a);
    apply_signs16(sv, a);
    float* blk = buf + w * 1024;
    reg_butterflies(a);
#pragma unroll
    for (int r = 0; r < 16; ++r) blk[swz(16 * l + r)] = a[r];
    wave_lds_sync();
#pragma unroll
    for (int r = 0; r < 16; ++r) a[r] = blk[swz(col_t(l, r))];
    reg_butterflies(a);
#pragma unroll
    for (int r = 0; r < 16; ++r) blk[swz(col_t(l, r))] = a[r];
    __syncthreads();
    // register r: bits 0-1 -> column bits 8-9, bits 2-3 -> column bits 10-11.
#pragma unroll
    for (int r = 0; r < 16; ++r) a[r] = buf[(r >> 2) * 1024 + swz(t | ((r & 3) << 8))];
    reg_butterflies(a);
#pragma unroll
    for (int r = 0; r < 16; ++r) buf[(r >> 2) * 1024 + swz(t | ((r & 3) << 8))] = a[r] * 0x1p-6f;
    __syncthreads();
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = buf[w * 1024 + swz(16 * l + i)];
    quantize16_store(v, prow + 8 * t, srow + (t >> 3), (t & 7) == 0);
}

}  // namespace
}  // namespace nv4
