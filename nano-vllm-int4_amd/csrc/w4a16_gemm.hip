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

typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

template <bool FP16>
struct W16Traits;
// The eight nibbles of a qweight word as bytes in k order: p0 = q0..q3,
// p1 = q4..q7 (two byte permutes of the low and high nibbles).
__device__ __forceinline__ void nibble_bytes(uint32_t w, uint32_t& p0, uint32_t& p1) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;  // q0 q2 q4 q6 / q1 q3 q5 q7
    p0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
    p1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
}

template <>
struct W16Traits<false> {
    typedef v8bf vec;
    typedef __bf16 elem;
    struct deq {
        float s, nzs;  // bf16-rounded scale, -(z+1) * s (exact in fp32)
    };
    __device__ static inline uint16_t cvt(float f) { return (uint16_t)f32_to_bf16_rne(f); }
    __device__ static inline float scale_of(uint16_t s_f16) {
        // fp16 -> fp32 (exact) -> bf16 (rne), as the reference copies fp16
        // scales into a bf16 buffer.
        return bf16_to_f32(f32_to_bf16_rne((float)__builtin_bit_cast(_Float16, s_f16)));
    }
    __device__ static inline deq prep(uint16_t s_f16, int zp1) {
        const float s = scale_of(s_f16);
        return {s, -((float)zp1 * s)};
    }
    // bf16 of (q - z - 1) * s for the word's 8 nibbles: fma(q, s, -(z+1) s)
    // is exact (every term is a small integer times a bf16), then one
    // rounding per value, two values per v_cvt_pk_bf16_f32.
    __device__ static inline vec dequant8(uint32_t w, const deq& d) {
        uint32_t p0, p1;
        nibble_bytes(w, p0, p1);
        float v[8];
        v[0] = __builtin_fmaf((float)(p0 & 0xffu), d.s, d.nzs);
        v[1] = __builtin_fmaf((float)((p0 >> 8) & 0xffu), d.s, d.nzs);
        v[2] = __builtin_fmaf((float)((p0 >> 16) & 0xffu), d.s, d.nzs);
        v[3] = __builtin_fmaf((float)(p0 >> 24), d.s, d.nzs);
        v[4] = __builtin_fmaf((float)(p1 & 0xffu), d.s, d.nzs);
        v[5] = __builtin_fmaf((float)((p1 >> 8) & 0xffu), d.s, d.nzs);
        v[6] = __builtin_fmaf((float)((p1 >> 16) & 0xffu), d.s, d.nzs);
        v[7] = __builtin_fmaf((float)(p1 >> 24), d.s, d.nzs);
        vec r;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const v2bf b = __builtin_convertvector((v2f){v[e], v[e + 1]}, v2bf);
            r[e] = b[0];
            r[e + 1] = b[1];
        }
        return r;
    }
};
template <>
struct W16Traits<true> {
    typedef v8h vec;
    typedef _Float16 elem;
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    struct deq {
        h2 s, nmz;  // (s, s) and (-(1024 + z + 1), ...) in fp16
    };
    __device__ static inline uint16_t cvt(float f) {
        return __builtin_bit_cast(uint16_t, (_Float16)f);
    }
    __device__ static inline float scale_of(uint16_t s_f16) {
        return (float)__builtin_bit_cast(_Float16, s_f16);
    }
    __device__ static inline deq prep(uint16_t s_f16, int zp1) {
        const _Float16 s = __builtin_bit_cast(_Float16, s_f16);
        const _Float16 m = (_Float16)(-(1024 + zp1));  // exact: an integer below 2048
        return {h2{s, s}, h2{m, m}};
    }
    // fp16 of (q - z - 1) * s for the word's 8 nibbles: each half is built
    // as the fp16 1024 + q (bit pattern 0x6400 | q), (1024 + q) - (1024 + z
    // + 1) is exact, and one packed multiply rounds (q - z - 1) * s once.
    __device__ static inline vec dequant8(uint32_t w, const deq& d) {
        uint32_t p0, p1;
        nibble_bytes(w, p0, p1);
        const uint32_t m = 0x64646464u;
        const uint32_t h[4] = {__builtin_amdgcn_perm(m, p0, 0x04010400u), __builtin_amdgcn_perm(m, p0, 0x04030402u),
                               __builtin_amdgcn_perm(m, p1, 0x04010400u), __builtin_amdgcn_perm(m, p1, 0x04030402u)};
        vec r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const h2 v = (__builtin_bit_cast(h2, h[e]) + d.nmz) * d.s;
            r[2 * e] = v[0];
            r[2 * e + 1] = v[1];
        }
        return r;
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

// ----------------------------------------------------------------------------
// Decode-sized kernel (M <= 64) with a deterministic split over K.
//
// At decode sizes the 16-column kernel above is bound by load latency (one
// 4-byte weight load per lane and 32-k step, waited on in turn) and by every
// workgroup re-reading the whole bf16 activation block.  Here a workgroup
// owns 64 columns and one 1024-deep K slice (grid: column blocks x slices):
//  * weights: lane l loads 16 contiguous bytes of a qweight row -- columns
//    4(l%16) .. +3 of k-octet l/16 -- so a wave reads four 256-byte runs per
//    32-k step, and all of the slice's loads (8 per lane) are issued up
//    front; the four words feed four MFMAs whose output columns are
//    4c + j (j = word);
//  * activations: the slice's rows (ROWS x 1024 bf16) are copied into LDS in
//    whole lines once per workgroup and read back as MFMA A operands
//    (16-byte chunks XOR-swizzled by row);
//  * dequantization (W16Traits::dequant8): two byte permutes put a word's
//    nibbles in k order as bytes; bf16 takes fma(q, s, -(z+1) s) (exact in
//    fp32) and rounds once per value, fp16 builds each half as 1024 + q
//    (bit pattern 0x6400 | q) and rounds (q - z - 1) * s once with packed
//    fp16 arithmetic -- the reference's rounding of the dequantized weight;
//  * wave w takes the 8 consecutive 32-k steps 8w .. 8w+7 of the slice (two
//    groups, so two scale/zero preparations per column); the four waves'
//    fp32 tiles are added in wave order in LDS, and the slice's [M, N] fp32
//    partial goes to the workspace; a second kernel adds the slices in order
//    and rounds once (no atomics, same bits on every run).
// ----------------------------------------------------------------------------
constexpr int K3_KS = 1024;  // k per slice
constexpr int K3_RSRC_WORD3 = 0x00020000;  // buffer resource word 3 (CDNA): 32-bit data format
constexpr int K3_NB = 64;    // columns per workgroup

__device__ __forceinline__ int k3_swz(int r, int c) { return r * (K3_KS * 2) + ((c ^ (r & 7)) << 4); }

template <int MB, bool XF16>
__global__ void __launch_bounds__(256, 1)
k3_dec(const uint16_t* __restrict__ x, const int32_t* __restrict__ qweight, const int32_t* __restrict__ qzeros,
       const uint16_t* __restrict__ scales, float* __restrict__ ws, int M, int N, int K) {
    using TR = W16Traits<XF16>;
    constexpr int ROWS = MB * 16;
    __shared__ __align__(16) uint8_t smem[ROWS * K3_KS * 2];  // activation slice, then the wave partials
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int n0 = blockIdx.x * K3_NB;
    const int slice = blockIdx.y;
    const int ks = slice * K3_KS;
    const int klen = min(K3_KS, K - ks);  // multiple of 128
    const int steps = klen >> 5;
    const int c4 = lane & 15, kq = lane >> 4;
    // Column quad of this lane; quads at or beyond N load the last valid quad (results dropped).
    const int ncol = min(n0 + 4 * c4, N - 4);

    // ---- loads, in the order their data is needed (vector loads return in
    // issue order, so a wait for one load is a wait for every earlier one):
    // the activation slice, then the slice's zero points and scales, then the
    // weights, which keep streaming in while the first k-steps run.
    // Activation slice (row r: 128 chunks of 16 bytes).  Rows at or beyond M
    // are not loaded: their LDS rows are zero and their results dropped.
    constexpr int CH = ROWS * (K3_KS / 8);  // 16-byte chunks
    constexpr int PER = CH / 256;
    // A buffer resource over the M rows: a load at or past its end returns
    // zeros without a memory access, so the loads stay unconditional (a load
    // under a branch makes the compiler wait for it at the join).
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x), (short)0, (int)((uint32_t)M * K * 2u), K3_RSRC_WORD3);
    v4u xv[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int q = t + i * 256;
        const int r = q >> 7, c = q & 127;
        const int cc = min(c, (klen >> 3) - 1);
        xv[i] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)(((uint32_t)r * K + ks + cc * 8) * 2u), 0, 0));
    }
    // Wave w takes the 8 consecutive 32-k steps 8w .. 8w+7 (groups 2w, 2w+1
    // of the slice).
    uint32_t zw[2];
    uint2 sv[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int g = (ks >> 7) + max(0, min(2 * wave + i, (klen >> 7) - 1));
        zw[i] = (uint32_t)qzeros[(int64_t)g * (N >> 3) + (ncol >> 3)];
        sv[i] = *reinterpret_cast<const uint2*>(scales + (int64_t)g * N + ncol);
    }
    const int nst = min(8, steps - 8 * wave);  // steps of this wave (may be <= 0)
    v4u wq[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int st = max(0, min(8 * wave + i, steps - 1));
        const int64_t row = (int64_t)((ks >> 3) + st * 4 + kq);
        wq[i] = *reinterpret_cast<const v4u*>(qweight + row * N + ncol);
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int q = t + i * 256;
        *reinterpret_cast<v4u*>(&smem[k3_swz(q >> 7, q & 127)]) = xv[i];
    }
    __syncthreads();

    v4f acc[MB][4];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[mb][j] = v4f{0.f, 0.f, 0.f, 0.f};
    const int zsh = 16 * (c4 & 1);  // the quad's 4 zero-point nibbles within its qzeros word
    // Per group and column: the scale (as the activation dtype rounds it)
    // and the zero-point offset.
    typename TR::deq dq[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t h = ((j < 2 ? sv[i].x : sv[i].y) >> (16 * (j & 1))) & 0xffffu;
            dq[i][j] = TR::prep((uint16_t)h, (int)((zw[i] >> (zsh + 4 * j)) & 15u) + 1);
        }
    auto kstep = [&](int i) {
        const int st = 8 * wave + i;
        typename TR::vec bop[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) bop[j] = TR::dequant8(wq[i][j], dq[i >> 2][j]);
        const int c = st * 4 + kq;  // 16-byte chunk of the k-octet in the slice row
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const v4u av = *reinterpret_cast<const v4u*>(&smem[k3_swz(mb * 16 + c4, c)]);
            const typename TR::vec aop = __builtin_bit_cast(typename TR::vec, av);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (XF16)
                    acc[mb][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop[j], acc[mb][j], 0, 0, 0);
                else
                    acc[mb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop, bop[j], acc[mb][j], 0, 0, 0);
            }
        }
    };
    // A full slice gives every wave all 8 steps: that loop has no branch, so
    // the weight loads stay where they were issued and each step waits only
    // for its own (a load used only under a branch is moved into it and
    // waited for there in full).
    if (nst == 8) {
#pragma unroll
        for (int i = 0; i < 8; ++i) kstep(i);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (i < nst) kstep(i);  // uniform over the wave
    }
    __syncthreads();  // the activation slice is dead; its LDS takes the wave partials
    float* part = reinterpret_cast<float*>(smem);  // [wave][mb][j][256]
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            *reinterpret_cast<v4f*>(&part[((wave * MB + mb) * 4 + j) * 256 + lane * 4]) = acc[mb][j];
    __syncthreads();
    // Thread t sums entry e = t of each (mb, j) tile over the waves in order:
    // MFMA lane e/4, result e%4 -> row 4 (lane/16) + e%4, column 4 (lane%16) + j.
    const int el = t >> 2, ei = t & 3;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int o = (mb * 4 + j) * 256 + t;
            float v = part[o];
            v = v + part[(MB * 4) * 256 + o];
            v = v + part[2 * (MB * 4) * 256 + o];
            v = v + part[3 * (MB * 4) * 256 + o];
            const int m = mb * 16 + 4 * (el >> 4) + ei, n = n0 + 4 * (el & 15) + j;
            if (m < M && n < N) ws[((int64_t)slice * M + m) * N + n] = v;
        }
}

// out[m, n] = round(sum over slices s in order of ws[s, m, n]).
template <bool OF16>
__global__ void __launch_bounds__(256)
k3_reduce(const float* __restrict__ ws, void* __restrict__ out, int64_t MN, int S) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= MN) return;
    v4f v = *reinterpret_cast<const v4f*>(ws + i);
    for (int s = 1; s < S; ++s) {
        const v4f w = *reinterpret_cast<const v4f*>(ws + (int64_t)s * MN + i);
        v = v4f{v[0] + w[0], v[1] + w[1], v[2] + w[2], v[3] + w[3]};
    }
    uint16_t h[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
        h[k] = OF16 ? __builtin_bit_cast(uint16_t, (_Float16)v[k]) : (uint16_t)f32_to_bf16_rne(v[k]);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + i) =
        make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
}

// ----------------------------------------------------------------------------
// Decode-sized kernel in one launch (M <= 16 any K, M <= 32 with K <= 4096).  A workgroup of 16 waves
// owns 32 output columns over the whole K, so every output is finished inside
// the workgroup: no workspace, no second launch.
//  * Rounds: a round is one quantisation group (128 k = four 32-k steps) of
//    one wave; wave w takes groups w, w + 16, w + 32, ...  A pass is two
//    rounds per wave (4096 k for the workgroup); K beyond that runs further
//    passes in the same launch.
//  * Loads: every load of a pass is issued before any of its data is used,
//    in the order it is needed -- the rounds' scale and zero words, round 0's
//    activations and weights, then round 1's -- so the wave waits once per
//    round on an in-order queue instead of once per load.
//  * Weights: lane l (column slot c = l % 16, k-octet o = l / 16) loads the
//    two words of columns n0 + 2c, n0 + 2c + 1 of one qweight row per step
//    (non-temporal: read once).  Word j feeds the MFMA of column tile j,
//    whose column i is n0 + 2i + j.
//  * Activations: a round's rows (M x 128 k) are read in whole lines -- 16
//    lanes per row and round, 256 contiguous bytes -- into the wave's own
//    LDS slot, each row's 16-byte octets XOR-swizzled by the row, and read
//    back as MFMA A operands (rows past M repeat row M - 1; their results are
//    dropped).  Up to 16 rows, both rounds go through VGPRs and are written
//    octet-ordered (see below).  At 17..32 rows a round is 8 KiB per wave:
//    round 0 goes straight from memory into the slot (buffer load to LDS),
//    round 1 into VGPRs and into the slot once round 0 has been read.  No
//    workgroup barrier before the epilogue: each wave reads only its slot.
//  * Dequantisation by group: the MFMA B operand is the biased code
//    128 + q (bf16 0x4300 | q) or 1024 + q (fp16 0x6400 | q), exact; a
//    further MFMA with an all-ones B gives the activation sums X over the
//    same k.  For the four steps of one group the product is then
//        sum x (q - z - 1) s = s * (S - (bias + z + 1) X),
//    two fmas per output and group instead of a rounded dequantised weight
//    per code.  (The reference rounds each dequantised weight to the
//    activation dtype; this form omits that rounding, a difference far
//    inside the 1e-2 tolerance of a product the reference itself sums in a
//    nondeterministic split-K order.)  Codes come out of a word in the
//    order q0 q4 q1 q5 q2 q6 q3 q7, so activation octets are reordered the
//    same way (octet_order) before they meet the codes.
//  * Epilogue: each wave's fp32 tile goes to its own slot, then the 16 tiles
//    are added in wave order and rounded once (deterministic, no atomics).
// ----------------------------------------------------------------------------
constexpr int K3R_WAVES = 16;
constexpr int K3R_NB = 32;  // columns per workgroup

template <bool F16>
struct BiasCode;
template <>
struct BiasCode<false> {
    typedef v8bf vec;
    static constexpr uint32_t HI = 0x43004300u;  // bf16 128 in both halves
    static constexpr float BIAS = 128.0f;
    static constexpr uint32_t ONE = 0x3F803F80u;
    __device__ static inline float scale_of(uint16_t s_f16) {
        return bf16_to_f32(f32_to_bf16_rne((float)__builtin_bit_cast(_Float16, s_f16)));
    }
};
template <>
struct BiasCode<true> {
    typedef v8h vec;
    static constexpr uint32_t HI = 0x64006400u;  // fp16 1024 in both halves
    static constexpr float BIAS = 1024.0f;
    static constexpr uint32_t ONE = 0x3C003C00u;
    __device__ static inline float scale_of(uint16_t s_f16) { return (float)__builtin_bit_cast(_Float16, s_f16); }
};

// The eight biased codes of a qweight word in the order q0 q4 q1 q5 q2 q6 q3 q7.
template <bool F16>
__device__ __forceinline__ typename BiasCode<F16>::vec biased8(uint32_t w) {
    const uint32_t m = 0x000F000Fu, hi = BiasCode<F16>::HI;
    const v4u r = {(w & m) | hi, ((w >> 4) & m) | hi, ((w >> 8) & m) | hi, ((w >> 12) & m) | hi};
    return __builtin_bit_cast(typename BiasCode<F16>::vec, r);
}

// An activation octet x0..x7 (16-bit pairs) reordered to x0 x4 x1 x5 x2 x6 x3 x7.
__device__ __forceinline__ v4u octet_order(v4u v) {
    return v4u{__builtin_amdgcn_perm(v[2], v[0], 0x05040100u), __builtin_amdgcn_perm(v[2], v[0], 0x07060302u),
               __builtin_amdgcn_perm(v[3], v[1], 0x05040100u), __builtin_amdgcn_perm(v[3], v[1], 0x07060302u)};
}

// 16 bytes per lane from a buffer straight into LDS: lane l's bytes land at
// lds + 16 l (the address is wave-uniform).
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, off, 0, 0, 0);
}

// s_waitcnt immediate that waits until at most n vector-memory loads are
// outstanding (expcnt and lgkmcnt left at their maxima).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

template <int MR, bool MULTI, bool XF16, bool OF16>
__global__ void __launch_bounds__(K3R_WAVES * 64)
k3_rows(const uint16_t* __restrict__ x, const int32_t* __restrict__ qweight, const int32_t* __restrict__ qzeros,
        const uint16_t* __restrict__ scales, void* __restrict__ out, int M, int N, int K) {
    using BC = BiasCode<XF16>;
    using vec = typename BC::vec;
    constexpr int NWV = K3R_WAVES, NT = 2, MB = MR > 16 ? 2 : 1;
    constexpr bool DMA = MR > 16;                     // round 0 straight into LDS
    constexpr int MRL = MR < 4 ? 4 : MR;              // rows laid out per slot (whole 1 KiB loads)
    constexpr int LA = MRL / 4;                       // activation loads per lane and round
    constexpr int SLOT = MRL * 256;                   // one round of activations
    constexpr int PART = MB * NT * 1024;              // a wave's fp32 tiles
    constexpr int REG = (DMA ? SLOT : 2 * SLOT) > PART ? (DMA ? SLOT : 2 * SLOT) : PART;
    extern __shared__ __align__(16) uint8_t smem[];
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int c = lane & 15, o = lane >> 4;
    const int n0 = blockIdx.x * K3R_NB;
    const int ncol = min(n0 + NT * c, N - NT);  // slots beyond N load the last valid columns (results dropped)
    const int G128 = K >> 7;
    // Buffer resources: offsets with bit 31 set are out of range and read nothing.
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x), (short)0, (int)((uint32_t)M * K * 2u), K3_RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(qweight), (short)0, (int)((uint32_t)(K >> 3) * N * 4u), K3_RSRC_WORD3);
    uint8_t* reg = smem + wave * REG;
    const vec ones = __builtin_bit_cast(vec, v4u{BC::ONE, BC::ONE, BC::ONE, BC::ONE});
    const int zsh = 4 * (ncol & 7);
    const int row_a = lane >> 4;  // activation load: row 4 i + row_a, octet (lane % 16) ^ row
    v4f total[MB][NT];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < NT; ++j) total[mb][j] = v4f{0.f, 0.f, 0.f, 0.f};

    // Two rounds per pass, all loads of both issued up front.  Several passes
    // (K > 4096) only up to 16 rows: at 17..32 rows the pass loop's live state
    // beside round 1's staging would spill.
    static_assert(!(MULTI && DMA), "17..32 rows take K <= 4096 (one pass)");
    constexpr int RPP = 2;
    const int passes = MULTI ? (G128 + RPP * NWV - 1) / (RPP * NWV) : 1;  // MULTI false: K <= 4096
    for (int p = 0; p < passes; ++p) {
        int g[RPP];
        uint32_t dead[RPP], aoff[RPP][LA], woff[RPP][4];
#pragma unroll
        for (int r = 0; r < RPP; ++r) {
            const int gr = (RPP * p + r) * NWV + wave;
            dead[r] = (uint32_t)(gr >= G128) << 31;  // rounds past K read nothing and add nothing
            g[r] = min(gr, G128 - 1);
            if constexpr (!DMA) {
#pragma unroll
                for (int i = 0; i < LA; ++i) {
                    const int row = 4 * i + row_a, oc = (lane & 15) ^ (row & 15);
                    aoff[r][i] = (((uint32_t)row * K + g[r] * 128 + oc * 8) * 2u) | dead[r] |
                                 ((uint32_t)(row >= M) << 31);
                }
                const uint32_t w0 = (uint32_t)((g[r] * 16 + o) * N + ncol) * 4u;
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) woff[r][s2] = (w0 + (uint32_t)s2 * 16u * (uint32_t)N) | dead[r];
            }
        }
        // ---- loads, issued before any of their data is used; offsets are
        // computed ahead of them (no address arithmetic between the loads)
        uint32_t sw[RPP], zw[RPP];
        v4u xa[RPP][LA];
        uint32_t wq[RPP][4][NT];
        auto load_sz = [&]() {
#pragma unroll
            for (int r = 0; r < RPP; ++r) {
                sw[r] = *reinterpret_cast<const uint32_t*>(scales + (int64_t)g[r] * N + ncol);
                zw[r] = (uint32_t)qzeros[(int64_t)g[r] * (N >> 3) + (ncol >> 3)];
            }
        };
        auto load_w = [&](int r) {
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2) {
                const auto v = __builtin_amdgcn_raw_buffer_load_b64(rw, (int)woff[r][s2], 0, 2);
                wq[r][s2][0] = v[0];
                wq[r][s2][1] = v[1];
            }
        };
        if constexpr (!DMA) {
            // up to 16 rows: the activations of both rounds (hot in L2, shared by every
            // workgroup), the scale/zero words, then the weights
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < RPP; ++r)
#pragma unroll
                for (int i = 0; i < LA; ++i)
                    xa[r][i] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)aoff[r][i], 0, 0));
            load_sz();
#pragma unroll
            for (int r = 0; r < RPP; ++r) load_w(r);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < RPP; ++r)
#pragma unroll
                for (int i = 0; i < LA; ++i)
                    *reinterpret_cast<v4u*>(reg + r * SLOT + (4 * i + row_a) * 256 + ((lane & 15) << 4)) =
                        octet_order(xa[r][i]);
        } else {
            // 17..32 rows: scale/zero words, then per round its activations and
            // weights (offsets of a round computed just before its loads)
            load_sz();
#pragma unroll
            for (int r = 0; r < RPP; ++r) {
#pragma unroll
                for (int i = 0; i < LA; ++i) {
                    const int row = 4 * i + row_a, oc = (lane & 15) ^ (row & 15);
                    aoff[r][i] = (((uint32_t)row * K + g[r] * 128 + oc * 8) * 2u) | dead[r] |
                                 ((uint32_t)(row >= M) << 31);
                }
                const uint32_t w0 = (uint32_t)((g[r] * 16 + o) * N + ncol) * 4u;
#pragma unroll
                for (int s2 = 0; s2 < 4; ++s2) woff[r][s2] = (w0 + (uint32_t)s2 * 16u * (uint32_t)N) | dead[r];
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < LA; ++i) {
                    if (r == 0)
                        load_lds16(rx, reg + i * 1024, aoff[r][i]);
                    else
                        xa[r][i] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)aoff[r][i], 0, 0));
                }
                load_w(r);
                __builtin_amdgcn_sched_barrier(0);
            }
            // round 0 in (the load to LDS included): round 1's loads may still be out
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(LA + 4));
        }
#pragma unroll
        for (int r = 0; r < RPP; ++r) {
            uint8_t* slot = reg + (DMA ? 0 : r * SLOT);
            const bool raw = DMA && r == 0;  // written by the load itself: octets still in memory order
            if (DMA && r == 1) {
                // round 1 through VGPRs: octet-ordered into the slot after round 0's reads
                // (a wave's LDS operations complete in order)
#pragma unroll
                for (int i = 0; i < LA; ++i)
                    *reinterpret_cast<v4u*>(slot + (4 * i + row_a) * 256 + ((lane & 15) << 4)) = octet_order(xa[r][i]);
            }
            float sj[NT], cj[NT];
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                sj[j] = BC::scale_of((uint16_t)(sw[r] >> (16 * j)));
                cj[j] = BC::BIAS + (float)((zw[r] >> (zsh + 4 * j)) & 15u) + 1.0f;
            }
            v4f S[MB][NT], X[MB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                X[mb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < NT; ++j) S[mb][j] = v4f{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int s2 = 0; s2 < 4; ++s2) {
                const int oc = 4 * s2 + o;
                vec b[NT];
#pragma unroll
                for (int j = 0; j < NT; ++j) b[j] = biased8<XF16>(wq[r][s2][j]);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    const int mr = min(mb * 16 + c, M - 1);
                    v4u av = *reinterpret_cast<const v4u*>(slot + mr * 256 + ((oc ^ (mr & 15)) << 4));
                    if (raw) av = octet_order(av);
                    const vec a = __builtin_bit_cast(vec, av);
#pragma unroll
                    for (int j = 0; j < NT; ++j) {
                        if constexpr (XF16)
                            S[mb][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[j], S[mb][j], 0, 0, 0);
                        else
                            S[mb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[j], S[mb][j], 0, 0, 0);
                    }
                    if constexpr (XF16)
                        X[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ones, X[mb], 0, 0, 0);
                    else
                        X[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ones, X[mb], 0, 0, 0);
                }
            }
            // total += s * (S - (bias + z + 1) X) over the round's group (rounds past K add nothing)
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int j = 0; j < NT; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float v = __builtin_fmaf(sj[j], __builtin_fmaf(-cj[j], X[mb][e], S[mb][j][e]),
                                                       total[mb][j][e]);
                        total[mb][j][e] = dead[r] ? total[mb][j][e] : v;
                    }
        }
        // the next pass writes the slots again (a load to LDS does not wait for this wave's reads)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(63) & ~(15 << 8));
        __builtin_amdgcn_sched_barrier(0);
    }
    // ---- epilogue: the wave's tiles into its own region, then the 16 tiles in wave order
    float* part = reinterpret_cast<float*>(reg);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < NT; ++j) *reinterpret_cast<v4f*>(&part[(mb * NT + j) * 256 + lane * 4]) = total[mb][j];
    __syncthreads();
    // Entry e of tile (mb, j): MFMA lane e/4, result e%4 -> row 16 mb + 4 (lane/16) + e%4,
    // column n0 + 2 (lane%16) + j.
    constexpr int ENT = MB * NT * 256, T = NWV * 64;
#pragma unroll
    for (int e0 = 0; e0 < ENT; e0 += T) {
        const int e = e0 + t;
        if (e < ENT) {
            const int tile = e >> 8, el = (e & 255) >> 2, ei = e & 3;
            const int mb = tile / NT, j = tile % NT;
            float v = reinterpret_cast<const float*>(smem)[e];
#pragma unroll
            for (int w = 1; w < NWV; ++w) v = v + reinterpret_cast<const float*>(smem + w * REG)[e];
            const int m = mb * 16 + 4 * (el >> 4) + ei, n = n0 + NT * (el & 15) + j;
            if (m < M && n < N) {
                const uint16_t h = OF16 ? __builtin_bit_cast(uint16_t, (_Float16)v) : (uint16_t)f32_to_bf16_rne(v);
                static_cast<uint16_t*>(out)[(int64_t)m * N + n] = h;
            }
        }
    }
}

template <int MR, bool XF, bool OF>
hipError_t launch_rows(const void* x, const int32_t* qw, const int32_t* qz, const void* sc, void* out, int M, int N,
                       int K, hipStream_t st) {
    constexpr int MB = MR > 16 ? 2 : 1, MRL = MR < 4 ? 4 : MR, SLOT = MRL * 256, PART = MB * 2 * 1024;
    constexpr int REG = (MR > 16 ? SLOT : 2 * SLOT) > PART ? (MR > 16 ? SLOT : 2 * SLOT) : PART;
    const dim3 grid((unsigned)((N + K3R_NB - 1) / K3R_NB)), block(K3R_WAVES * 64);
    if (K <= 2 * K3R_WAVES * 128) {
        hipLaunchKernelGGL((k3_rows<MR, false, XF, OF>), grid, block, K3R_WAVES * REG, st,
                           static_cast<const uint16_t*>(x), qw, qz, static_cast<const uint16_t*>(sc), out, M, N, K);
    } else {
        if constexpr (MR > 16) return hipErrorInvalidValue;  // one_launch_fits keeps 17..32 rows at K <= 4096
        else
            hipLaunchKernelGGL((k3_rows<MR, true, XF, OF>), grid, block, K3R_WAVES * REG, st,
                               static_cast<const uint16_t*>(x), qw, qz, static_cast<const uint16_t*>(sc), out, M, N, K);
    }
    return hipGetLastError();
}

// Whether the one-launch kernel serves this shape: the weight under 2 GiB (so
// every 32-bit buffer offset, with its out-of-range bit, is exact) and M <= 16,
// or M <= 32 with K <= 4096 and at most one workgroup per CU.  Every workgroup
// reads all M x K activations, so at 17..32 rows a longer K (down: 12288) or
// several workgroups per CU (gate/up: 768) read more per CU than the split-K
// form, which measured faster there (down at M = 32: 17.6 us against 21.4).
bool one_launch_fits(int64_t M, int64_t N, int64_t K) {
    if (M > 32 || K * N / 2 >= (1LL << 31)) return false;
    return M <= 16 || (K <= 2 * K3R_WAVES * 128 && (N + K3R_NB - 1) / K3R_NB <= device_cu_count());
}

template <bool XF, bool OF>
hipError_t dispatch_rows(const void* x, const int32_t* qw, const int32_t* qz, const void* sc, void* out, int M, int N,
                         int K, hipStream_t st) {
    if (M <= 2) return launch_rows<2, XF, OF>(x, qw, qz, sc, out, M, N, K, st);
    if (M <= 4) return launch_rows<4, XF, OF>(x, qw, qz, sc, out, M, N, K, st);
    if (M <= 8) return launch_rows<8, XF, OF>(x, qw, qz, sc, out, M, N, K, st);
    if (M <= 16) return launch_rows<16, XF, OF>(x, qw, qz, sc, out, M, N, K, st);
    return launch_rows<32, XF, OF>(x, qw, qz, sc, out, M, N, K, st);
}

template <int MB, bool XF, bool OF>
hipError_t launch_dec(const void* x, const int32_t* qw, const int32_t* qz, const void* sc, void* out, float* ws,
                      int M, int N, int K, hipStream_t st) {
    const int S = (K + K3_KS - 1) / K3_KS;
    hipLaunchKernelGGL((k3_dec<MB, XF>), dim3((unsigned)((N + K3_NB - 1) / K3_NB), (unsigned)S), dim3(256), 0, st,
                       static_cast<const uint16_t*>(x), qw, qz, static_cast<const uint16_t*>(sc), ws, M, N, K);
    const int64_t MN = (int64_t)M * N;  // N % 8 == 0, so MN % 4 == 0
    hipLaunchKernelGGL((k3_reduce<OF>), dim3((unsigned)((MN / 4 + 255) / 256)), dim3(256), 0, st, ws, out, MN, S);
    return hipGetLastError();
}

template <bool XF, bool OF>
hipError_t dispatch_dec(const void* x, const int32_t* qw, const int32_t* qz, const void* sc, void* out, float* ws,
                        int M, int N, int K, hipStream_t st) {
    if (M <= 16) return launch_dec<1, XF, OF>(x, qw, qz, sc, out, ws, M, N, K, st);
    if (M <= 32) return launch_dec<2, XF, OF>(x, qw, qz, sc, out, ws, M, N, K, st);
    if (M <= 48) return launch_dec<3, XF, OF>(x, qw, qz, sc, out, ws, M, N, K, st);
    return launch_dec<4, XF, OF>(x, qw, qz, sc, out, ws, M, N, K, st);
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

// ----------------------------------------------------------------------------
// Dequantization to a dense [K, N] weight for prefill-sized M (the product
// then runs as a plain library GEMM).  Thread = one qweight row segment of 8
// columns (8 words, 32 bytes): it writes the 8 k-rows of those columns, 16
// bytes per row, with the same per-element rounding as the GEMM kernels:
// w[k][n] = cvt(float(q - z - 1) * scale).
// ----------------------------------------------------------------------------
template <bool F16>
__global__ void __launch_bounds__(256)
w4a16_dequant(const int32_t* __restrict__ qweight, const int32_t* __restrict__ qzeros,
              const uint16_t* __restrict__ scales, uint16_t* __restrict__ w, int N, int K) {
    using TR = W16Traits<F16>;
    const int nb = N >> 3;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)(K >> 3) * nb) return;
    const int k8 = (int)(idx / nb), c8 = (int)(idx % nb);
    const int n0 = c8 * 8, g = k8 >> 4;  // 16 qweight rows per 128-deep group
    const v4u q0 = *reinterpret_cast<const v4u*>(qweight + (int64_t)k8 * N + n0);
    const v4u q1 = *reinterpret_cast<const v4u*>(qweight + (int64_t)k8 * N + n0 + 4);
    const uint32_t zw = (uint32_t)qzeros[(int64_t)g * nb + c8];
    const v4u sv = *reinterpret_cast<const v4u*>(scales + (int64_t)g * N + n0);
    const uint32_t qw[8] = {q0[0], q0[1], q0[2], q0[3], q1[0], q1[1], q1[2], q1[3]};
    float sc[8];
    int zp1[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        sc[j] = TR::scale_of((uint16_t)(sv[j >> 1] >> (16 * (j & 1))));
        zp1[j] = (int)((zw >> (4 * j)) & 15u) + 1;
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        uint32_t h[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = TR::cvt((float)((int)((qw[j] >> (4 * r)) & 15u) - zp1[j]) * sc[j]);
        const v4u o = {h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
        *reinterpret_cast<v4u*>(w + (int64_t)(8 * k8 + r) * N + n0) = o;
    }
}

}  // namespace
}  // namespace nv4

extern "C" int nv4_w4a16_dequant(const int32_t* qweight, const int32_t* qzeros, const void* scales, void* w,
                                 int w_dtype, int64_t N, int64_t K, int group, void* stream) {
    using namespace nv4;
    if (!qweight || !qzeros || !scales || !w) return NV4_E_NULL;
    if (w_dtype != NV4_BF16 && w_dtype != NV4_FP16) return NV4_E_DTYPE;
    if (group != 128) return NV4_E_GROUP;
    if (N < 8 || N % 8 || K < 128 || K % 128 || N > 0x7fffffffLL || K > (1LL << 24)) return NV4_E_SHAPE;
    const int64_t threads = (K / 8) * (N / 8);
    if ((threads + 255) / 256 > 0x7fffffffLL) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(qweight) % 16 || reinterpret_cast<uintptr_t>(qzeros) % 4 ||
        reinterpret_cast<uintptr_t>(scales) % 16 || reinterpret_cast<uintptr_t>(w) % 16)
        return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid((unsigned)((threads + 255) / 256));
    if (w_dtype == NV4_FP16)
        hipLaunchKernelGGL((w4a16_dequant<true>), grid, dim3(256), 0, st, qweight, qzeros,
                           static_cast<const uint16_t*>(scales), static_cast<uint16_t*>(w), (int)N, (int)K);
    else
        hipLaunchKernelGGL((w4a16_dequant<false>), grid, dim3(256), 0, st, qweight, qzeros,
                           static_cast<const uint16_t*>(scales), static_cast<uint16_t*>(w), (int)N, (int)K);
    return (int)hipGetLastError();
}

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
    // Decode batches: the one-launch kernel (8-byte weight and 4-byte scale loads).
    if (one_launch_fits(M, N, K) && reinterpret_cast<uintptr_t>(qweight) % 8 == 0 &&
        reinterpret_cast<uintptr_t>(scales) % 4 == 0) {
        if (x_dtype == NV4_FP16)
            e = out_dtype == NV4_FP16 ? dispatch_rows<true, true>(x, qweight, qzeros, scales, out, m, n, k, st)
                                      : dispatch_rows<true, false>(x, qweight, qzeros, scales, out, m, n, k, st);
        else
            e = out_dtype == NV4_FP16 ? dispatch_rows<false, true>(x, qweight, qzeros, scales, out, m, n, k, st)
                                      : dispatch_rows<false, false>(x, qweight, qzeros, scales, out, m, n, k, st);
        return (int)e;
    }
    if (x_dtype == NV4_FP16)
        e = out_dtype == NV4_FP16 ? dispatch<true, true>(x, qweight, qzeros, scales, out, m, n, k, st)
                                  : dispatch<true, false>(x, qweight, qzeros, scales, out, m, n, k, st);
    else
        e = out_dtype == NV4_FP16 ? dispatch<false, true>(x, qweight, qzeros, scales, out, m, n, k, st)
                                  : dispatch<false, false>(x, qweight, qzeros, scales, out, m, n, k, st);
    return (int)e;
}

extern "C" int nv4_w4a16_gemm_ws(const void* x, int x_dtype, const int32_t* qweight, const int32_t* qzeros,
                                 const void* scales, void* out, int out_dtype, float* workspace,
                                 int64_t workspace_bytes, int64_t M, int64_t N, int64_t K, int group, void* stream) {
    using namespace nv4;
    if (M > 64) return nv4_w4a16_gemm(x, x_dtype, qweight, qzeros, scales, out, out_dtype, M, N, K, group, stream);
    if (!x || !qweight || !qzeros || !scales || !out || !workspace) return NV4_E_NULL;
    if ((x_dtype != NV4_BF16 && x_dtype != NV4_FP16) || (out_dtype != NV4_BF16 && out_dtype != NV4_FP16))
        return NV4_E_DTYPE;
    if (group != 128) return NV4_E_GROUP;
    if (M < 1 || N < 8 || N % 8 || K < 128 || K % 128 || N > 0x7fffffffLL || K > (1LL << 24)) return NV4_E_SHAPE;
    const int64_t S = (K + K3_KS - 1) / K3_KS;
    if (workspace_bytes < S * M * N * 4 || (N + K3_NB - 1) / K3_NB > 0x7fffffffLL || S > 65535) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(qweight) % 16 ||
        reinterpret_cast<uintptr_t>(qzeros) % 4 || reinterpret_cast<uintptr_t>(scales) % 8 ||
        reinterpret_cast<uintptr_t>(out) % 8 || reinterpret_cast<uintptr_t>(workspace) % 16)
        return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int m = (int)M, n = (int)N, k = (int)K;
    hipError_t e;
    if (x_dtype == NV4_FP16)
        e = out_dtype == NV4_FP16 ? dispatch_dec<true, true>(x, qweight, qzeros, scales, out, workspace, m, n, k, st)
                                  : dispatch_dec<true, false>(x, qweight, qzeros, scales, out, workspace, m, n, k, st);
    else
        e = out_dtype == NV4_FP16 ? dispatch_dec<false, true>(x, qweight, qzeros, scales, out, workspace, m, n, k, st)
                                  : dispatch_dec<false, false>(x, qweight, qzeros, scales, out, workspace, m, n, k, st);
    return (int)e;
}
