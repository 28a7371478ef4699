// K2, prefill-sized M, on the fp6 matrix cores: grouped W4A4 INT4 GEMM with
// the INT4 codes carried as fp6 (e3m2) values.
//
// Numerical contract (nanovllm/kernels/w4a4_grouped_kernel.py:64-90, oracle
// benchmarks/verify_w4a4_aw_grouped.py:13-29), bit for bit: for g in order,
//   total = fmaf(float(dot_g), float(sa[m,g]) * float(sw[n,g]), total)
// (per-channel weight scales: total = fmaf(float(dot_g), sa[m,g], total),
// C = bf16(total * sw[n])), then C = bf16_rne(total) or the fp32 total.
//
// e3m2 (sign, 3 exponent bits with bias 3, 2 mantissa bits) holds every
// integer of [-8, 8] exactly: 1, 2, 4, 8 as powers of two, 3 = 2 * 1.5,
// 5, 6, 7 = 4 * 1.25, 1.5, 1.75.  Products of two codes are integers of
// magnitude <= 64 and the partial sums of a 128-deep group integers of
// magnitude <= 8192, exact in fp32 in any order: with unit E8M0 scales,
// v_mfma_scale_f32_32x32x64_f8f6f4 (A and B format 3, e3m2) returns each
// group dot exactly, at twice the fp8 rate, from 6-bit operands (a quarter
// fewer bytes to stage than fp8).  The scale product sa * sw comes from a
// bf16 MFMA as in the fp8 kernel; one VALU fma per output and group remains.
//
// Operand format (written by i4_to_f6_tiles into the caller's workspace, or
// for weights converted once by nv4_w4a4_weights_to_f6): rows in tiles of 128; per tile and group one 12 KiB block laid out as LDS
// reads it.  A group row's 128 codes are four quarters of 32 (k = 32q ..
// 32q + 31, 24 bytes each, code k at bit 6k of the quarter, little endian),
// and each quarter is split into its first 16 bytes (P) and last 8 (R):
//   P[q][row] at q * 2048 + row * 16,  R[q][row] at 8192 + q * 1024 + row * 8.
// A block moves global -> LDS as twelve contiguous 1 KiB pieces (buffer
// loads writing LDS directly), and an operand read -- lane (rc, h) of a
// 32-row block in k-step s takes quarter 2h + s of row rc: one 16-byte and
// one 8-byte read -- touches consecutive LDS addresses across the lanes,
// free of bank conflicts.  MFMA 32x32x64, 6-bit formats: lane l supplies
// row (A) / column (W) l%32 and 32 codes (six registers, code i at bit 6i);
// A and W read the same quarters, so every product pairs equal k.  Result
// layout as fp8: lane l holds C[8*(i/4) + 4*(l/32) + i%4][l%32], i = 0..15.
//
// Workgroup = 4 waves, 128 x 128 output tile, whole K, two workgroups per
// CU, XCD-aware tile order, a two-stage operand ring with one barrier per
// group and the bf16 scales in 8-group windows (as the fp8 kernel).
#include "nv4_common.h"

namespace nv4 {
namespace {

constexpr int F6_BM = 128, F6_BN = 128, F6_T = 256;
constexpr int F6_BLOCK = 12 * 1024;                     // one operand tile, one group
constexpr int F6_R = 8192;                              // R part of a block
constexpr int F6_STAGE = 2 * F6_BLOCK;                  // A block then W block
constexpr int F6_WSZ = 8 * (F6_BM + F6_BN) * 2;         // 8 groups x (sa[128], sw[128]) bf16
static_assert(2 * F6_STAGE + 2 * F6_WSZ == 56 * 1024, "56 KiB of LDS: two workgroups per CU");
constexpr int F6_GM = 8;                                // M-tiles per column sweep
constexpr int F6_RSRC_WORD3 = 0x00020000;               // buffer resource word 3 (CDNA): 32-bit data format
constexpr int F6_FMT = 3;                               // f8f6f4 operand format: e3m2

typedef int v8i __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void* lds_ptr;

// e3m2 codes of the INT4 values: nibble n (two's complement) -> code byte.
// Four nibbles (one per byte, values 0..15) at a time: two 8-entry byte
// lookups (v_perm) for n < 8 and n >= 8, merged by bit 3.
__device__ __forceinline__ uint32_t nib4_to_e3m2(uint32_t x) {
    const uint32_t sel = x & 0x07070707u;
    const uint32_t pos = __builtin_amdgcn_perm(0x17161514u, 0x12100C00u, sel);  //  0  1  2  3  4  5  6  7
    const uint32_t neg = __builtin_amdgcn_perm(0x2C303234u, 0x35363738u, sel);  // -8 -7 -6 -5 -4 -3 -2 -1
    const uint32_t m = ((x >> 3) & 0x01010101u) * 0xFFu;
    return (neg & m) | (pos & ~m);
}

// One packed dword (8 codes: byte j holds k = 2j low nibble, 2j + 1 high) ->
// 48 bits, code k at bit 6k.
__device__ __forceinline__ uint64_t packed4_to_e3m2(uint32_t d) {
    const uint32_t clo = nib4_to_e3m2(d & 0x0F0F0F0Fu);         // k = 0, 2, 4, 6
    const uint32_t chi = nib4_to_e3m2((d >> 4) & 0x0F0F0F0Fu);  // k = 1, 3, 5, 7
    // 12-bit pairs in 16-bit lanes: ev = (k0 k1, k4 k5), od = (k2 k3, k6 k7)
    const uint32_t ev = (clo & 0x00FF00FFu) | ((chi & 0x00FF00FFu) << 6);
    const uint32_t od = ((clo >> 8) & 0x00FF00FFu) | (((chi >> 8) & 0x00FF00FFu) << 6);
    return (uint64_t)(ev & 0xFFFu) | ((uint64_t)(od & 0xFFFu) << 12) | ((uint64_t)(ev >> 16) << 24) |
           ((uint64_t)(od >> 16) << 36);
}

// Packed INT4 rows -> fp6 tile blocks, both operands in one launch.  Thread u
// converts one quarter (16 packed bytes, 32 codes) of one group row: u =
// ((tile * G + g) * 128 + row) * 4 + q, A tiles first, then W tiles, so four
// consecutive lanes read one row's 64 contiguous group bytes (and a wave the
// whole 1 KiB block of a tiled weight group) and a wave's stores are four
// contiguous runs of P and of R.  A is in
// the reference layout [M][K/2]; W in the reference layout or, with W_TILED,
// the MFMA-tiled one ([N/16][G][64 lanes][16 bytes], lane l holding packed
// bytes 64g + 16(l/16) .. +15 of row 16cb + l%16).  Rows past the matrix
// edge repeat its last row (their results are never stored).  Either half
// may be empty: ua = 0 converts weights only, uw = 0 activations only (the
// threads past A then return without touching w6).
template <bool W_TILED>
__global__ void __launch_bounds__(256)
i4_to_f6_tiles(const int8_t* __restrict__ a, uint8_t* __restrict__ a6, int64_t ua, int M, const int8_t* __restrict__ w,
               uint8_t* __restrict__ w6, int64_t uw, int N, int G, int K) {
    int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool is_a = u < ua;
    if (!is_a) u -= ua;
    if (!is_a && u >= uw) return;
    const int q = (int)(u & 3), r = (int)((u >> 2) & 127);
    const int64_t tg = u >> 9;
    const int g = (int)(tg % G);
    const int64_t tile = tg / G;
    const int64_t row = min(tile * 128 + r, (int64_t)(is_a ? M : N) - 1);
    const int8_t* src;
    if (!is_a && W_TILED)
        src = w + (((row >> 4) * G + g) * 64 + (row & 15) + 16 * q) * 16;
    else
        src = (is_a ? a : w) + row * (K >> 1) + 64 * g + 16 * q;
    const v4u v = *reinterpret_cast<const v4u*>(src);
    const uint64_t x0 = packed4_to_e3m2(v[0]), x1 = packed4_to_e3m2(v[1]);
    const uint64_t x2 = packed4_to_e3m2(v[2]), x3 = packed4_to_e3m2(v[3]);
    const v4u p = {(uint32_t)x0, (uint32_t)((x0 >> 32) | (x1 << 16)), (uint32_t)(x1 >> 16), (uint32_t)x2};
    uint2 rr;
    rr.x = (uint32_t)((x2 >> 32) | (x3 << 16));
    rr.y = (uint32_t)(x3 >> 16);
    uint8_t* blk = (is_a ? a6 : w6) + tg * F6_BLOCK;
    *reinterpret_cast<v4u*>(blk + q * 2048 + r * 16) = p;
    *reinterpret_cast<uint2*>(blk + F6_R + q * 1024 + r * 8) = rr;
}

// Tile order: linear workgroup ids are dealt round-robin over the 8 XCDs, so
// ids b, b + 8, ... share an L2; consecutive ids of one XCD sweep a band of
// F6_GM M-tiles down each column of N-tiles (the band's A tiles and one W
// tile stay hot in that L2).
__device__ __forceinline__ void f6_tile(int tm, int tn, int& mt, int& nt) {
    const int T = tm * tn;
    const int b = blockIdx.x;
    const int t = (T & 7) == 0 ? (b & 7) * (T >> 3) + (b >> 3) : b;
    const int per = F6_GM * tn;
    const int grp = t / per;
    const int first = grp * F6_GM;
    const int gm = min(tm - first, F6_GM);
    const int r = t - grp * per;
    mt = first + r % gm;
    nt = r / gm;
}

template <bool SG, bool OF, bool WIN>
__global__ void __launch_bounds__(F6_T, 2)
k2_prefill_f6(const uint8_t* __restrict__ a, const uint8_t* __restrict__ w, const uint16_t* __restrict__ sa,
              const uint16_t* __restrict__ sw, void* __restrict__ out, int M, int N, int K, int tm, int tn) {
    // Two operand stages (A block then W block) and the scales (8-group
    // windows, or one slot per group), as separate arrays so that reads of
    // one stage are not ordered behind the direct-to-LDS loads in flight into
    // the other.
    __shared__ __align__(16) uint8_t st0[F6_STAGE];
    __shared__ __align__(16) uint8_t st1[F6_STAGE];
    __shared__ __align__(16) uint16_t win[WIN ? F6_WSZ : 2 * (F6_BM + F6_BN)];
    int mt, nt;
    f6_tile(tm, tn, mt, nt);
    const int m0 = mt * F6_BM, n0 = nt * F6_BN;
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int G = K >> 7;

    // Direct-to-LDS staging: load i (0..2) of wave w copies the 1 KiB at
    // (3w + i) * 1024 of the group's A block (then of its W block), lane l
    // the 16 bytes at l * 16.  Buffer resources over the tile's G blocks, so
    // the loads take a fixed lane offset and the group offset as a scalar.
    const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(a + (int64_t)mt * G * F6_BLOCK), (short)0, G * F6_BLOCK, F6_RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t rsw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(w + (int64_t)nt * G * F6_BLOCK), (short)0, G * F6_BLOCK, F6_RSRC_WORD3);
    const uint32_t offl = (uint32_t)(3 * wave * 1024 + lane * 16);
    auto dma = [&](int g, uint8_t* st) {
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_ptr)(st + (3 * wave + i) * 1024), 16, offl + i * 1024,
                                                     g * F6_BLOCK, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsw, (lds_ptr)(st + F6_BLOCK + (3 * wave + i) * 1024), 16,
                                                     offl + i * 1024, g * F6_BLOCK, 0, 0);
        }
    };
    // Scales: two windows of 8 groups, [group % 8][sa row 0..127, sw column
    // 0..127] bf16 (without windows -- scale pointers off a 16-byte boundary
    // or G not a multiple of 8 -- one slot per group, two groups ahead);
    // thread t < 128 moves the sa of tile row t, the others the sw of tile
    // column t-128 (per-channel form: an unused sa).
    const bool is_sa = t < F6_BM;
    const uint16_t* s_t = is_sa ? sa + (int64_t)m0 * G : (SG ? sw + (int64_t)n0 * G : sa + (int64_t)m0 * G);
    const uint32_t offs = (uint32_t)(is_sa ? min(t, M - 1 - m0) * G : (SG ? min(t - F6_BM, N - 1 - n0) * G : 0));
    auto slot = [&](int x) {
        return WIN ? win + ((x >> 3) & 1) * (F6_WSZ / 2) + (x & 7) * (F6_BM + F6_BN) : win + (x & 1) * (F6_BM + F6_BN);
    };
    uint32_t rs;
    v4u rwin;
    auto load_win = [&](int wi) { rwin = *reinterpret_cast<const v4u*>(s_t + offs + 8 * wi); };
    auto store_win = [&](int wi) {
#pragma unroll
        for (int gl = 0; gl < 8; ++gl) {
            const uint32_t h = (rwin[gl >> 1] >> (16 * (gl & 1))) & 0xffffu;
            slot(wi * 8 + gl)[t] = (uint16_t)h;
        }
    };

    // Operand reads: lane (rc, half) of the 32-row block at tile row b0, k-step s:
    // quarter q = 2 half + s of row b0 + rc, P at q*2048 + row*16, R at
    // 8192 + q*1024 + row*8.
    const int rc = lane & 31, half = lane >> 5;
    int op[2], orr[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int q = 2 * half + s;
        op[s] = q * 2048 + rc * 16;
        orr[s] = F6_R + q * 1024 + rc * 8;
    }
    float total[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) total[i][j][v] = 0.0f;

    v8i pa[2][2], pw[2][2];
    v16f acc[2];
    auto fetch = [&](const uint8_t* st) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const int ra = wm * 64 + i * 32, rw = wn * 64 + i * 32;
                const v4u a0 = *reinterpret_cast<const v4u*>(st + op[s] + ra * 16);
                const uint2 a1 = *reinterpret_cast<const uint2*>(st + orr[s] + ra * 8);
                const v4u w0 = *reinterpret_cast<const v4u*>(st + F6_BLOCK + op[s] + rw * 16);
                const uint2 w1 = *reinterpret_cast<const uint2*>(st + F6_BLOCK + orr[s] + rw * 8);
                pa[i][s] = v8i{(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1.x, (int)a1.y, 0, 0};
                pw[i][s] = v8i{(int)w0[0], (int)w0[1], (int)w0[2], (int)w0[3], (int)w1.x, (int)w1.y, 0, 0};
            }
    };
    // Blocks in the order (0,0), (0,1), (1,1), (1,0).
    auto mma = [&](int b) {
        const int i = b >> 1, j = (b ^ (b >> 1)) & 1;
        v16f c = {};
#pragma unroll
        for (int s = 0; s < 2; ++s)
            c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(pa[i][s], pw[j][s], c, F6_FMT, F6_FMT, 0, 127, 0,
                                                                127);
        acc[b & 1] = c;
    };
    // Scale products on the matrix cores: a product of two bf16 values has
    // at most 16 significant bits, so sa[m] * sw[n] is exact in fp32 unless
    // it falls below the normal range, and a bf16 MFMA whose only non-zero k
    // term is (sa[row], sw[column]) returns the fp32 product the reference
    // multiplies (sa alone, times bf16 1.0, for per-channel weight scales).
    // Scales whose products reach the fp32 subnormals are in the parity tests
    // and match the oracle bit for bit.  32x32x16 bf16 operands: lane l
    // supplies row / column l%32, k = 8(l/32) .. +7, so lanes 32..63 supply
    // zeros; the result has the layout of the fp6 dot.
    const uint32_t keep = half ? 0u : 0xffffu;
    uint32_t sab[2], swb[2];
    auto read_scales = [&](const uint16_t* sg) {
#pragma unroll
        for (int i = 0; i < 2; ++i) sab[i] = sg[wm * 64 + i * 32 + rc] & keep;
#pragma unroll
        for (int j = 0; j < 2; ++j) swb[j] = (SG ? (uint32_t)sg[F6_BM + wn * 64 + j * 32 + rc] : 0x3f80u) & keep;
    };
    v16f prod[2];
    auto pmma = [&](int b) {
        const int i = b >> 1, j = (b ^ (b >> 1)) & 1;
        const v4u av = {sab[i], 0u, 0u, 0u}, bv = {swb[j], 0u, 0u, 0u};
        prod[b & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, av),
                                                              __builtin_bit_cast(v8bf, bv), v16f{}, 0, 0, 0);
    };
    auto epi = [&](int b) {
        const int i = b >> 1, j = (b ^ (b >> 1)) & 1;
#pragma unroll
        for (int v = 0; v < 16; ++v) total[i][j][v] = __builtin_fmaf(acc[b & 1][v], prod[b & 1][v], total[i][j][v]);
    };
    // One group.  The explicit vmcnt(0) completes this wave's direct-to-LDS
    // loads before the barrier, so after it the whole stage of group g (and,
    // without windows, the scales of group g) is in LDS and the other stage is
    // free.  Every LDS read of the step is issued before the next group's
    // loads, so none of them waits on those.
    auto step = [&](int g, const uint8_t* st, uint8_t* st_next) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
        fetch(st);
        read_scales(slot(g));
        __builtin_amdgcn_sched_barrier(0);
        if (g + 1 < G) dma(g + 1, st_next);
        if constexpr (!WIN) {
            if (g + 1 < G) slot(g + 1)[t] = (uint16_t)rs;
            if (g + 2 < G) rs = (s_t + g + 2)[offs];
        }
        __builtin_amdgcn_sched_barrier(0);
        pmma(0);
        mma(0);
        pmma(1);
        mma(1);
        epi(0);
        pmma(2);
        mma(2);
        epi(1);
        pmma(3);
        mma(3);
        epi(2);
        epi(3);
        if constexpr (WIN) {
            if ((g & 7) == 3 && (g >> 3) + 1 < (G >> 3)) load_win((g >> 3) + 1);
            if ((g & 7) == 7 && (g >> 3) + 1 < (G >> 3)) store_win((g >> 3) + 1);
        }
    };

    if constexpr (WIN) {
        load_win(0);
        store_win(0);
    } else {
        slot(0)[t] = (s_t + 0)[offs];
        if (G > 1) rs = (s_t + 1)[offs];
    }
    dma(0, st0);
    for (int g = 0; g < G; g += 2) {
        step(g, st0, st1);
        if (g + 1 < G) step(g + 1, st1, st0);
    }

#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 64 + j * 32 + rc;
        float swn = 1.0f;
        if constexpr (!SG) swn = bf16_to_f32(sw[min(n, N - 1)]);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                if (m < M && n < N) {
                    float val = total[i][j][v];
                    if constexpr (!SG) val = val * swn;
                    if constexpr (OF)
                        static_cast<float*>(out)[(int64_t)m * N + n] = val;
                    else
                        static_cast<uint16_t*>(out)[(int64_t)m * N + n] = (uint16_t)f32_to_bf16_rne(val);
                }
            }
    }
}

template <bool SG, bool OF>
hipError_t launch_f6(const uint8_t* a6, const uint8_t* w6, const uint16_t* sa, const uint16_t* sw, void* out,
                     int M, int N, int K, hipStream_t st) {
    const int tm = (M + F6_BM - 1) / F6_BM, tn = (N + F6_BN - 1) / F6_BN;
    const bool win = (K / 128) % 8 == 0 && reinterpret_cast<uintptr_t>(sa) % 16 == 0 &&
                     (!SG || reinterpret_cast<uintptr_t>(sw) % 16 == 0);
    if (win)
        hipLaunchKernelGGL((k2_prefill_f6<SG, OF, true>), dim3((unsigned)(tm * tn)), dim3(F6_T), 0, st, a6, w6, sa,
                           sw, out, M, N, K, tm, tn);
    else
        hipLaunchKernelGGL((k2_prefill_f6<SG, OF, false>), dim3((unsigned)(tm * tn)), dim3(F6_T), 0, st, a6, w6, sa,
                           sw, out, M, N, K, tm, tn);
    return hipGetLastError();
}

}  // namespace
}  // namespace nv4

extern "C" int64_t nv4_w4a4_gemm_f6_workspace(int64_t M, int64_t N, int64_t K) {
    using namespace nv4;
    if (M < 1 || N < 1 || K < 128 || K % 128) return -1;
    return ((M + F6_BM - 1) / F6_BM + (N + F6_BN - 1) / F6_BN) * (K / 128) * (int64_t)F6_BLOCK;
}

extern "C" int64_t nv4_w4a4_weights_f6_bytes(int64_t N, int64_t K) {
    using namespace nv4;
    if (N < 1 || K < 128 || K % 128) return -1;
    return (N + F6_BN - 1) / F6_BN * (K / 128) * (int64_t)F6_BLOCK;
}

// Packed weights -> the fp6 tile blocks the GEMM reads (the W half of the
// per-call conversion), for weights converted once and kept.
extern "C" int nv4_w4a4_weights_to_f6(const int8_t* w, int w_tiled, uint8_t* w6, int64_t N, int64_t K,
                                      int64_t w6_bytes, void* stream) {
    using namespace nv4;
    if (!w || !w6) return NV4_E_NULL;
    if (N < 1 || K < 128 || K % 128 || N % 8 || (w_tiled != 0 && w_tiled != 1) || (w_tiled && N % 16))
        return NV4_E_SHAPE;
    if (N > 0x7fffffffLL || K > (1LL << 20)) return NV4_E_SHAPE;
    const int64_t G = K / 128, tn = (N + F6_BN - 1) / F6_BN;
    if (G * F6_BLOCK > 0x7fffffffLL || N * G > 0x7fffffffLL || tn * G * 512 > 0xffffff00LL) return NV4_E_SHAPE;
    if (w6_bytes < tn * G * F6_BLOCK) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(w) % 16 || reinterpret_cast<uintptr_t>(w6) % 16) return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int64_t uw = tn * G * 512;
    const unsigned cgrid = (unsigned)((uw + 255) / 256);
    if (w_tiled)
        hipLaunchKernelGGL(i4_to_f6_tiles<true>, dim3(cgrid), dim3(256), 0, st, nullptr, nullptr, (int64_t)0, 1, w,
                           w6, uw, (int)N, (int)G, (int)K);
    else
        hipLaunchKernelGGL(i4_to_f6_tiles<false>, dim3(cgrid), dim3(256), 0, st, nullptr, nullptr, (int64_t)0, 1, w,
                           w6, uw, (int)N, (int)G, (int)K);
    return (int)hipGetLastError();
}

extern "C" int nv4_w4a4_gemm_f6(const int8_t* a, const int8_t* w, int w_form, const void* sa, const void* sw,
                                int sw_grouped, void* out, int out_fp32, int64_t M, int64_t N, int64_t K,
                                void* workspace, int64_t workspace_bytes, void* stream) {
    using namespace nv4;
    if (!a || !w || !sa || !sw || !out || !workspace) return NV4_E_NULL;
    if (w_form < 0 || w_form > 2) return NV4_E_SHAPE;
    if (M < 1 || N < 1 || K < 128 || K % 128 || N % 8 || (w_form == 1 && N % 16)) return NV4_E_SHAPE;
    if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > (1LL << 20)) return NV4_E_SHAPE;
    const int64_t G = K / 128;
    const int64_t tm = (M + F6_BM - 1) / F6_BM, tn = (N + F6_BN - 1) / F6_BN;
    // Buffer resources span one tile's G blocks (32-bit range); dispatch grids
    // count work-items in 32 bits: the conversion launches one per quarter
    // group row of both padded operands, the GEMM 256 per output tile.
    if (G * F6_BLOCK > 0x7fffffffLL || M * G > 0x7fffffffLL || N * G > 0x7fffffffLL) return NV4_E_SHAPE;
    if (tm * tn * F6_T > 0xffffffffLL || (tm + tn) * G * 512 > 0xffffff00LL) return NV4_E_SHAPE;
    // Weights already in fp6 tiles (w_form 2) need workspace for A only.
    if (workspace_bytes < (w_form == 2 ? tm : tm + tn) * G * F6_BLOCK) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(a) % 16 || reinterpret_cast<uintptr_t>(w) % 16 ||
        reinterpret_cast<uintptr_t>(sa) % 2 || reinterpret_cast<uintptr_t>(sw) % 2 ||
        reinterpret_cast<uintptr_t>(out) % (out_fp32 ? 4 : 2) || reinterpret_cast<uintptr_t>(workspace) % 16)
        return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint8_t* a6 = static_cast<uint8_t*>(workspace);
    const bool w_ready = w_form == 2;
    uint8_t* w6 = w_ready ? const_cast<uint8_t*>(reinterpret_cast<const uint8_t*>(w)) : a6 + tm * G * F6_BLOCK;
    const int64_t ua = tm * G * 512, uw = w_ready ? 0 : tn * G * 512;
    const unsigned cgrid = (unsigned)((ua + uw + 255) / 256);
    if (w_form == 1)
        hipLaunchKernelGGL(i4_to_f6_tiles<true>, dim3(cgrid), dim3(256), 0, st, a, a6, ua, (int)M, w, w6, uw, (int)N,
                           (int)G, (int)K);
    else
        hipLaunchKernelGGL(i4_to_f6_tiles<false>, dim3(cgrid), dim3(256), 0, st, a, a6, ua, (int)M, w, w6, uw,
                           (int)N, (int)G, (int)K);
    const auto* sap = static_cast<const uint16_t*>(sa);
    const auto* swp = static_cast<const uint16_t*>(sw);
    const int m = (int)M, n = (int)N, k = (int)K;
    hipError_t e;
    if (sw_grouped)
        e = out_fp32 ? launch_f6<true, true>(a6, w6, sap, swp, out, m, n, k, st)
                     : launch_f6<true, false>(a6, w6, sap, swp, out, m, n, k, st);
    else
        e = out_fp32 ? launch_f6<false, true>(a6, w6, sap, swp, out, m, n, k, st)
                     : launch_f6<false, false>(a6, w6, sap, swp, out, m, n, k, st);
    return (int)e;
}
