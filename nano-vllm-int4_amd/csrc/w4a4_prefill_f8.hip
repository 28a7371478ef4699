// K2, prefill-sized M, on the fp8 matrix cores: grouped W4A4 INT4 GEMM with
// the INT4 codes carried as fp8 (e4m3) values.
//
// Numerical contract (nanovllm/kernels/w4a4_grouped_kernel.py:64-90, oracle
// benchmarks/verify_w4a4_aw_grouped.py:13-29), bit for bit: for g in order,
//   total = fmaf(float(dot_g), float(sa[m,g]) * float(sw[n,g]), total)
// (per-channel weight scales: total = fmaf(float(dot_g), sa[m,g], total),
// C = bf16(total * sw[n])), then C = bf16_rne(total) or the fp32 total.
//
// Every INT4 code q in [-8, 7] is an e4m3 value exactly (integers up to 16
// have at most 4 significant bits), every product of two codes is an integer
// of magnitude <= 64 and every partial sum of a 128-deep group an integer of
// magnitude <= 8192: all exact in fp32, in any summation order.  So
// v_mfma_scale_f32_32x32x64_f8f6f4 (unit E8M0 scales) returns each group dot
// exactly, as fp32, with no integer-to-float conversion, and the staging
// copies bytes (no nibble widening).  The scale product sa * sw comes from a
// bf16 MFMA (exact, see read_scales below), which leaves one VALU fma per
// output and group.  The operands are first written as fp8 rows -- A [M, K]
// and W [N, K], one byte per code, k in order -- into a caller's workspace by
// a byte-lookup conversion kernel (reference or MFMA-tiled weight layout).
//
// Layout as k2_prefill (w4a4_prefill.hip): workgroup = 4 waves, 128 x 128
// output tile, whole K, two workgroups per CU, XCD-aware tile order.  Per
// group the A and W tiles (128 rows x 128 bytes each) go global -> LDS with
// buffer loads that write LDS directly, into a two-stage ring with one
// barrier per group; the bf16 scales move in 8-group windows.  An LDS row
// holds the group's 128 codes as eight 16-byte chunks, chunk c at
// c ^ (row % 8) ^ ((row / 8) % 2): the 16 rows that 16 consecutive lanes read
// in one LDS cycle of a 16-byte read then cover all 64 banks.
// MFMA 32x32x64: lane l supplies row (A) / column (W) l%32 and 32 bytes of k
// -- chunks 4h + 2s, 4h + 2s + 1 of half h = l/32 in k-step s (0..1); A and
// W read the same chunks, so every product pairs equal k.  Result: lane l
// holds C[8*(i/4) + 4*(l/32) + i%4][l%32], i = 0..15.
#include "nv4_common.h"

namespace nv4 {
namespace {

constexpr int F8_BM = 128, F8_BN = 128, F8_T = 256;
constexpr int F8_A = F8_BM * 128;                       // A tile bytes per group
constexpr int F8_W = F8_BN * 128;                       // W tile bytes per group
constexpr int F8_STAGE = F8_A + F8_W;
constexpr int F8_WSZ = 8 * (F8_BM + F8_BN) * 2;         // 8 groups x (sa[128], sw[128]) bf16
static_assert(2 * F8_STAGE + 2 * F8_WSZ == 72 * 1024, "72 KiB of LDS: two workgroups per CU");
constexpr int F8_GM = 8;                                // M-tiles per column sweep
constexpr int F8_RSRC_WORD3 = 0x00020000;               // buffer resource word 3 (CDNA): 32-bit data format

typedef int v8i __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void* lds_ptr;

// e4m3 codes of the INT4 values: nibble n (two's complement) -> fp8 byte.
// Four nibbles (one per byte, values 0..15) at a time: two 8-entry byte
// lookups (v_perm) for n < 8 and n >= 8, merged by bit 3.
__device__ __forceinline__ uint32_t nib4_to_e4m3(uint32_t x) {
    const uint32_t sel = x & 0x07070707u;
    const uint32_t pos = __builtin_amdgcn_perm(0x4E4C4A48u, 0x44403800u, sel);  //  0  1  2  3  4  5  6  7
    const uint32_t neg = __builtin_amdgcn_perm(0xB8C0C4C8u, 0xCACCCED0u, sel);  // -8 -7 -6 -5 -4 -3 -2 -1
    const uint32_t m = ((x >> 3) & 0x01010101u) * 0xFFu;
    return (neg & m) | (pos & ~m);
}

// 8 packed bytes (16 codes, k = 2j low nibble, 2j + 1 high nibble) -> 16 fp8 bytes in k order.
__device__ __forceinline__ v4u packed8_to_e4m3(uint32_t d0, uint32_t d1) {
    v4u r;
    const uint32_t d[2] = {d0, d1};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t lo = d[i] & 0x0F0F0F0Fu, hi = (d[i] >> 4) & 0x0F0F0F0Fu;  // k even / odd of 4 bytes
        // interleave: bytes (lo0 hi0 lo1 hi1) and (lo2 hi2 lo3 hi3)
        r[2 * i] = nib4_to_e4m3(__builtin_amdgcn_perm(hi, lo, 0x05010400u));
        r[2 * i + 1] = nib4_to_e4m3(__builtin_amdgcn_perm(hi, lo, 0x07030602u));
    }
    return r;
}

// Packed INT4 rows -> fp8 rows, both operands in one launch: thread u < ua
// converts 16-byte unit u of A, the others unit u - ua of W.  A is in the
// reference layout [M][K/2] (unit u = row * K/32 + c); W in the reference
// layout or, with W_TILED, the MFMA-tiled one (unit u = (cb*G + g)*64 + l
// holds packed bytes 64g + 16(l/16) .. +15 of row 16cb + l%16).  Each unit
// becomes 32 fp8 bytes of its row.
template <bool W_TILED>
__global__ void __launch_bounds__(256)
i4_to_f8_rows(const int8_t* __restrict__ a, uint8_t* __restrict__ a8, int64_t ua, const int8_t* __restrict__ w,
              uint8_t* __restrict__ w8, int64_t uw, int G, int K) {
    int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool is_a = u < ua;
    if (!is_a) u -= ua;
    if (!is_a && u >= uw) return;
    const v4u v = *reinterpret_cast<const v4u*>((is_a ? a : w) + u * 16);
    int64_t row;
    int kb;  // first packed byte of the unit within its row
    if (!is_a && W_TILED) {
        const int l = (int)(u & 63);
        const int64_t cg = u >> 6;
        const int g = (int)(cg % G);
        row = (cg / G) * 16 + (l & 15);
        kb = 64 * g + 16 * (l >> 4);
    } else {
        const int per = K >> 5;
        row = u / per;
        kb = (int)(u % per) * 16;
    }
    uint8_t* d = (is_a ? a8 : w8) + row * K + 2 * kb;
    *reinterpret_cast<v4u*>(d) = packed8_to_e4m3(v[0], v[1]);
    *reinterpret_cast<v4u*>(d + 16) = packed8_to_e4m3(v[2], v[3]);
}

__device__ __forceinline__ void f8_tile(int tm, int tn, int& mt, int& nt) {
    const int T = tm * tn;
    const int b = blockIdx.x;
    const int t = (T & 7) == 0 ? (b & 7) * (T >> 3) + (b >> 3) : b;
    const int per = F8_GM * tn;
    const int grp = t / per;
    const int first = grp * F8_GM;
    const int gm = min(tm - first, F8_GM);
    const int r = t - grp * per;
    mt = first + r % gm;
    nt = r / gm;
}

template <bool SG, bool OF, bool WIN>
__global__ void __launch_bounds__(F8_T, 2)
k2_prefill_f8(const uint8_t* __restrict__ a, const uint8_t* __restrict__ w, const uint16_t* __restrict__ sa,
              const uint16_t* __restrict__ sw, void* __restrict__ out, int M, int N, int K, int tm, int tn) {
    // Two operand stages (A tile then W tile) and the scale windows, as
    // separate arrays so that reads of one stage are not ordered behind the
    // direct-to-LDS loads in flight into the other.
    __shared__ __align__(16) uint8_t st0[F8_STAGE];
    __shared__ __align__(16) uint8_t st1[F8_STAGE];
    __shared__ __align__(16) uint16_t win[F8_WSZ];
    int mt, nt;
    f8_tile(tm, tn, mt, nt);
    const int m0 = mt * F8_BM, n0 = nt * F8_BN;
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int G = K >> 7;

    // Direct-to-LDS staging: load i (0..3) of wave w fills the 1 KiB at
    // (4w + i) * 1024 of a tile, lane l the 16 bytes at l * 16: tile row
    // r = 8(4w + i) + l/8 and LDS slot l%8, which holds the row's chunk
    // (l%8) ^ (r%8) ^ (i%2).  Rows past the matrix edge repeat the last row (never stored).
    const uint8_t* a_t = a + (int64_t)m0 * K;
    const uint8_t* w_t = w + (int64_t)n0 * K;
    uint32_t offa[4], offw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 8 * (4 * wave + i) + (lane >> 3), c = (lane & 7) ^ ((lane >> 3) & 7) ^ (i & 1);
        offa[i] = (uint32_t)(min(r, M - 1 - m0) * K + c * 16);
        offw[i] = (uint32_t)(min(r, N - 1 - n0) * K + c * 16);
    }
    // Buffer resources over the tile rows (at most 128 * K bytes), so the
    // loads take 32-bit lane offsets and the group offset as a scalar.
    const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(a_t), (short)0, min(F8_BM, M - m0) * K, F8_RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t rsw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(w_t), (short)0, min(F8_BN, N - n0) * K, F8_RSRC_WORD3);
    auto dma = [&](int g, uint8_t* st) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_ptr)(st + (4 * wave + i) * 1024), 16, offa[i], g * 128, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsw, (lds_ptr)(st + F8_A + (4 * wave + i) * 1024), 16, offw[i],
                                                     g * 128, 0, 0);
        }
    };
    // Scales: two windows of 8 groups, [group % 8][sa row 0..127, sw column
    // 0..127] bf16; thread t < 128 moves the sa of tile row t, the others the
    // sw of tile column t-128 (per-channel form: an unused sa).
    const bool is_sa = t < F8_BM;
    const uint16_t* s_t = is_sa ? sa + (int64_t)m0 * G : (SG ? sw + (int64_t)n0 * G : sa + (int64_t)m0 * G);
    const uint32_t offs = (uint32_t)(is_sa ? min(t, M - 1 - m0) * G : (SG ? min(t - F8_BM, N - 1 - n0) * G : 0));
    auto slot = [&](int x) { return win + ((x >> 3) & 1) * (F8_WSZ / 2) + (x & 7) * (F8_BM + F8_BN); };
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

    // Operand reads: lane (rc, half) of block rows base + rc, k-step s:
    // chunks 4*half + 2s and 4*half + 2s + 1 (the block base is a multiple
    // of 32 rows, so the swizzle depends on rc only).
    const int rc = lane & 31, half = lane >> 5;
    const int rxor = (rc & 7) ^ ((rc >> 3) & 1);
    int oa[2][2], ow[2][2];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int cs = (((4 * half + 2 * s + e) ^ rxor) << 4) + rc * 128;
            oa[s][e] = cs + wm * 64 * 128;
            ow[s][e] = cs + F8_A + wn * 64 * 128;
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
                const v4u a0 = *reinterpret_cast<const v4u*>(st + oa[s][0] + i * 32 * 128);
                const v4u a1 = *reinterpret_cast<const v4u*>(st + oa[s][1] + i * 32 * 128);
                const v4u w0 = *reinterpret_cast<const v4u*>(st + ow[s][0] + i * 32 * 128);
                const v4u w1 = *reinterpret_cast<const v4u*>(st + ow[s][1] + i * 32 * 128);
                pa[i][s] = v8i{(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3],
                               (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
                pw[i][s] = v8i{(int)w0[0], (int)w0[1], (int)w0[2], (int)w0[3],
                               (int)w1[0], (int)w1[1], (int)w1[2], (int)w1[3]};
            }
    };
    // Blocks in the order (0,0), (0,1), (1,1), (1,0).
    auto mma = [&](int b) {
        const int i = b >> 1, j = (b ^ (b >> 1)) & 1;
        v16f c = {};
#pragma unroll
        for (int s = 0; s < 2; ++s)
            c = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(pa[i][s], pw[j][s], c, 0, 0, 0, 127, 0, 127);
        acc[b & 1] = c;
    };
    // Scale products on the matrix cores: a product of two bf16 values has
    // at most 16 significant bits, so sa[m] * sw[n] is exact in fp32 unless
    // it falls below the normal range, and a bf16 MFMA whose only non-zero k
    // term is (sa[row], sw[column]) returns the fp32 product the reference
    // multiplies (sa alone, times bf16 1.0, for per-channel weight scales).
    // Scales whose products reach the fp32 subnormals (bf16 subnormals, 2^-126)
    // are in the parity tests and match the oracle bit for bit.  32x32x16 bf16 operands:
    // lane l supplies row / column l%32, k = 8(l/32) .. +7, so lanes 32..63
    // supply zeros; the result has the layout of the fp8 dot.
    const uint32_t keep = half ? 0u : 0xffffu;
    uint32_t sab[2], swb[2];
    auto read_scales = [&](const uint16_t* sg) {
#pragma unroll
        for (int i = 0; i < 2; ++i) sab[i] = sg[wm * 64 + i * 32 + rc] & keep;
#pragma unroll
        for (int j = 0; j < 2; ++j) swb[j] = (SG ? (uint32_t)sg[F8_BM + wn * 64 + j * 32 + rc] : 0x3f80u) & keep;
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
hipError_t launch_f8(const uint8_t* a8, const uint8_t* w8, const uint16_t* sa, const uint16_t* sw, void* out,
                     int M, int N, int K, hipStream_t st) {
    const int tm = (M + F8_BM - 1) / F8_BM, tn = (N + F8_BN - 1) / F8_BN;
    const bool win = (K / 128) % 8 == 0 && reinterpret_cast<uintptr_t>(sa) % 16 == 0 &&
                     (!SG || reinterpret_cast<uintptr_t>(sw) % 16 == 0);
    if (win)
        hipLaunchKernelGGL((k2_prefill_f8<SG, OF, true>), dim3((unsigned)(tm * tn)), dim3(F8_T), 0, st, a8, w8, sa,
                           sw, out, M, N, K, tm, tn);
    else
        hipLaunchKernelGGL((k2_prefill_f8<SG, OF, false>), dim3((unsigned)(tm * tn)), dim3(F8_T), 0, st, a8, w8, sa,
                           sw, out, M, N, K, tm, tn);
    return hipGetLastError();
}

}  // namespace
}  // namespace nv4

extern "C" int nv4_w4a4_gemm_f8(const int8_t* a, const int8_t* w, int w_tiled, const void* sa, const void* sw,
                                int sw_grouped, void* out, int out_fp32, int64_t M, int64_t N, int64_t K,
                                void* workspace, int64_t workspace_bytes, void* stream) {
    using namespace nv4;
    if (!a || !w || !sa || !sw || !out || !workspace) return NV4_E_NULL;
    if (M < 1 || N < 1 || K < 128 || K % 128 || N % 8 || (w_tiled && N % 16)) return NV4_E_SHAPE;
    if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > (1LL << 20)) return NV4_E_SHAPE;
    if (128 * K > 0x7fffffffLL || M * (K / 128) > 0x7fffffffLL || N * (K / 128) > 0x7fffffffLL) return NV4_E_SHAPE;
    // Dispatch grids count work-items in 32 bits: the conversion launches one
    // per 16 packed bytes of both operands, the GEMM 256 per output tile.
    if (((M + 127) / 128) * ((N + F8_BN - 1) / F8_BN) * F8_T > 0xffffffffLL) return NV4_E_SHAPE;
    if ((M + N) * (K / 32) > 0xffffff00LL) return NV4_E_SHAPE;
    if (workspace_bytes < (M + N) * K) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(a) % 16 || reinterpret_cast<uintptr_t>(w) % 16 ||
        reinterpret_cast<uintptr_t>(sa) % 2 || reinterpret_cast<uintptr_t>(sw) % 2 ||
        reinterpret_cast<uintptr_t>(out) % (out_fp32 ? 4 : 2) || reinterpret_cast<uintptr_t>(workspace) % 16)
        return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint8_t* a8 = static_cast<uint8_t*>(workspace);
    uint8_t* w8 = a8 + M * K;
    const int G = (int)(K / 128);
    const int64_t ua = M * K / 32, uw = N * K / 32;
    const unsigned cgrid = (unsigned)((ua + uw + 255) / 256);
    if (w_tiled)
        hipLaunchKernelGGL(i4_to_f8_rows<true>, dim3(cgrid), dim3(256), 0, st, a, a8, ua, w, w8, uw, G, (int)K);
    else
        hipLaunchKernelGGL(i4_to_f8_rows<false>, dim3(cgrid), dim3(256), 0, st, a, a8, ua, w, w8, uw, G, (int)K);
    const auto* sap = static_cast<const uint16_t*>(sa);
    const auto* swp = static_cast<const uint16_t*>(sw);
    const int m = (int)M, n = (int)N, k = (int)K;
    hipError_t e;
    if (sw_grouped)
        e = out_fp32 ? launch_f8<true, true>(a8, w8, sap, swp, out, m, n, k, st)
                     : launch_f8<true, false>(a8, w8, sap, swp, out, m, n, k, st);
    else
        e = out_fp32 ? launch_f8<false, true>(a8, w8, sap, swp, out, m, n, k, st)
                     : launch_f8<false, false>(a8, w8, sap, swp, out, m, n, k, st);
    return (int)e;
}
