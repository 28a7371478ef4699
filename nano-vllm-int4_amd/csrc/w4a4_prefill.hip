// K2, prefill-sized M: grouped W4A4 INT4 GEMM on LDS-staged 128x128 tiles.
//
// Numerical contract (nanovllm/kernels/w4a4_grouped_kernel.py:64-90, oracle
// benchmarks/verify_w4a4_aw_grouped.py:13-29), bit for bit: for g in order,
//   total = fmaf(float(dot_g), float(sa[m,g]) * float(sw[n,g]), total)
// (per-channel weight scales: total = fmaf(float(dot_g), sa[m,g], total),
// C = bf16(total * sw[n])), then C = bf16_rne(total) or the fp32 total.
//
// Work per output element and group is one int32 dot of 128 products on the
// matrix cores (v_mfma_i32_32x32x32_i8 on nibbles widened to 16*q, so the
// MFMA returns 256*dot) and an fp32 epilogue on the vector ALUs: convert,
// scale product, fma.  The >>8 that turns 256*dot into dot is folded into
// the activation scale: sa' = sa * 2^-8 is exact for every finite bf16 sa,
// and fmaf(256*dot, RN(sa' * sw), t) == fmaf(dot, RN(sa * sw), t) whenever
// RN(sa' * sw) == RN(sa * sw) * 2^-8, i.e. when the exact product sa*sw
// stays a normal float after the 2^-8 (scales zero, or with magnitudes in
// [2^-59, 2^63]: bf16 products have at most 16 significant bits).  A
// workgroup whose scales are not all in that range (tiny activation groups
// from near-zero rows, for instance) runs the literal sequence instead:
// d = acc >> 8, s = sa * sw, fmaf(float(d), s, t).  With per-channel weight
// scales the product 256*dot*sa' inside the fma is exact for any finite sa,
// so that form always takes the short path.
//
// Layout: workgroup = 4 waves (one per SIMD), 128 (M) x 128 (N) output tile,
// whole K, no split-K, no atomics; two workgroups per CU.  Wave (wm, wn)
// owns rows 64*wm.., columns 64*wn.. as 2x2 blocks of 32x32.  Per group the
// A and W tiles and the fp32 scale vectors go through a two-stage LDS ring
// filled from registers loaded one group ahead, with one barrier per group.
// Each group is issued as: LDS reads; the MFMAs of block b next to the
// epilogue of block b-1 (two rotating accumulators), the first block's
// MFMAs next to the staging of the next group; the last epilogue.  The
// vector ALUs bound this kernel (a wave64 VALU op holds the SIMD for 4
// cycles; the epilogue is 3 of them per output element and group against
// one 32-cycle MFMA per 32x32x32), so the loop is written for instruction
// count:
//  * the staging threads widen the nibbles on the way into LDS (each tile
//    row is read by two waves, so this halves the widening work);
//  * the group loop is unrolled by the two LDS stages, so every LDS address
//    is a per-lane base plus an immediate offset;
//  * global loads use a wave-uniform tile base and a 32-bit lane offset.
// An LDS row holds a group's 128 int8 operands as eight 16-byte chunks,
// chunk u = packed bytes 8u..8u+7 widened (lo nibbles of bytes 0-3, hi
// nibbles of bytes 0-3, then the same for bytes 4-7), stored at chunk
// u ^ (row % 8) ^ ((row / 8) % 2): the sixteen rows read by sixteen
// consecutive lanes fall in distinct bank groups, and so do the chunks eight
// consecutive staging lanes write.
//
// MFMA 32x32x32 i8: lane l supplies row (A) / column (W) l%32 and the
// k-slots of half h = l/32; k-step s (0..3) reads chunk 4h + s.  A and W use
// the same chunks, so every product pairs equal k.  Result: lane l holds
// C[8*(i/4) + 4*(l/32) + i%4][l%32], i = 0..15.
//
// Tile order is XCD-aware: workgroups are dispatched round-robin over the 8
// XCDs, so workgroup b is given tile (b%8)*(T/8) + b/8 of an M-grouped order
// (8 M-tiles per column sweep): the tiles resident on one XCD at a time form
// an 8x8 block that shares its A rows and W columns through that XCD's L2.
#include "k2_launch.h"
#include "nv4_common.h"

namespace nv4 {
namespace {

constexpr int PF_BM = 128, PF_BN = 128, PF_T = 256;
constexpr int PF_A = PF_BM * 128;                       // widened A tile bytes per group
constexpr int PF_W = PF_BN * 128;                       // widened W tile bytes per group
constexpr int PF_STAGE = PF_A + PF_W;                   // one operand stage
constexpr int PF_WIN = 2 * PF_STAGE;                    // scale windows after the two stages
constexpr int PF_WSZ = 8 * (PF_BM + PF_BN) * 4;         // 8 groups x (sa[128], sw[128]) fp32
constexpr int PF_LDS = PF_WIN + 2 * PF_WSZ;             // 80 KiB: two workgroups fill 160 KiB
constexpr int PF_GM = 8;                                // M-tiles per column sweep

// Row r's 16-byte chunk u sits at u ^ (r % 8) ^ ((r / 8) % 2): the 16 rows that
// 16 consecutive lanes read in one LDS cycle of a 16-byte read cover all 64 banks.
__device__ __forceinline__ int pf_rxor(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int pf_swz(int r, int u) { return r * 128 + ((u ^ pf_rxor(r)) << 4); }

// Scale magnitudes for which the 2^-8 fold is exact (see the file comment).
__device__ __forceinline__ bool pf_scale_ok(uint32_t h) {
    const uint32_t e = (h >> 7) & 0xffu;
    return (h & 0x7fffu) == 0 || (e >= 127u - 59u && e <= 127u + 63u);
}

__device__ __forceinline__ void pf_tile(int tm, int tn, int& mt, int& nt) {
    const int T = tm * tn;
    const int b = blockIdx.x;
    const int t = (T & 7) == 0 ? (b & 7) * (T >> 3) + (b >> 3) : b;
    const int per = PF_GM * tn;
    const int grp = t / per;
    const int first = grp * PF_GM;
    const int gm = min(tm - first, PF_GM);
    const int r = t - grp * per;
    mt = first + r % gm;
    nt = r / gm;
}

template <bool OUT_F32>
__device__ __forceinline__ void pf_store(void* out, int64_t idx, float v) {
    if constexpr (OUT_F32) {
        static_cast<float*>(out)[idx] = v;
    } else {
        static_cast<uint16_t*>(out)[idx] = (uint16_t)f32_to_bf16_rne(v);
    }
}

template <bool FAST, bool SG, bool OF, bool WIN, bool TW>
__device__ __forceinline__ void pf_body(const int8_t* __restrict__ a, const int8_t* __restrict__ w,
                                        const uint16_t* __restrict__ sa, const uint16_t* __restrict__ sw,
                                        void* __restrict__ out, int M, int N, int K, int m0, int n0,
                                        uint8_t* smem) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int G = K >> 7;
    const int KB = K >> 1;

    // Staging: thread t moves packed A chunks q = t, t+256 (row q/4, chunk
    // q%4, widened into LDS chunks 2(q%4), 2(q%4)+1) and the same W chunks.
    // Tile bases are wave-uniform; lane offsets stay below 128 * K/2 bytes.
    // Scales live in two LDS windows of 8 groups each, [group % 8][sa row
    // 0..127, sw column 0..127] as fp32 (sa scaled by 2^-8 on the short
    // path): thread t < 128 moves the sa of tile row t, the others the sw of
    // tile column t-128 (per-channel form: they reload an sa entry and leave
    // it unused).  With WIN the scales of a row are contiguous and 16-byte
    // aligned (G % 8 == 0), so one 16-byte load brings 8 groups and the
    // window is written every 8 groups; otherwise each group's scale is
    // loaded and written on its own -- a 2-byte load per row and group would
    // otherwise cost as many cache requests as all the operand data.
    // With the MFMA-tiled weight layout (TW: [N/16][G][64 lanes][16 bytes])
    // thread q instead moves lane q%64 of the tile's column block q/64 (tile
    // row 16 (q/64) + q%16, chunk (q%64)/16): whole 1 KiB blocks per wave.
    const int8_t* a_t = a + (int64_t)m0 * KB;
    const int8_t* w_t = TW ? w + (int64_t)(n0 >> 4) * G * 1024 : w + (int64_t)n0 * KB;
    uint32_t offa[2], offw[2];
    int la[2], lw[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int q = t + i * PF_T, r = q >> 2, c = q & 3;
        offa[i] = (uint32_t)(min(r, M - 1 - m0) * KB + c * 16);
        la[i] = pf_swz(r, 2 * c);  // chunk 2c+1 lands at la ^ 16
        if constexpr (TW) {
            const int j = q >> 6, l = q & 63;
            offw[i] = (uint32_t)(min(j, ((N - n0) >> 4) - 1) * G * 1024 + l * 16);
            lw[i] = pf_swz(j * 16 + (l & 15), 2 * (l >> 4));
        } else {
            offw[i] = (uint32_t)(min(r, N - 1 - n0) * KB + c * 16);
            lw[i] = la[i];
        }
    }
    const bool is_sa = t < PF_BM;
    const uint16_t* s_t = is_sa ? sa + (int64_t)m0 * G : (SG ? sw + (int64_t)n0 * G : sa + (int64_t)m0 * G);
    const uint32_t offs = (uint32_t)(is_sa ? min(t, M - 1 - m0) * G
                                           : (SG ? min(t - PF_BM, N - 1 - n0) * G : 0));
    // Short path: sa * 2^-8 (exact for every finite bf16 value).
    const float sfac = (FAST && is_sa) ? 0x1p-8f : 1.0f;
    auto slot = [&](int x) { return PF_WIN + ((x >> 3) & 1) * PF_WSZ + (x & 7) * ((PF_BM + PF_BN) * 4); };

    v4u ra[2], rw[2];
    uint32_t rs;
    auto load = [&](int g) {
        const int8_t* ag = a_t + g * 64;
        const int8_t* wg = w_t + g * (TW ? 1024 : 64);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            ra[i] = *reinterpret_cast<const v4u*>(ag + offa[i]);
            rw[i] = *reinterpret_cast<const v4u*>(wg + offw[i]);
        }
        if constexpr (!WIN) rs = (s_t + g)[offs];
    };
    // Operands of the next group into stage st; without WIN also its scale.
    auto store = [&](uint8_t* st, int x) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            // chunk 2c at la, chunk 2c+1 at la with the slot index's bit 0 flipped
            const int l0 = la[i], l1 = la[i] ^ 16;
            *reinterpret_cast<v4i*>(st + l0) = unpack8_x16(ra[i][0], ra[i][1]);
            *reinterpret_cast<v4i*>(st + l1) = unpack8_x16(ra[i][2], ra[i][3]);
            const int m0w = lw[i], m1w = lw[i] ^ 16;
            *reinterpret_cast<v4i*>(st + PF_A + m0w) = unpack8_x16(rw[i][0], rw[i][1]);
            *reinterpret_cast<v4i*>(st + PF_A + m1w) = unpack8_x16(rw[i][2], rw[i][3]);
        }
        if constexpr (!WIN) *reinterpret_cast<float*>(smem + slot(x) + t * 4) = bf16_to_f32(rs) * sfac;
    };
    v4u rwin;
    auto load_win = [&](int wi) { rwin = *reinterpret_cast<const v4u*>(s_t + offs + 8 * wi); };
    auto store_win = [&](int wi) {
#pragma unroll
        for (int gl = 0; gl < 8; ++gl) {
            const uint32_t h = (rwin[gl >> 1] >> (16 * (gl & 1))) & 0xffffu;
            *reinterpret_cast<float*>(smem + slot(wi * 8 + gl) + t * 4) = bf16_to_f32(h) * sfac;
        }
    };

    // Operand reads: lane (rc, half) reads row r = base + rc, chunk 4*half + s
    // at r*128 + (((4*half + s) ^ pf_rxor(rc)) << 4) (the block base is a
    // multiple of 32 rows, so the swizzle depends on rc only).
    const int rc = lane & 31, half = lane >> 5;
    int oa[4], ow[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int cs = (((4 * half + s) ^ pf_rxor(rc)) << 4) + rc * 128;
        oa[s] = cs + wm * 64 * 128;
        ow[s] = cs + PF_A + wn * 64 * 128;
    }
    float total[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) total[i][j][v] = 0.0f;

    // Blocks in the order (0,0), (0,1), (1,1), (1,0).
    v4i pa[2][4], pw[2][4];
    v16i acc[2];
    auto fetch = [&](const uint8_t* st) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                pa[i][s] = *reinterpret_cast<const v4i*>(st + oa[s] + i * 32 * 128);
                pw[i][s] = *reinterpret_cast<const v4i*>(st + ow[s] + i * 32 * 128);
            }
    };
    auto mma = [&](int b) {
        const int i = b >> 1, j = (b ^ (b >> 1)) & 1;
        v16i c = {};
#pragma unroll
        for (int s = 0; s < 4; ++s) c = __builtin_amdgcn_mfma_i32_32x32x32_i8(pa[i][s], pw[j][s], c, 0, 0, 0);
        acc[b & 1] = c;
    };
    // Epilogue of block b: row scales for rows 8q + 4*half + e (q, e = 0..3)
    // are four 16-byte LDS reads (broadcast within each half-wave), the
    // column scale one.
    auto epi = [&](int b, const uint8_t* sg) {
        const int i = b >> 1, j = (b ^ (b >> 1)) & 1;
        const float* sal = reinterpret_cast<const float*>(sg) + wm * 64 + i * 32 + 4 * half;
        const float swc = SG ? reinterpret_cast<const float*>(sg)[PF_BM + wn * 64 + j * 32 + rc] : 1.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const v4f s4 = *reinterpret_cast<const v4f*>(sal + 8 * q);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int v = 4 * q + e;
                const float s = SG ? s4[e] * swc : s4[e];
                const float d = FAST ? (float)acc[b & 1][v] : (float)(acc[b & 1][v] >> 8);
                total[i][j][v] = __builtin_fmaf(d, s, total[i][j][v]);
            }
        }
    };
    // One group.  Branch-free, so the whole step is one scheduling region:
    // the last steps reload group G-1 and restage it into the idle stage,
    // which nothing reads again.
    auto step = [&](int g, uint8_t* st, uint8_t* st_next) {
        __syncthreads();  // this stage written; the other one no longer read
        const uint8_t* sg = smem + slot(g);
        fetch(st);
        mma(0);
        store(st_next, g + 1);
        load(min(g + 2, G - 1));
        mma(1);
        epi(0, sg);
        mma(2);
        epi(1, sg);
        mma(3);
        epi(2, sg);
        epi(3, sg);
        // Scale windows: load the next one four groups ahead, write it
        // after the last group that reads the buffer it replaces (the
        // buffer's previous window ended 8 groups ago).
        if constexpr (WIN) {
            if ((g & 7) == 3) load_win(min((g >> 3) + 1, (G >> 3) - 1));
            if ((g & 7) == 7) store_win((g >> 3) + 1);
        }
    };

    if constexpr (WIN) {
        load_win(0);
        store_win(0);
    } else {
        load(0);  // scale of group 0 (its operands are reloaded below)
        *reinterpret_cast<float*>(smem + slot(0) + t * 4) = bf16_to_f32(rs) * sfac;
    }
    load(0);
    store(smem, 1);
    load(min(1, G - 1));
    uint8_t* const s0 = smem;
    uint8_t* const s1 = smem + PF_STAGE;
    for (int g = 0; g < G; g += 2) {
        step(g, s0, s1);
        if (g + 1 < G) step(g + 1, s1, s0);
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
                    pf_store<OF>(out, (int64_t)m * N + n, val);
                }
            }
    }
}

template <bool SG, bool OF, bool WIN, bool TW>
__global__ void __launch_bounds__(PF_T, 2)
k2_prefill(const int8_t* __restrict__ a, const int8_t* __restrict__ w, const uint16_t* __restrict__ sa,
           const uint16_t* __restrict__ sw, void* __restrict__ out, int M, int N, int K, int tm, int tn) {
    __shared__ __align__(16) uint8_t smem[PF_LDS];
    int mt, nt;
    pf_tile(tm, tn, mt, nt);
    const int m0 = mt * PF_BM, n0 = nt * PF_BN;
    // Grouped weight scales: check every scale of the tile's rows and
    // columns (contiguous ranges of sa and sw) for the range in which the
    // short epilogue is exact.  Per-channel weight scales: always exact.
    bool fast = true;
    if constexpr (SG) {
        const int G = K >> 7;
        const int64_t na = (int64_t)min(PF_BM, M - m0) * G;
        const int64_t nw = (int64_t)min(PF_BN, N - n0) * G;
        const uint16_t* pa = sa + (int64_t)m0 * G;
        const uint16_t* pw = sw + (int64_t)n0 * G;
        bool ok = true;
        for (int64_t e = threadIdx.x; e < na; e += PF_T) ok = ok && pf_scale_ok(pa[e]);
        for (int64_t e = threadIdx.x; e < nw; e += PF_T) ok = ok && pf_scale_ok(pw[e]);
        // Workgroup AND through a flag in the (not yet used) staging memory.
        int* flag = reinterpret_cast<int*>(smem);
        if (threadIdx.x == 0) *flag = 1;
        __syncthreads();
        if (!ok) *flag = 0;
        __syncthreads();
        fast = *flag != 0;
        __syncthreads();
    }
    if (fast)
        pf_body<true, SG, OF, WIN, TW>(a, w, sa, sw, out, M, N, K, m0, n0, smem);
    else
        pf_body<false, SG, OF, WIN, TW>(a, w, sa, sw, out, M, N, K, m0, n0, smem);
}

template <bool SG, bool OF, bool TW>
hipError_t launch(const int8_t* a, const int8_t* w, const void* sa, const void* sw, void* out, int M, int N,
                  int K, hipStream_t st) {
    const int tm = (M + PF_BM - 1) / PF_BM, tn = (N + PF_BN - 1) / PF_BN;
    const auto* sap = static_cast<const uint16_t*>(sa);
    const auto* swp = static_cast<const uint16_t*>(sw);
    // 8-group scale windows: rows of 8*k scales starting on 16-byte boundaries.
    const bool win = (K / 128) % 8 == 0 && reinterpret_cast<uintptr_t>(sa) % 16 == 0 &&
                     (!SG || reinterpret_cast<uintptr_t>(sw) % 16 == 0);
    if (win)
        hipLaunchKernelGGL((k2_prefill<SG, OF, true, TW>), dim3((unsigned)(tm * tn)), dim3(PF_T), 0, st, a, w, sap,
                           swp, out, M, N, K, tm, tn);
    else
        hipLaunchKernelGGL((k2_prefill<SG, OF, false, TW>), dim3((unsigned)(tm * tn)), dim3(PF_T), 0, st, a, w, sap,
                           swp, out, M, N, K, tm, tn);
    return hipGetLastError();
}

}  // namespace

hipError_t k2_prefill_launch(const int8_t* a, const int8_t* w, const void* sa, const void* sw,
                             bool sw_grouped, void* out, bool out_fp32, bool w_tiled, int M, int N, int K,
                             hipStream_t st) {
    if (w_tiled) {
        if (sw_grouped)
            return out_fp32 ? launch<true, true, true>(a, w, sa, sw, out, M, N, K, st)
                            : launch<true, false, true>(a, w, sa, sw, out, M, N, K, st);
        return out_fp32 ? launch<false, true, true>(a, w, sa, sw, out, M, N, K, st)
                        : launch<false, false, true>(a, w, sa, sw, out, M, N, K, st);
    }
    if (sw_grouped)
        return out_fp32 ? launch<true, true, false>(a, w, sa, sw, out, M, N, K, st)
                        : launch<true, false, false>(a, w, sa, sw, out, M, N, K, st);
    return out_fp32 ? launch<false, true, false>(a, w, sa, sw, out, M, N, K, st)
                    : launch<false, false, false>(a, w, sa, sw, out, M, N, K, st);
}

}  // namespace nv4
