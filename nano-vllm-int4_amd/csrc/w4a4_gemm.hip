// K2: grouped W4A4 INT4 GEMM for gfx950.
//
// Numerical contract (nanovllm/kernels/w4a4_grouped_kernel.py:64-90, oracle
// benchmarks/verify_w4a4_aw_grouped.py:13-29), reproduced bit for bit:
//   for g = 0..K/128-1 in order:
//     d = sum_{k in group g} qa[m,k] * qw[n,k]          exact int32
//     grouped Sw:  total = fmaf(float(d), float(sa[m,g]) * float(sw[n,g]), total)
//     per-channel: total = fmaf(float(d), float(sa[m,g]), total)
//   C = bf16_rne(total)                (per-channel: bf16_rne(total * sw[n]))
//   or the fp32 total itself (diagnostic output).
//
// gfx950 has no INT4 MFMA.  Nibbles are widened to int8 in registers with two
// VALU ops per 8 nibbles: the nibble is placed in the high half of its byte
// (value * 16), which is exact for two's complement.  Both operands carry the
// x16, the int32 MFMA result is 256 * d (|256 d| <= 2^21), and an arithmetic
// shift by 8 recovers d exactly before the fp32 epilogue.  The k order inside
// a group is irrelevant for an exact integer sum, so A and W are unpacked by
// the same routine and fed to v_mfma_i32_*_i8 in matching lanes.
//
// Weights come in the reference layout [N][K/2] or in the MFMA-tiled layout
// (nv4_w4a4_tile_weights: 16 columns x 128 k of one column block and group
// as 1 KiB in lane order), which lets every weight load be whole cache
// lines; the results are the same bits.
//
// Three kernels, no split-K, no atomics:
//  * k2_dec (M <= 64): one workgroup per 16 output columns (two 16-column
//    blocks when one each would put two workgroups, each reading all of the
//    activations, on some CUs) and all M rows.
//    Its 8 or 16 waves each take one K group per round, compute the exact
//    int32 group dots with v_mfma_i32_16x16x64_i8 and hand them through LDS
//    to the whole workgroup, which runs the fp32 epilogue in group order.
//    Loads run several rounds ahead.
//  * k2_wide (M <= 32, wide N): waves own column blocks over the whole K,
//    activations widened once per CU into LDS.
//  * k2_prefill (M > 64, w4a4_prefill.hip): LDS-staged 128x128 tiles.
#include "k2_launch.h"
#include "norm_ops.h"
#include "nv4_common.h"

namespace nv4 {
namespace {

template <bool OUT_F32>
__device__ __forceinline__ void store_out(void* out, int64_t idx, float v) {
    if constexpr (OUT_F32) {
        static_cast<float*>(out)[idx] = v;
    } else {
        static_cast<uint16_t*>(out)[idx] = (uint16_t)f32_to_bf16_rne(v);
    }
}

// ----------------------------------------------------------------------------
// Decode kernel (M <= 64).  Workgroup = one 16-column block, all M rows
// (MB row blocks of 16), whole K; its NW waves (8, or 16 when one workgroup
// per CU covers N) split the K groups: in round r wave w takes group
// NW r + w.  Per group the wave computes the exact int32 dots of the
// 16-column x ROWS tile (v_mfma_i32_16x16x64_i8, two per row block) and
// writes them to LDS as int16; after the round's barrier each thread owning
// an output advances its in-order fp32 epilogue over the round's NW groups
// while later rounds' loads are in flight.  Dots, activation slices and
// scales are double buffered, so one barrier per round suffices.
//
// Loads are shaped for the CU's load path, which moves whole contiguous
// 128-byte lines several times faster than the 16 half-lines of a per-lane
// MFMA operand load:
//  * weights: with the MFMA-tiled layout (TW) one group of a column block is
//    1 KiB, lane l's 16 bytes at l*16, so a wave loads whole lines; with the
//    reference layout [N][K/2] lane l loads column l%16, bytes 16*(l/16) of
//    the group's 64;
//  * activations: the round's slice (ROWS rows x NW*64 bytes) is loaded in
//    whole lines by all threads, staged in LDS one round ahead and read back
//    as MFMA operands.
// All loads of a round ride in a register ring D rounds deep, together with
// the round's scales (sa of every row and sw of the 16 columns, NW groups).
// They are buffer loads whose per-thread offsets are fixed for the kernel:
// the round enters as a scalar offset, so the ring costs no vector address
// arithmetic.
//
// Layouts.  MFMA 16x16x64 i8: A operand lane l supplies row l%16, B operand
// column l%16, both the k-slots of set l/16; lane l of the result holds
// C[4*(l/16) + i][l%16], i = 0..3.  LDS activation slice: row r at
// r*NW*64 bytes, its 16-byte chunk c at chunk (c & ~7) | ((c ^ r) & 7), so
// the 16 rows of one operand load fall in distinct bank groups.  Tile output
// o = rb*256 + 4*l + i (row block rb, MFMA lane l, result i) is row
// 16 rb + 4 (l/16) + i, column l%16: the epilogue's dot reads are
// consecutive int16 over the threads.  Round scales: sal[row][group % NW]
// and swl[column][group % NW], read four at a time.  Each phase issues all
// of its LDS reads before their first use (the compiler would otherwise wait
// on each read in turn).
//
// Every global load is unconditional (offsets clamped into range): a load
// under a thread-dependent branch makes the compiler drain all outstanding
// loads at the branch join, which would serialise the ring.
// ----------------------------------------------------------------------------
constexpr int DC_RSRC_WORD3 = 0x00020000;  // buffer resource word 3 (CDNA): 32-bit data format
// Cache policy of k2_dec's weight loads: non-temporal (each weight byte is
// read once per call); measured 3-5 % faster than the default on qkv, o and
// down, while k2_wide measured 9 % slower with it and keeps the default.
constexpr int DC_NT = 2;

template <int MB, int NW, int D, bool TW, bool RT, bool SW_GROUPED, bool OUT_F32, int CB = 1>
__global__ void __launch_bounds__(NW * 64, 16 / NW)
k2_dec(const int8_t* __restrict__ a, const int8_t* __restrict__ w,
       const uint16_t* __restrict__ sa, const uint16_t* __restrict__ sw,
       void* __restrict__ out, int M, int N, int K) {
    constexpr int DC_T = NW * 64;
    constexpr int ROWS = MB * 16, TOUT = ROWS * 16, NOUT = TOUT * CB;  // CB column blocks of 16
    constexpr int GR = NW;                                              // groups per round
    constexpr int SLB = GR * 64;                                        // slice bytes per row and round
    constexpr int CPR = SLB / 16;                                       // 16-byte chunks per row and round
    constexpr int OPT = (NOUT + DC_T - 1) / DC_T;                      // outputs per thread
    constexpr int APT = ROWS * CPR / DC_T;                              // activation chunks per thread
    constexpr int NA = RT ? MB : APT;                                   // activation loads per thread and round
    constexpr int N_SA = ROWS * GR;                                     // scale entries per round
    constexpr int N_SW = SW_GROUPED ? 16 * CB * GR : 0;
    constexpr int SPT = (N_SA + N_SW + DC_T - 1) / DC_T;
    static_assert(RT || APT * DC_T == ROWS * CPR, "activation slice must split evenly");
    static_assert(!RT || TW, "row-tiled activations go with tiled weights");
    static_assert(CB == 1 || TW, "several column blocks per workgroup read tiled weights");
    static_assert(N_SA % 64 == 0 && N_SW % 64 == 0, "scale classes must be wave-uniform");
    __shared__ __align__(16) uint8_t a_l[2][RT ? 16 : ROWS * SLB];
    __shared__ __align__(16) int16_t dots[2][GR][NOUT];
    __shared__ __align__(16) float sal[2][ROWS][GR];  // a row's scales of the round together
    __shared__ __align__(16) float swl[2][16 * CB][GR];
    __shared__ float ssink[1];

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int n0 = blockIdx.x * 16 * CB;
    const int G = K >> 7;
    const int R = (G + GR - 1) / GR;  // rounds
    const int KB = K >> 1;
    const int rc = lane & 15, part = lane >> 4;

    // Every global load is a buffer load whose per-thread offset is fixed for
    // the whole kernel; the round enters as a scalar offset, so the ring's
    // address work is scalar.  All offsets are clamped into range.
    // Weights: the column block's K/128 tiled 1 KiB groups (lane l's 16 bytes
    // at l*16), or its rows of the reference layout [N][K/2].
    // With CB column blocks per workgroup their tiled groups are consecutive
    // (block b at b * G KiB); a block past N reads the last one (results dropped).
    const int8_t* wblk = TW ? w + (int64_t)blockIdx.x * CB * G * 1024 : w + (int64_t)n0 * KB;
    const int ncb = TW ? min(CB, (N - n0 + 15) / 16) : 1;  // column blocks of this workgroup inside N
    const __amdgpu_buffer_rsrc_t rsw_w = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(wblk), (short)0, TW ? ncb * G * 1024 : min(16, N - n0) * KB, DC_RSRC_WORD3);
    const int w_voff = TW ? lane * 16 : (min(n0 + rc, N - 1) - n0) * KB + part * 16;
    const int wstep = TW ? 1024 : 64;
    // Activations: thread t moves chunks q = t + DC_T i (row q / CPR, chunk
    // q % CPR of the row's SLB-byte slice).  The slice of round r starts at
    // byte SLB r, moved back so that it ends at the row end when the last
    // round is partial.
    // Row-tiled activations (RT): row block mb of group g is the 1 KiB at
    // (mb * G + g) KiB, lane l's operand bytes at 16 l.
    const __amdgpu_buffer_rsrc_t rsw_a = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(a), (short)0, RT ? MB * G * 1024 : M * KB, DC_RSRC_WORD3);
    int a_voff[RT ? 1 : APT], a_dst[RT ? 1 : APT];
#pragma unroll
    for (int i = 0; i < (RT ? 0 : APT); ++i) {
        const int q = t + i * DC_T;
        const int r = q / CPR, c = q % CPR;
        a_voff[i] = min(r, M - 1) * KB + c * 16;
        a_dst[i] = r * SLB + (((c & ~7) | ((c ^ r) & 7)) << 4);
    }
    auto slice_start = [&](int r) { return max(0, min(r * SLB, KB - SLB)); };

    // Scale staging: entry e < N_SA is sa[row = e/GR][GR r + e%GR] (stored at
    // sal[.][e/GR][e%GR]), then sw.  Whether an entry is sa, sw or nothing is
    // uniform over a wave, so each wave picks one buffer resource; the group
    // index is clamped per thread (a min with a scalar), the rest of the
    // offset is fixed.
    const __amdgpu_buffer_rsrc_t rsw_sa =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(sa), (short)0, M * G * 2, DC_RSRC_WORD3);
    const __amdgpu_buffer_rsrc_t rsw_sw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(sw), (short)0, (SW_GROUPED ? N * G : N) * 2, DC_RSRC_WORD3);
    int s_voff[SPT], sgl[SPT], sstride[SPT];
    float* sdst[SPT];
#pragma unroll
    for (int q = 0; q < SPT; ++q) {
        const int e = t + q * DC_T;
        sgl[q] = e % GR;
        if (e < N_SA) {
            const int row = e / GR;
            s_voff[q] = min(row, M - 1) * G * 2;
            sdst[q] = &sal[0][row][sgl[q]];
            sstride[q] = GR * ROWS;
        } else if (e < N_SA + N_SW) {
            const int col = (e - N_SA) / GR;
            s_voff[q] = min(n0 + col, N - 1) * G * 2;
            sdst[q] = &swl[0][col][sgl[q]];
            sstride[q] = GR * 16 * CB;
        } else {  // nothing to stage: load a valid scale, store to the sink
            s_voff[q] = 0;
            sgl[q] = 0;
            sdst[q] = ssink;
            sstride[q] = 0;
        }
    }

    v4u rw[D][CB], ra[D][NA];
    uint16_t rs[D][SPT];
    auto issue = [&](int r, v4u (&w_out)[CB], v4u (&a_out)[NA], uint16_t (&s_out)[SPT]) {
        const int gw = min(r * GR + wave, G - 1);  // the wave's group of round r
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
            w_out[cb] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(
                                                    rsw_w, w_voff, (min(cb, ncb - 1) * G + gw) * wstep, DC_NT));
        const int rr = min(r, R - 1);        // rounds past the end reload the last one (unused)
        if constexpr (RT) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                a_out[mb] = __builtin_bit_cast(
                    v4u, __builtin_amdgcn_raw_buffer_load_b128(rsw_a, lane * 16, (mb * G + gw) * 1024, 0));
        } else {
            const int aoff = slice_start(rr);
#pragma unroll
            for (int i = 0; i < APT; ++i)
                a_out[i] =
                    __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rsw_a, a_voff[i], aoff, 0));
        }
        const int glast = G - 1 - rr * GR;   // the round's last valid group, relative (>= 0)
#pragma unroll
        for (int q = 0; q < SPT; ++q) {
            const int ew = wave * 64 + q * DC_T;  // scalar: the wave's entry class
            const bool live = ew < N_SA + N_SW;
            const __amdgpu_buffer_rsrc_t rs_q = ew < N_SA || !live ? rsw_sa : rsw_sw;
            s_out[q] = __builtin_amdgcn_raw_buffer_load_b16(rs_q, s_voff[q] + min(sgl[q], glast) * 2,
                                                            live ? rr * GR * 2 : 0, 0);
        }
        // Keep each round's loads together and in round order: loads return
        // in issue order, so a round's data must not queue behind later ones.
        __builtin_amdgcn_sched_barrier(0);
    };
    auto stage_a = [&](int r, const v4u (&a_in)[NA]) {
        if constexpr (!RT) {
#pragma unroll
            for (int i = 0; i < APT; ++i) *reinterpret_cast<v4u*>(&a_l[r & 1][a_dst[i]]) = a_in[i];
        }
    };
    // A-operand LDS offsets: group g's chunk in the slice is 4 j + part with
    // j = (64 g - slice start) / 64 (scalar), so its swizzled position is
    // 128 (j >> 1) + x[j & 1] with x precomputed per lane.
    const int ax0 = rc * SLB + (((part ^ rc) & 7) << 4);
    const int ax1 = rc * SLB + ((((4 + part) ^ rc) & 7) << 4);
    auto mma = [&](int r, const v4u (&w_in)[CB], const v4u (&a_in)[NA], const uint16_t (&s_in)[SPT]) {
        const int buf = r & 1;
        if (r * GR + wave < G) {  // uniform over the wave
            v4u av[MB];  // every operand read issued before the first use
            if constexpr (RT) {
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) av[mb] = a_in[mb];
            } else {
                const int j = ((r * GR + wave) * 64 - slice_start(r)) >> 6;
                const int aoff = buf * (ROWS * SLB) + 128 * (j >> 1) + ((j & 1) ? ax1 : ax0);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
                    av[mb] = *reinterpret_cast<const v4u*>(&a_l[0][aoff + mb * 16 * SLB]);
                __builtin_amdgcn_sched_barrier(0);
            }
            v4i w0[CB], w1[CB];
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                w0[cb] = unpack8_x16(w_in[cb][0], w_in[cb][1]);
                w1[cb] = unpack8_x16(w_in[cb][2], w_in[cb][3]);
            }
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const v4i a0 = unpack8_x16(av[mb][0], av[mb][1]);
                const v4i a1 = unpack8_x16(av[mb][2], av[mb][3]);
#pragma unroll
                for (int cb = 0; cb < CB; ++cb) {
                    v4i acc = {0, 0, 0, 0};
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, w0[cb], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, w1[cb], acc, 0, 0, 0);
                    // 256 * dot -> dot: |dot| <= 8192, so bytes 1..2 of 256 * dot
                    // are the int16 dot; one byte permute packs two of them.
                    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)acc[1], (uint32_t)acc[0], 0x06050201u);
                    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)acc[3], (uint32_t)acc[2], 0x06050201u);
                    *reinterpret_cast<uint2*>(&dots[buf][wave][cb * TOUT + mb * 256 + lane * 4]) = make_uint2(lo, hi);
                }
            }
        }
#pragma unroll
        for (int q = 0; q < SPT; ++q) sdst[q][buf * sstride[q]] = bf16_to_f32(s_in[q]);
    };

    float total[OPT];
#pragma unroll
    for (int oi = 0; oi < OPT; ++oi) total[oi] = 0.0f;
    auto epilogue = [&](int r) {
        const int buf = r & 1;
        const int ng = min(GR, G - r * GR);
#pragma unroll
        for (int oi = 0; oi < OPT; ++oi) {
            const int o = t + oi * DC_T;
            if (o < NOUT) {
                const int l = (o >> 2) & 63, ot = o % TOUT;
                const int row = (ot >> 8) * 16 + 4 * (l >> 4) + (o & 3), col = (o / TOUT) * 16 + (l & 15);
                if (ng == GR) {
                    // All LDS reads first (one wait), then the in-order chain.
                    int dr[GR];
#pragma unroll
                    for (int gl = 0; gl < GR; ++gl) dr[gl] = dots[buf][gl][o];
                    v4f av[GR / 4], wv[GR / 4];
#pragma unroll
                    for (int i = 0; i < GR / 4; ++i) {
                        av[i] = *reinterpret_cast<const v4f*>(&sal[buf][row][4 * i]);
                        wv[i] = v4f{1.0f, 1.0f, 1.0f, 1.0f};
                        if constexpr (SW_GROUPED) wv[i] = *reinterpret_cast<const v4f*>(&swl[buf][col][4 * i]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int gl = 0; gl < GR; ++gl) {
                        const float sa_g = av[gl >> 2][gl & 3];
                        const float s = SW_GROUPED ? sa_g * wv[gl >> 2][gl & 3] : sa_g;
                        total[oi] = __builtin_fmaf((float)dr[gl], s, total[oi]);
                    }
                } else {
                    for (int gl = 0; gl < ng; ++gl) {
                        const float d = (float)dots[buf][gl][o];
                        const float s = SW_GROUPED ? sal[buf][row][gl] * swl[buf][col][gl] : sal[buf][row][gl];
                        total[oi] = __builtin_fmaf(d, s, total[oi]);
                    }
                }
            }
        }
    };

    // Every wave's first-round loads enter the CU's memory pipeline before any
    // wave's later rounds: the pipeline moves ~64 bytes per cycle, and loads
    // of later rounds queued ahead of another wave's first round would hold
    // up the first barrier (qkv / o / down at M = 32: 6.13 / 4.87 / 9.25 ->
    // 5.84 / 4.52 / 9.00 us).
    issue(0, rw[0], ra[0], rs[0]);
    __builtin_amdgcn_s_barrier();
    static_for<1, D>([&](auto U) { issue(U, rw[U], ra[U], rs[U]); });
    if constexpr (!RT) {
        stage_a(0, ra[0]);
        __syncthreads();
    }
    // Steady state: round r uses slot r % D, stages the activation slice of
    // round r + 1 (slot (r+1) % D) and refills slot r % D with round r + D.
    int r0 = 0;
    for (; r0 + D < R; r0 += D) {
        static_for<0, D>([&](auto U) {
            constexpr int u = U, un = (u + 1) % D;
            mma(r0 + u, rw[u], ra[u], rs[u]);
            stage_a(r0 + u + 1, ra[un]);
            issue(r0 + u + D, rw[u], ra[u], rs[u]);
            __syncthreads();
            epilogue(r0 + u);
        });
    }
    // Tail: the last (at most D) rounds are already in flight.
    static_for<0, D>([&](auto U) {
        constexpr int u = U, un = (u + 1) % D;
        if (r0 + u < R) {
            mma(r0 + u, rw[u], ra[u], rs[u]);
            if (r0 + u + 1 < R) stage_a(r0 + u + 1, ra[un]);
            __syncthreads();
            epilogue(r0 + u);
        }
    });

#pragma unroll
    for (int oi = 0; oi < OPT; ++oi) {
        const int o = t + oi * DC_T;
        const int l = (o >> 2) & 63, ot = o % TOUT;
        const int row = (ot >> 8) * 16 + 4 * (l >> 4) + (o & 3), n = n0 + (o / TOUT) * 16 + (l & 15);
        if (o < NOUT && row < M && n < N) {
            float v = total[oi];
            if constexpr (!SW_GROUPED) v = v * bf16_to_f32(sw[n]);
            store_out<OUT_F32>(out, (int64_t)row * N + n, v);
        }
    }
}

// ----------------------------------------------------------------------------
// Wide decode kernel (M <= 32, large N: gate_up).  Each wave owns one 16-row
// block and 16 output columns over the whole K: it streams its weight
// columns group by group through a register ring D groups deep and keeps its
// running totals in registers, so the main loop has no barrier and no LDS
// exchange.  The two row blocks of a column block are separate waves (the
// second wave's weight loads hit the lines the first one brought into the
// CU), which doubles the waves per SIMD that hide each other's MFMA and LDS
// latencies.  The workgroup (CBW column blocks, one workgroup per CU for
// gate_up) first copies into LDS the activation block, already widened to
// MFMA int8 operands (16*q per byte), and the activation and weight scales
// as fp32: every CU fetches and unpacks the activations once instead of once
// per 16-column tile and group, and the main loop issues weight loads only.
//
// LDS activation layout: row r holds K int8 operands (K bytes) as 16-byte
// units; unit u of a row (packed chunk c = u/2 widened: half u%2) is stored
// at unit (u & ~7) | ((u ^ r) & 7), so the 16 rows read by one operand load
// (same unit, rows r..r+15) fall in distinct bank groups.
//
// Per group g the wave does: two operand loads from LDS, 2
// v_mfma_i32_16x16x64_i8, and for each of its 4 outputs (rows 4*(l/16)+i of
// its block, column l%16) total = fmaf(float(dot), sa*sw, total).
// ----------------------------------------------------------------------------
constexpr int WIDE_A_BYTES = 128 * 1024;  // widened activation block limit (M x K bytes)
constexpr int WIDE_SCALES = 1024;         // G * ROWS limit
constexpr int WIDE_WSCALES = 3072;        // G * CBW * 16 limit

template <int MB, int CBW, int D, bool TW, bool RT, bool SW_GROUPED, bool OUT_F32, bool PAIR = false, int GC = 0>
__global__ void __launch_bounds__(CBW * MB * 64)
k2_wide(const int8_t* __restrict__ a, const int8_t* __restrict__ w,
        const uint16_t* __restrict__ sa, const uint16_t* __restrict__ sw,
        void* __restrict__ out, int M, int N, int K) {
    constexpr int T = CBW * MB * 64, ROWS = MB * 16, COLS = CBW * 16;
    static_assert(!PAIR || (CBW % 2 == 0 && !OUT_F32), "gate/up pairs: an even block count, bf16 output");
    constexpr int AC = (WIDE_A_BYTES / 32 + T - 1) / T;  // packed 16-byte chunks per thread (upper bound)
    constexpr int SC = (WIDE_SCALES + T - 1) / T;
    constexpr int WC = SW_GROUPED ? (WIDE_WSCALES + T - 1) / T : 0;
    __shared__ __align__(16) uint8_t a_l[WIDE_A_BYTES + 32];  // + sink
    __shared__ __align__(16) float sa_l[WIDE_SCALES + 4];     // [g][row] + sink
    __shared__ float sw_l[WIDE_WSCALES + 1];                  // [g][col] + sink
    __shared__ uint32_t wave_bad[CBW * MB];                   // scale-range flags, one per wave
    __shared__ float up_l[PAIR ? CBW / 2 * MB * 256 : 1];    // PAIR: the up halves' bf16 results

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int cbl = wave / MB, mb = wave % MB;  // local column block, row block
    // GC > 0: K = 128 GC known at compile time, so the prologue's divisions
    // by G (chunk and scale indices) become shifts and multiplies.
    const int G = GC > 0 ? GC : K >> 7;
    const int KB = G * 64;
    const int chunks_row = KB >> 4;             // packed 16-byte chunks per row
    const int a_chunks = ROWS * chunks_row;
    const int rc = lane & 15, part = lane >> 4;
    // Column block of local block lb: consecutive blocks, or (PAIR) the gate
    // blocks of the workgroup's CBW/2 output blocks followed by the matching
    // up blocks N/32 blocks further (the fused gate/up weight, up rows after
    // gate rows).
    const int HB = N >> 5;  // PAIR: 16-column blocks per half
    auto block_of = [&](int lb) {
        if constexpr (PAIR)
            return lb < CBW / 2 ? blockIdx.x * (CBW / 2) + lb : HB + blockIdx.x * (CBW / 2) + lb - CBW / 2;
        else
            return (int)blockIdx.x * CBW + lb;
    };
    const int col = block_of(cbl) * 16 + rc;
    // Weights: tiled layout [N/16][G][64 lanes][16 bytes] (TW) or [N][K/2].
    const int8_t* wp = TW ? w + (int64_t)min(block_of(cbl), (N >> 4) - 1) * G * 1024 + lane * 16
                          : w + (int64_t)min(col, N - 1) * KB + part * 16;
    constexpr int WSTEP = TW ? 1024 : 64;

    // ---- activation block + scales: loads first, then the weight ring.
    // Packed chunk q (16 bytes): row r, chunk c of the row.  Reference layout:
    // rows of KB bytes; row-tiled layout (RT): the buffer is the MB row blocks'
    // G KiB blocks in order, lane l of block (rb, g) holding chunk 4 g + l/16
    // of row 16 rb + l%16, so chunk q sits at byte 16 q.
    auto chunk_rc = [&](int q, int& r, int& c) {
        if constexpr (RT) {
            // T is a multiple of 64, so the block of a thread's chunk is
            // uniform over its wave: divide on the scalar unit.
            const int l = q & 63, blk = __builtin_amdgcn_readfirstlane(q >> 6);
            r = (blk / G) * 16 + (l & 15);
            c = (blk % G) * 4 + (l >> 4);
        } else {
            r = q / chunks_row;
            c = q - r * chunks_row;
        }
    };
    v4u ra[AC];
    uint16_t rsa[SC], rsw[WC > 0 ? WC : 1];
#pragma unroll
    for (int i = 0; i < AC; ++i) {
        const int q = min(t + i * T, a_chunks - 1);
        int r, c;
        chunk_rc(q, r, c);
        ra[i] = RT ? *reinterpret_cast<const v4u*>(a + (int64_t)q * 16)
                   : *reinterpret_cast<const v4u*>(a + (int64_t)min(r, M - 1) * KB + c * 16);
    }
#pragma unroll
    for (int i = 0; i < SC; ++i) {
        const int e = min(t + i * T, G * ROWS - 1);  // e = row * G + g
        rsa[i] = sa[(int64_t)min(e / G, M - 1) * G + e % G];
    }
#pragma unroll
    for (int i = 0; i < WC; ++i) {
        const int e = min(t + i * T, G * COLS - 1);  // e = local col * G + g
        const int lc = e / G;
        rsw[i] = sw[(int64_t)min(block_of(lc >> 4) * 16 + (lc & 15), N - 1) * G + e % G];
    }
    v4u rw[D];
    auto issue = [&](int g, v4u& w_out) {
        w_out = *reinterpret_cast<const v4u*>(wp + (int64_t)min(g, G - 1) * WSTEP);  // (non-temporal: slower here)
    };
    static_for<0, D>([&](auto U) { issue(U, rw[U]); });
    // Widen and store: packed chunk c of row r -> units 2c, 2c+1.
#pragma unroll
    for (int i = 0; i < AC; ++i) {
        const int q = t + i * T;
        int r, c;
        chunk_rc(min(q, a_chunks - 1), r, c);
        const bool live = q < a_chunks;
        const int u0 = 2 * c, u1 = 2 * c + 1;
        const int s0 = (u0 & ~7) | ((u0 ^ r) & 7), s1 = (u1 & ~7) | ((u1 ^ r) & 7);
        const v4i lo = unpack8_x16(ra[i][0], ra[i][1]);
        const v4i hi = unpack8_x16(ra[i][2], ra[i][3]);
        *reinterpret_cast<v4i*>(&a_l[live ? r * K + s0 * 16 : WIDE_A_BYTES]) = lo;
        *reinterpret_cast<v4i*>(&a_l[live ? r * K + s1 * 16 : WIDE_A_BYTES + 16]) = hi;
    }
    // The >> 8 that turns the MFMA's 256 * dot into the dot can ride on the
    // weight scale instead: cvt(256 d) * sa * (sw * 2^-8) inside the fma is
    // the same exact product as d * (sa * sw) whenever sw * 2^-8 and the
    // scale product stay normal fp32, which holds when every scale of the
    // workgroup is 0 or of magnitude in [2^-59, 2^63).  Each wave flags the
    // scales it staged; after the prologue's barrier the workgroup folds only
    // if no wave flagged one, else it runs the literal sequence.  (Grouped
    // weight scales only; not with 8 column blocks, whose second loop body
    // would not fit 128 VGPRs.)
    auto fold_ok = [](uint32_t b) {
        const uint32_t e = (b >> 7) & 0xffu;
        return (b & 0x7fffu) == 0 || (e >= 127 - 59 && e < 127 + 63);
    };
    bool bad = false;
#pragma unroll
    for (int i = 0; i < SC; ++i) bad |= !fold_ok(rsa[i]);
#pragma unroll
    for (int i = 0; i < WC; ++i) bad |= !fold_ok(rsw[i]);
    const bool wave_flag = __builtin_amdgcn_ballot_w64(bad) != 0;
    if (lane == 0) wave_bad[wave] = wave_flag ? 1u : 0u;
#pragma unroll
    for (int i = 0; i < SC; ++i) {
        const int e = t + i * T;
        const int ec = min(e, G * ROWS - 1);
        sa_l[e < G * ROWS ? (ec % G) * ROWS + ec / G : WIDE_SCALES] = bf16_to_f32(rsa[i]);
    }
#pragma unroll
    for (int i = 0; i < WC; ++i) {
        const int e = t + i * T;
        const int ec = min(e, G * COLS - 1);
        sw_l[e < G * COLS ? (ec % G) * COLS + ec / G : WIDE_WSCALES] = bf16_to_f32(rsw[i]);
    }
    __syncthreads();
    bool fold = SW_GROUPED && CBW < 8;
#pragma unroll
    for (int i = 0; i < CBW * MB; ++i) fold = fold && wave_bad[i] == 0;

    float total[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int r = mb * 16 + rc;
    const float* sap = &sa_l[mb * 16 + 4 * part];
    const float* swq = &sw_l[cbl * 16 + rc];

    // A group's LDS operands (two activation operands, the four rows'
    // activation scales, the column's weight scale) are read one group ahead
    // of their use, so the wave's MFMAs never wait on an LDS round trip.
    struct Ops {
        v4i a0, a1;
        v4f s_a;
        float s_w;
    };
    auto lds_ops = [&](int g, Ops& o) {
        const int u0 = (g * 4 + part) * 2, u1 = u0 + 1;
        o.a0 = *reinterpret_cast<const v4i*>(&a_l[r * K + (((u0 & ~7) | ((u0 ^ r) & 7)) << 4)]);
        o.a1 = *reinterpret_cast<const v4i*>(&a_l[r * K + (((u1 & ~7) | ((u1 ^ r) & 7)) << 4)]);
        o.s_a = *reinterpret_cast<const v4f*>(sap + g * ROWS);
        o.s_w = SW_GROUPED ? swq[g * COLS] : 1.0f;
    };
    // FOLD: the column's weight scale carries the 2^-8 and the dot is taken
    // as 256 d.
    auto main_loop = [&](auto FOLD) {
        auto consume = [&](const v4u& w_in, const Ops& o) {
            const v4i w0 = unpack8_x16(w_in[0], w_in[1]);
            const v4i w1 = unpack8_x16(w_in[2], w_in[3]);
            v4i acc = {0, 0, 0, 0};
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.a0, w0, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.a1, w1, acc, 0, 0, 0);
            const float s_w = FOLD ? o.s_w * 0x1p-8f : o.s_w;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float d = FOLD ? (float)acc[i] : (float)(acc[i] >> 8);
                total[i] = SW_GROUPED ? __builtin_fmaf(d, o.s_a[i] * s_w, total[i])
                                      : __builtin_fmaf(d, o.s_a[i], total[i]);
            }
        };
        Ops cur;
        lds_ops(0, cur);
        int g0 = 0;
        for (; g0 + D < G; g0 += D) {
            static_for<0, D>([&](auto U) {
                Ops nxt;
                lds_ops(g0 + U + 1, nxt);  // g0 + U + 1 < G inside the loop
                __builtin_amdgcn_sched_barrier(0);
                consume(rw[U], cur);
                issue(g0 + U + D, rw[U]);
                cur = nxt;
            });
        }
        static_for<0, D>([&](auto U) {
            if (g0 + U < G) {
                Ops nxt;
                lds_ops(min(g0 + U + 1, G - 1), nxt);
                __builtin_amdgcn_sched_barrier(0);
                consume(rw[U], cur);
                cur = nxt;
            }
        });
    };
    if constexpr (SW_GROUPED && CBW < 8) {
        if (fold) {
            main_loop(std::true_type{});
        } else {
            main_loop(std::false_type{});
        }
    } else {
        main_loop(std::false_type{});
    }

    if constexpr (PAIR) {
        // y = silu(g) * u on the bf16 results of the paired gate and up
        // columns, as the separate SiLU-and-mul would compute it from the
        // stored [M, N] output; y is [M, N/2].
        float swn = 1.0f;
        if constexpr (!SW_GROUPED) swn = bf16_to_f32(sw[min(col, N - 1)]);
        float vb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) vb[i] = round_bf16(SW_GROUPED ? total[i] : total[i] * swn);
        if (cbl >= CBW / 2)
            *reinterpret_cast<v4f*>(&up_l[((cbl - CBW / 2) * MB + mb) * 256 + lane * 4]) = v4f{vb[0], vb[1], vb[2], vb[3]};
        __syncthreads();
        if (cbl < CBW / 2 && col < N / 2) {
            const v4f u = *reinterpret_cast<const v4f*>(&up_l[(cbl * MB + mb) * 256 + lane * 4]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = mb * 16 + 4 * part + i;
                if (row < M) store_out<false>(out, (int64_t)row * (N / 2) + col, silu_mul1(vb[i], u[i]));
            }
        }
    } else if (col < N) {
        float swn = 1.0f;
        if constexpr (!SW_GROUPED) swn = bf16_to_f32(sw[col]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = mb * 16 + 4 * part + i;
            if (row < M) {
                float v = total[i];
                if constexpr (!SW_GROUPED) v = v * swn;
                store_out<OUT_F32>(out, (int64_t)row * N + col, v);
            }
        }
    }
}

template <int MB, bool TW, bool RT, bool SG, bool OF>
hipError_t launch_dec(const int8_t* a, const int8_t* w, const void* sa, const void* sw, void* out,
                      int M, int N, int K, hipStream_t st) {
    const int blocks = (N + 15) / 16;
    const dim3 grid((unsigned)blocks);
    const auto* sap = static_cast<const uint16_t*>(sa);
    const auto* swp = static_cast<const uint16_t*>(sw);
    // When one workgroup per CU covers every column block, 16 waves with a
    // two-round ring (16 groups per round) hide more latency than 8 waves;
    // with more column blocks than CUs, two 8-wave workgroups share a CU.
    // With more 16-column blocks than CUs (some CUs would run two workgroups,
    // each reading all M x K activations) and tiled weights, a workgroup takes
    // two column blocks instead: the activations are read once per CU.
    if constexpr (MB <= 2) {
        const int cus = device_cu_count();
        if (K >= 2048 && blocks <= cus) {
            hipLaunchKernelGGL((k2_dec<MB, 16, 2, TW, RT, SG, OF>), grid, dim3(16 * 64), 0, st, a, w, sap, swp, out, M,
                               N, K);
            return hipGetLastError();
        }
        if constexpr (TW) {
            if (K >= 2048 && (blocks + 1) / 2 <= cus) {
                hipLaunchKernelGGL((k2_dec<MB, 16, 2, TW, RT, SG, OF, 2>), dim3((unsigned)((blocks + 1) / 2)),
                                   dim3(16 * 64), 0, st, a, w, sap, swp, out, M, N, K);
                return hipGetLastError();
            }
        }
    }
    constexpr int D = 4;  // rounds in flight: all of them for K <= 4096
    hipLaunchKernelGGL((k2_dec<MB, 8, D, TW, RT, SG, OF>), grid, dim3(8 * 64), 0, st, a, w, sap, swp, out, M, N, K);
    return hipGetLastError();
}

// The wide kernel needs the widened activation block and the scales to fit
// in LDS, whole 8-chunk lines per row (swizzle), and at least 4 column blocks
// per CU.
bool wide_fits(int M, int N, int K) {
    const int mb = (M + 15) / 16;
    const int per_cu = ((N + 15) / 16 + device_cu_count() - 1) / device_cu_count();
    return M <= 32 && K % 256 == 0 && (int64_t)mb * 16 * K <= WIDE_A_BYTES &&
           (int64_t)(K / 128) * mb * 16 <= WIDE_SCALES && per_cu >= 4 && per_cu <= 8 &&
           (int64_t)(K / 128) * 16 * (per_cu <= 4 ? 4 : per_cu <= 6 ? 6 : 8) <= WIDE_WSCALES;
}

template <int MB, int CBW, bool TW, bool RT, bool SG, bool OF, bool PAIR = false>
hipError_t launch_wide_cbw(const int8_t* a, const int8_t* w, const void* sa, const void* sw, void* out,
                           int M, int N, int K, hipStream_t st) {
    constexpr int D = 8;  // groups in flight per wave
    // PAIR: CBW/2 output blocks of 16 (gate and up block each) per workgroup.
    const int nb = PAIR ? N / 32 : (N + 15) / 16, per = PAIR ? CBW / 2 : CBW;
    const dim3 grid((unsigned)((nb + per - 1) / per)), block(CBW * MB * 64);
    const auto* sap = static_cast<const uint16_t*>(sa);
    const auto* swp = static_cast<const uint16_t*>(sw);
    if (K == 4096)  // the decoder's hidden size: group count known at compile time
        hipLaunchKernelGGL((k2_wide<MB, CBW, D, TW, RT, SG, OF, PAIR, 32>), grid, block, 0, st, a, w, sap, swp, out,
                           M, N, K);
    else
        hipLaunchKernelGGL((k2_wide<MB, CBW, D, TW, RT, SG, OF, PAIR>), grid, block, 0, st, a, w, sap, swp, out, M,
                           N, K);
    return hipGetLastError();
}

template <int MB, bool TW, bool RT, bool SG, bool OF, bool PAIR = false>
hipError_t launch_wide(const int8_t* a, const int8_t* w, const void* sa, const void* sw, void* out,
                       int M, int N, int K, hipStream_t st) {
    // Column blocks per workgroup: enough that one workgroup per CU covers N.
    const int per_cu = ((N + 15) / 16 + device_cu_count() - 1) / device_cu_count();
    if (per_cu <= 4) return launch_wide_cbw<MB, 4, TW, RT, SG, OF, PAIR>(a, w, sa, sw, out, M, N, K, st);
    if (per_cu <= 6) return launch_wide_cbw<MB, 6, TW, RT, SG, OF, PAIR>(a, w, sa, sw, out, M, N, K, st);
    return launch_wide_cbw<MB, 8, TW, RT, SG, OF, PAIR>(a, w, sa, sw, out, M, N, K, st);
}

template <bool TW, bool SG, bool OF>
hipError_t dispatch(const int8_t* a, const int8_t* w, const void* sa, const void* sw, void* out,
                    int M, int N, int K, hipStream_t st) {
    // Wide N: waves own column blocks, activations fetched once per CU.
    if (wide_fits(M, N, K)) {
        return M <= 16 ? launch_wide<1, TW, false, SG, OF>(a, w, sa, sw, out, M, N, K, st)
                       : launch_wide<2, TW, false, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    }
    if (M <= 16) return launch_dec<1, TW, false, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    if (M <= 32) return launch_dec<2, TW, false, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    if (M <= 48) return launch_dec<3, TW, false, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    if (M <= 64) return launch_dec<4, TW, false, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    return k2_prefill_launch(a, w, sa, sw, SG, out, OF, TW, M, N, K, st);
}

// Row-tiled activations (M <= 32) on tiled weights.
template <bool SG, bool OF>
hipError_t dispatch_rt(const int8_t* a, const int8_t* w, const void* sa, const void* sw, void* out,
                       int M, int N, int K, hipStream_t st) {
    if (wide_fits(M, N, K)) {
        return M <= 16 ? launch_wide<1, true, true, SG, OF>(a, w, sa, sw, out, M, N, K, st)
                       : launch_wide<2, true, true, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    }
    return M <= 16 ? launch_dec<1, true, true, SG, OF>(a, w, sa, sw, out, M, N, K, st)
                   : launch_dec<2, true, true, SG, OF>(a, w, sa, sw, out, M, N, K, st);
}

// MFMA-tiled weight layout <-> reference layout [N][K/2]: 16-byte unit
// u = (cb*G + g)*64 + l of the tiled buffer is bytes 64 g + 16 (l/16) ..
// +15 of column 16 cb + l%16.  One thread per unit, both directions.
template <bool TO_TILED>
__global__ void __launch_bounds__(256)
tile_weights(const int8_t* __restrict__ src, int8_t* __restrict__ dst, int64_t units, int G, int KB) {
    const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (u >= units) return;
    const int l = (int)(u & 63);
    const int64_t cg = u >> 6;  // cb * G + g
    const int64_t cb = cg / G;
    const int g = (int)(cg - cb * G);
    const int64_t ref = (cb * 16 + (l & 15)) * KB + g * 64 + (l >> 4) * 16;
    if constexpr (TO_TILED)
        *reinterpret_cast<v4u*>(dst + u * 16) = *reinterpret_cast<const v4u*>(src + ref);
    else
        *reinterpret_cast<v4u*>(dst + ref) = *reinterpret_cast<const v4u*>(src + u * 16);
}

int gemm_impl(const int8_t* a, const int8_t* w, const void* sa, const void* sw, int sw_grouped, void* out,
              int out_fp32, bool tiled, bool rowtiled, int64_t M, int64_t N, int64_t K, void* stream) {
    if (!a || !w || !sa || !sw || !out) return NV4_E_NULL;
    if (M < 1 || N < 1 || K < 128 || K % 128 || N % 8 || (tiled && N % 16)) return NV4_E_SHAPE;
    if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > (1LL << 20)) return NV4_E_SHAPE;
    if (rowtiled && (M > 32 || !tiled)) return NV4_E_SHAPE;
    if (M * (K / 128) > 0x7fffffffLL || N * (K / 128) > 0x7fffffffLL) return NV4_E_SHAPE;
    if (((M + 127) / 128) * ((N + 127) / 128) > 0x7fffffffLL) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(a) % 16 || reinterpret_cast<uintptr_t>(w) % 16 ||
        reinterpret_cast<uintptr_t>(sa) % 2 || reinterpret_cast<uintptr_t>(sw) % 2 ||
        reinterpret_cast<uintptr_t>(out) % (out_fp32 ? 4 : 2))
        return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int m = (int)M, n = (int)N, k = (int)K;
    hipError_t e;
    if (rowtiled) {
        if (sw_grouped)
            e = out_fp32 ? dispatch_rt<true, true>(a, w, sa, sw, out, m, n, k, st)
                         : dispatch_rt<true, false>(a, w, sa, sw, out, m, n, k, st);
        else
            e = out_fp32 ? dispatch_rt<false, true>(a, w, sa, sw, out, m, n, k, st)
                         : dispatch_rt<false, false>(a, w, sa, sw, out, m, n, k, st);
    } else if (tiled) {
        if (sw_grouped)
            e = out_fp32 ? dispatch<true, true, true>(a, w, sa, sw, out, m, n, k, st)
                         : dispatch<true, true, false>(a, w, sa, sw, out, m, n, k, st);
        else
            e = out_fp32 ? dispatch<true, false, true>(a, w, sa, sw, out, m, n, k, st)
                         : dispatch<true, false, false>(a, w, sa, sw, out, m, n, k, st);
    } else {
        if (sw_grouped)
            e = out_fp32 ? dispatch<false, true, true>(a, w, sa, sw, out, m, n, k, st)
                         : dispatch<false, true, false>(a, w, sa, sw, out, m, n, k, st);
        else
            e = out_fp32 ? dispatch<false, false, true>(a, w, sa, sw, out, m, n, k, st)
                         : dispatch<false, false, false>(a, w, sa, sw, out, m, n, k, st);
    }
    return (int)e;
}

int linear_impl(const void* x, const int8_t* signs, const int8_t* w, const void* sw, void* out,
                int8_t* a_packed, void* a_scale, bool tiled, bool rowtiled, int64_t M, int64_t N, int64_t K,
                void* stream) {
    if (!x || !signs || !w || !sw || !out || !a_packed || !a_scale) return NV4_E_NULL;
    if (K != 4096 && K != 12288) return NV4_E_SHAPE;
    if (N < 1 || N % 8 || (tiled && N % 16)) return NV4_E_SHAPE;  // checked before K1 runs
    if (rowtiled && (M < 1 || M > 32)) return NV4_E_SHAPE;
    // Decode-sized calls: K1's idle CUs read the head of the weights ahead of
    // the GEMM (into the Infinity Cache; see the prefetch tail of K1).
    const int64_t pf = nv4_w4a4_prefetch_bytes(N, K);
    const int rc = rowtiled ? nv4_rht_quant_pack_rowtiled(x, signs, a_packed, a_scale, M, K, pf > 0 ? w : nullptr,
                                                          pf, stream)
                            : nv4_rht_quant_pack(x, signs, a_packed, a_scale, M, K, NV4_LAYOUT_REFERENCE, stream);
    if (rc != NV4_OK) return rc;
    return gemm_impl(a_packed, w, a_scale, sw, 1, out, 0, tiled, rowtiled, M, N, K, stream);
}

int tile_impl(const int8_t* src, int8_t* dst, bool to_tiled, int64_t N, int64_t K, void* stream) {
    if (!src || !dst) return NV4_E_NULL;
    if (N < 16 || N % 16 || K < 128 || K % 128 || K > (1LL << 20) || N > 0x7fffffffLL) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(src) % 16 || reinterpret_cast<uintptr_t>(dst) % 16) return NV4_E_ALIGN;
    const int64_t units = N * K / 32;
    if ((units + 255) / 256 > 0x7fffffffLL) return NV4_E_SHAPE;
    const dim3 grid((unsigned)((units + 255) / 256));
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (to_tiled)
        hipLaunchKernelGGL(tile_weights<true>, grid, dim3(256), 0, st, src, dst, units, (int)(K / 128), (int)(K / 2));
    else
        hipLaunchKernelGGL(tile_weights<false>, grid, dim3(256), 0, st, src, dst, units, (int)(K / 128), (int)(K / 2));
    return (int)hipGetLastError();
}

}  // namespace
}  // namespace nv4

extern "C" int64_t nv4_w4a4_prefetch_bytes(int64_t N, int64_t K) {
    // How much of a decode GEMM's packed weights the K1 before it reads
    // ahead.  Measured on the Qwen3-8B projections at M = 32 (K1 + GEMM per
    // call, graph replays over weight sets larger than the Infinity Cache):
    // a weight read whole beats a head of it (the GEMM then waits on no HBM
    // tail): down's 25 MB after K1 at K = 12288 (15.1 -> 13.3 us), o's 8.4 MB
    // (7.6-7.7 with 6 MB -> 7.2 us); gate_up's 50 MB is best at 9 MB (16.2
    // without, 15.4-16.0 with 6 MB, 15.3 with 9 MB, and 4.5 us slower whole);
    // qkv's 12.6 MB stays within 0.1 us from none to 6 MB (9 MB: +0.4 us).
    if (N < 1 || K < 128 || K % 128 || N > (1LL << 31) || K > (1LL << 20)) return 0;
    const int64_t bytes = N * K / 2;
    const int64_t cap = K >= 12288 || bytes <= (9LL << 20) ? (32LL << 20)
                        : bytes > (24LL << 20)             ? (9LL << 20)
                                                           : (6LL << 20);
    return bytes < cap ? bytes : cap;
}

extern "C" int nv4_w4a4_linear(const void* x, const int8_t* signs, const int8_t* w, const void* sw,
                               void* out, int8_t* a_packed, void* a_scale,
                               int64_t M, int64_t N, int64_t K, void* stream) {
    return nv4::linear_impl(x, signs, w, sw, out, a_packed, a_scale, false, false, M, N, K, stream);
}

extern "C" int nv4_w4a4_linear_tiled(const void* x, const int8_t* signs, const int8_t* w_tiled, const void* sw,
                                     void* out, int8_t* a_packed, void* a_scale,
                                     int64_t M, int64_t N, int64_t K, void* stream) {
    return nv4::linear_impl(x, signs, w_tiled, sw, out, a_packed, a_scale, true, false, M, N, K, stream);
}

extern "C" int nv4_w4a4_linear_rowtiled(const void* x, const int8_t* signs, const int8_t* w_tiled, const void* sw,
                                        void* out, int8_t* a_packed_rt, void* a_scale,
                                        int64_t M, int64_t N, int64_t K, void* stream) {
    return nv4::linear_impl(x, signs, w_tiled, sw, out, a_packed_rt, a_scale, true, true, M, N, K, stream);
}

extern "C" int nv4_w4a4_gemm(const int8_t* a, const int8_t* w, const void* sa, const void* sw,
                             int sw_grouped, void* out, int out_fp32,
                             int64_t M, int64_t N, int64_t K, void* stream) {
    return nv4::gemm_impl(a, w, sa, sw, sw_grouped, out, out_fp32, false, false, M, N, K, stream);
}

extern "C" int nv4_w4a4_gemm_tiled(const int8_t* a, const int8_t* w_tiled, const void* sa, const void* sw,
                                   int sw_grouped, void* out, int out_fp32,
                                   int64_t M, int64_t N, int64_t K, void* stream) {
    return nv4::gemm_impl(a, w_tiled, sa, sw, sw_grouped, out, out_fp32, true, false, M, N, K, stream);
}

extern "C" int nv4_w4a4_gemm_rowtiled(const int8_t* a_rt, const int8_t* w_tiled, const void* sa, const void* sw,
                                      int sw_grouped, void* out, int out_fp32,
                                      int64_t M, int64_t N, int64_t K, void* stream) {
    return nv4::gemm_impl(a_rt, w_tiled, sa, sw, sw_grouped, out, out_fp32, true, true, M, N, K, stream);
}

extern "C" int nv4_w4a4_gemm_rowtiled_silu(const int8_t* a_rt, const int8_t* w_tiled, const void* sa, const void* sw,
                                           int sw_grouped, void* out, int64_t M, int64_t N, int64_t K,
                                           void* stream) {
    using namespace nv4;
    if (!a_rt || !w_tiled || !sa || !sw || !out) return NV4_E_NULL;
    if (M < 1 || M > 32 || N < 32 || N % 32 || K < 128 || K % 128 || N > 0x7fffffffLL || K > (1LL << 20))
        return NV4_E_SHAPE;
    if (N * (K / 128) > 0x7fffffffLL || !wide_fits((int)M, (int)N, (int)K)) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(a_rt) % 16 || reinterpret_cast<uintptr_t>(w_tiled) % 16 ||
        reinterpret_cast<uintptr_t>(sa) % 2 || reinterpret_cast<uintptr_t>(sw) % 2 ||
        reinterpret_cast<uintptr_t>(out) % 2)
        return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int m = (int)M, n = (int)N, k = (int)K;
    hipError_t e;
    if (sw_grouped)
        e = m <= 16 ? launch_wide<1, true, true, true, false, true>(a_rt, w_tiled, sa, sw, out, m, n, k, st)
                    : launch_wide<2, true, true, true, false, true>(a_rt, w_tiled, sa, sw, out, m, n, k, st);
    else
        e = m <= 16 ? launch_wide<1, true, true, false, false, true>(a_rt, w_tiled, sa, sw, out, m, n, k, st)
                    : launch_wide<2, true, true, false, false, true>(a_rt, w_tiled, sa, sw, out, m, n, k, st);
    return (int)e;
}

extern "C" int nv4_w4a4_tile_weights(const int8_t* w, int8_t* w_tiled, int64_t N, int64_t K, void* stream) {
    return nv4::tile_impl(w, w_tiled, true, N, K, stream);
}

extern "C" int nv4_w4a4_untile_weights(const int8_t* w_tiled, int8_t* w, int64_t N, int64_t K, void* stream) {
    return nv4::tile_impl(w_tiled, w, false, N, K, stream);
}

