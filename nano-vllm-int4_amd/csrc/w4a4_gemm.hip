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
// Three kernels, no split-K, no atomics:
//  * k2_decode (M <= 64): one workgroup per 16 (or 32) output columns and all
//    M rows.  Its eight waves each take one K-group per sub-round, compute
//    the exact int32 group dots with v_mfma_i32_16x16x64_i8 and hand them to
//    the whole workgroup through LDS, which runs the fp32 epilogue in group
//    order.  Loads run several sub-rounds ahead.  The weight stream
//    (N*K/2 bytes) dominates, so this kernel is HBM-bound.
//  * k2_wide (M <= 32, wide N): waves own column blocks over the whole K,
//    activations widened once per CU into LDS.
//  * k2_prefill (M > 64, w4a4_prefill.hip): LDS-staged 128x128 tiles.
#include "k2_launch.h"
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
// Decode kernel (M <= 64).  Workgroup = 8 waves, output tile = all M rows
// (MB blocks of 16) x BN = 16*NB columns, whole K.  Groups are handed out in
// sub-rounds of 8: in sub-round j wave w computes the exact int32 dots of
// group 8j+w for the whole tile, the dots go through LDS, and every thread
// then runs the in-order fp32 epilogue of those 8 groups for the outputs it
// owns.  Loads run D sub-rounds ahead of use in a register ring; for
// K = 4096 every byte the workgroup needs is requested before the first MFMA.
//
// Weights go straight from the ring into MFMA operands: lane l loads 16 bytes
// of column l%16 (a quarter of the group's 64 bytes).  The activation slice
// of a sub-round (all rows x 512 bytes) is shared by the eight waves, so it
// is loaded cooperatively in whole 128-byte lines (8 lanes per line), staged
// in LDS one sub-round ahead and read back as MFMA operands: half-line
// per-lane loads would double the L1 misses of the activation re-reads, which
// every workgroup of the launch makes.
//
// MFMA 16x16x64 i8 layout used here (checked by the parity tests):
//   A operand: lane l supplies row l%16, B operand: lane l supplies column
//   l%16; both take the same 16 k-slots (set l/16), so identical unpacking
//   pairs every k.  Result: lane l holds C[4*(l/16) + i][l%16], i = 0..3.
// LDS activation slice: row r at r*512 bytes, its 16-byte chunk c stored at
// chunk (c & ~7) | ((c ^ r) & 7), so the 16 rows of one operand load fall in
// distinct bank groups.
//
// Every global load is unconditional (indices clamped into range): a load
// under a thread-dependent branch makes the compiler drain all outstanding
// loads at the branch join, which would serialise the ring.
// ----------------------------------------------------------------------------
constexpr int DEC_WAVES = 8;
constexpr int DEC_THREADS = DEC_WAVES * 64;

template <int MB, int NB, int D, bool SW_GROUPED, bool OUT_F32>
__global__ void __launch_bounds__(DEC_THREADS)
k2_decode(const int8_t* __restrict__ a, const int8_t* __restrict__ w,
          const uint16_t* __restrict__ sa, const uint16_t* __restrict__ sw,
          void* __restrict__ out, int M, int N, int K) {
    constexpr int BN = 16 * NB, NBLK = MB * NB, ROWS = MB * 16;
    constexpr int OPT = (NBLK * 256 + DEC_THREADS - 1) / DEC_THREADS;  // outputs per thread
    constexpr int N_SA = ROWS * 8;                                      // scale entries per sub-round
    constexpr int N_SW = SW_GROUPED ? BN * 8 : 0;
    constexpr int SPT = (N_SA + N_SW + DEC_THREADS - 1) / DEC_THREADS;  // scale entries per thread
    constexpr int APT = ROWS * 32 / DEC_THREADS;                        // activation chunks per thread (= MB)
    __shared__ __align__(16) uint8_t a_l[2][ROWS * 512];
    __shared__ int16_t dots[2][8][NBLK][256];
    __shared__ float sal[2][8][ROWS];
    __shared__ float swl[2][8][BN];
    __shared__ float ssink[1];

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int n0 = blockIdx.x * BN;
    const int G = K >> 7;
    const int S = (G + 7) >> 3;  // sub-rounds
    const int KB = K >> 1;       // packed bytes per row

    const int rc = lane & 15, part = lane >> 4;
    const int8_t* wp[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
        wp[nb] = w + (int64_t)min(n0 + nb * 16 + rc, N - 1) * KB + part * 16;

    // Activation staging: thread t moves chunks q = t + 512 i (row q/32,
    // chunk q%32 of the row's 512-byte slice).
    const int8_t* arow[APT];
    int a_c16[APT], a_dst[APT];
#pragma unroll
    for (int i = 0; i < APT; ++i) {
        const int q = t + i * DEC_THREADS;
        const int r = q >> 5, c = q & 31;
        arow[i] = a + (int64_t)min(r, M - 1) * KB;
        a_c16[i] = c * 16;
        a_dst[i] = r * 512 + (((c & ~7) | ((c ^ r) & 7)) << 4);
    }
    // Start of the 512-byte slice staged for sub-round j: 512 j, moved back
    // so that it ends at the row end when the last sub-round is partial.
    auto slice_start = [&](int j) { return max(0, min(j * 512, KB - 512)); };

    // Scale staging: entry e < N_SA is sa[row = e/8][8j + e%8], then sw.
    const uint16_t* sp[SPT];
    float* sdst[SPT];
    int sgl[SPT], sstride[SPT];
#pragma unroll
    for (int q = 0; q < SPT; ++q) {
        const int e = t + q * DEC_THREADS;
        sgl[q] = e & 7;
        if (e < N_SA) {
            const int row = e >> 3;
            sp[q] = sa + (int64_t)min(row, M - 1) * G;
            sdst[q] = &sal[0][sgl[q]][row];
            sstride[q] = 8 * ROWS;
        } else if (e < N_SA + N_SW) {
            const int col = (e - N_SA) >> 3;
            sp[q] = sw + (int64_t)min(n0 + col, N - 1) * G;
            sdst[q] = &swl[0][sgl[q]][col];
            sstride[q] = 8 * BN;
        } else {  // nothing to stage: load a valid scale, store to the sink
            sp[q] = sa;
            sdst[q] = ssink;
            sstride[q] = 0;
        }
    }

    v4u rw[D][NB], ra[D][APT];
    uint16_t rs[D][SPT];

    auto issue = [&](int j, v4u (&w_out)[NB], v4u (&a_out)[APT], uint16_t (&s_out)[SPT]) {
        const int64_t g = min(j * 8 + wave, G - 1);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) w_out[nb] = *reinterpret_cast<const v4u*>(wp[nb] + g * 64);
        const int aoff = slice_start(min(j, S - 1));
#pragma unroll
        for (int i = 0; i < APT; ++i)
            a_out[i] = *reinterpret_cast<const v4u*>(arow[i] + min(aoff + a_c16[i], KB - 16));
#pragma unroll
        for (int q = 0; q < SPT; ++q) s_out[q] = sp[q][min(j * 8 + sgl[q], G - 1)];
    };
    auto stage_a = [&](int j, const v4u (&a_in)[APT]) {
#pragma unroll
        for (int i = 0; i < APT; ++i) *reinterpret_cast<v4u*>(&a_l[j & 1][a_dst[i]]) = a_in[i];
    };

    float total[OPT];
#pragma unroll
    for (int oi = 0; oi < OPT; ++oi) total[oi] = 0.0f;

    auto consume = [&](int j, const v4u (&w_in)[NB], const v4u (&a_next)[APT], const uint16_t (&s_in)[SPT]) {
        const int buf = j & 1;
        const int g = j * 8 + wave;
        if (g < G) {  // uniform over the wave
            // Chunk of this group inside the staged slice.
            const int shift = j * 512 - slice_start(j);  // bytes the slice was moved back
            const int cbase = (wave * 64 + shift) >> 4;
            v4i w0[NB], w1[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                w0[nb] = unpack8_x16(w_in[nb][0], w_in[nb][1]);
                w1[nb] = unpack8_x16(w_in[nb][2], w_in[nb][3]);
            }
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int r = mb * 16 + rc;
                const int c = cbase + part;
                const v4u av = *reinterpret_cast<const v4u*>(
                    &a_l[buf][r * 512 + (((c & ~7) | ((c ^ r) & 7)) << 4)]);
                const v4i a0 = unpack8_x16(av[0], av[1]);
                const v4i a1 = unpack8_x16(av[2], av[3]);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    v4i acc = {0, 0, 0, 0};
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, w0[nb], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, w1[nb], acc, 0, 0, 0);
                    // 256 * dot -> dot (exact); |dot| <= 8192 fits int16.
                    const uint32_t lo = ((uint32_t)(acc[0] >> 8) & 0xffffu) | ((uint32_t)(acc[1] >> 8) << 16);
                    const uint32_t hi = ((uint32_t)(acc[2] >> 8) & 0xffffu) | ((uint32_t)(acc[3] >> 8) << 16);
                    *reinterpret_cast<uint2*>(&dots[buf][wave][mb * NB + nb][lane * 4]) = make_uint2(lo, hi);
                }
            }
        }
#pragma unroll
        for (int q = 0; q < SPT; ++q) sdst[q][buf * sstride[q]] = bf16_to_f32(s_in[q]);
        if (j + 1 < S) stage_a(j + 1, a_next);  // uniform
        __syncthreads();
        const int ng = min(8, G - j * 8);  // groups in this sub-round
#pragma unroll
        for (int oi = 0; oi < OPT; ++oi) {
            const int o = t + oi * DEC_THREADS;
            if (o < NBLK * 256) {
                const int row = o / BN, col = o % BN;
                const int blk = (row >> 4) * NB + (col >> 4);
                const int e = ((((row & 15) >> 2) * 16 + (col & 15)) << 2) + (row & 3);
                if (ng == 8) {
                    float d[8], s[8];
#pragma unroll
                    for (int gl = 0; gl < 8; ++gl) {
                        d[gl] = (float)dots[buf][gl][blk][e];
                        s[gl] = SW_GROUPED ? sal[buf][gl][row] * swl[buf][gl][col] : sal[buf][gl][row];
                    }
#pragma unroll
                    for (int gl = 0; gl < 8; ++gl) total[oi] = __builtin_fmaf(d[gl], s[gl], total[oi]);
                } else {
                    for (int gl = 0; gl < ng; ++gl) {
                        const float d = (float)dots[buf][gl][blk][e];
                        const float s = SW_GROUPED ? sal[buf][gl][row] * swl[buf][gl][col] : sal[buf][gl][row];
                        total[oi] = __builtin_fmaf(d, s, total[oi]);
                    }
                }
            }
        }
    };

    static_for<0, D>([&](auto U) { issue(U, rw[U], ra[U], rs[U]); });
    stage_a(0, ra[0]);
    __syncthreads();

    // Steady state: consume a slot, refill it D sub-rounds ahead.  The
    // activation slice of sub-round j+1 (slot u+1) is staged during j.
    int j0 = 0;
    for (; j0 + D < S; j0 += D) {
        static_for<0, D>([&](auto U) {
            constexpr int u = U, un = (u + 1) % D;
            consume(j0 + u, rw[u], ra[un], rs[u]);
            issue(j0 + u + D, rw[u], ra[u], rs[u]);
        });
    }
    // Tail: the last (at most D) sub-rounds are already in flight.
    static_for<0, D>([&](auto U) {
        constexpr int u = U, un = (u + 1) % D;
        if (j0 + u < S) consume(j0 + u, rw[u], ra[un], rs[u]);
    });

#pragma unroll
    for (int oi = 0; oi < OPT; ++oi) {
        const int o = t + oi * DEC_THREADS;
        const int row = o / BN, col = o % BN;
        const int n = n0 + col;
        if (o < NBLK * 256 && row < M && n < N) {
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

template <int MB, int CBW, int D, bool SW_GROUPED, bool OUT_F32>
__global__ void __launch_bounds__(CBW * MB * 64)
k2_wide(const int8_t* __restrict__ a, const int8_t* __restrict__ w,
        const uint16_t* __restrict__ sa, const uint16_t* __restrict__ sw,
        void* __restrict__ out, int M, int N, int K) {
    constexpr int T = CBW * MB * 64, ROWS = MB * 16, COLS = CBW * 16;
    constexpr int AC = (WIDE_A_BYTES / 32 + T - 1) / T;  // packed 16-byte chunks per thread (upper bound)
    constexpr int SC = (WIDE_SCALES + T - 1) / T;
    constexpr int WC = SW_GROUPED ? (WIDE_WSCALES + T - 1) / T : 0;
    __shared__ __align__(16) uint8_t a_l[WIDE_A_BYTES + 32];  // + sink
    __shared__ __align__(16) float sa_l[WIDE_SCALES + 4];     // [g][row] + sink
    __shared__ float sw_l[WIDE_WSCALES + 1];                  // [g][col] + sink

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int cbl = wave / MB, mb = wave % MB;  // local column block, row block
    const int G = K >> 7;
    const int KB = K >> 1;
    const int chunks_row = KB >> 4;             // packed 16-byte chunks per row
    const int a_chunks = ROWS * chunks_row;
    const int rc = lane & 15, part = lane >> 4;
    const int col0 = blockIdx.x * COLS;
    const int col = col0 + cbl * 16 + rc;
    const int8_t* wp = w + (int64_t)min(col, N - 1) * KB + part * 16;

    // ---- activation block + scales: loads first, then the weight ring.
    v4u ra[AC];
    uint16_t rsa[SC], rsw[WC > 0 ? WC : 1];
#pragma unroll
    for (int i = 0; i < AC; ++i) {
        const int q = min(t + i * T, a_chunks - 1);
        const int r = q / chunks_row, c = q - r * chunks_row;
        ra[i] = *reinterpret_cast<const v4u*>(a + (int64_t)min(r, M - 1) * KB + c * 16);
    }
#pragma unroll
    for (int i = 0; i < SC; ++i) {
        const int e = min(t + i * T, G * ROWS - 1);  // e = row * G + g
        rsa[i] = sa[(int64_t)min(e / G, M - 1) * G + e % G];
    }
#pragma unroll
    for (int i = 0; i < WC; ++i) {
        const int e = min(t + i * T, G * COLS - 1);  // e = col * G + g
        rsw[i] = sw[(int64_t)min(col0 + e / G, N - 1) * G + e % G];
    }
    v4u rw[D];
    auto issue = [&](int g, v4u& w_out) {
        w_out = *reinterpret_cast<const v4u*>(wp + (int64_t)min(g, G - 1) * 64);
    };
    static_for<0, D>([&](auto U) { issue(U, rw[U]); });
    // Widen and store: packed chunk c of row r -> units 2c, 2c+1.
#pragma unroll
    for (int i = 0; i < AC; ++i) {
        const int q = t + i * T;
        const int r = q / chunks_row, c = q - r * chunks_row;
        const bool live = q < a_chunks;
        const int u0 = 2 * c, u1 = 2 * c + 1;
        const int s0 = (u0 & ~7) | ((u0 ^ r) & 7), s1 = (u1 & ~7) | ((u1 ^ r) & 7);
        const v4i lo = unpack8_x16(ra[i][0], ra[i][1]);
        const v4i hi = unpack8_x16(ra[i][2], ra[i][3]);
        *reinterpret_cast<v4i*>(&a_l[live ? r * K + s0 * 16 : WIDE_A_BYTES]) = lo;
        *reinterpret_cast<v4i*>(&a_l[live ? r * K + s1 * 16 : WIDE_A_BYTES + 16]) = hi;
    }
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

    float total[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int r = mb * 16 + rc;
    const float* sap = &sa_l[mb * 16 + 4 * part];
    const float* swq = &sw_l[cbl * 16 + rc];

    auto consume = [&](int g, const v4u& w_in) {
        const v4i w0 = unpack8_x16(w_in[0], w_in[1]);
        const v4i w1 = unpack8_x16(w_in[2], w_in[3]);
        const int u0 = (g * 4 + part) * 2, u1 = u0 + 1;
        const v4i a0 = *reinterpret_cast<const v4i*>(&a_l[r * K + (((u0 & ~7) | ((u0 ^ r) & 7)) << 4)]);
        const v4i a1 = *reinterpret_cast<const v4i*>(&a_l[r * K + (((u1 & ~7) | ((u1 ^ r) & 7)) << 4)]);
        const v4f s_a = *reinterpret_cast<const v4f*>(sap + g * ROWS);
        const float s_w = SW_GROUPED ? swq[g * COLS] : 1.0f;
        v4i acc = {0, 0, 0, 0};
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, w0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, w1, acc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float d = (float)(acc[i] >> 8);
            total[i] = SW_GROUPED ? __builtin_fmaf(d, s_a[i] * s_w, total[i]) : __builtin_fmaf(d, s_a[i], total[i]);
        }
    };

    int g0 = 0;
    for (; g0 + D < G; g0 += D) {
        static_for<0, D>([&](auto U) {
            consume(g0 + U, rw[U]);
            issue(g0 + U + D, rw[U]);
        });
    }
    static_for<0, D>([&](auto U) {
        if (g0 + U < G) consume(g0 + U, rw[U]);
    });

    if (col < N) {
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

template <int MB, int NB, bool SG, bool OF>
hipError_t launch_decode(const int8_t* a, const int8_t* w, const void* sa, const void* sw, void* out,
                         int M, int N, int K, hipStream_t st) {
    // Sub-rounds in flight: all of them for K <= 4096, six beyond.
    const dim3 grid((unsigned)((N + 16 * NB - 1) / (16 * NB)));
    const uint16_t* sap = static_cast<const uint16_t*>(sa);
    const uint16_t* swp = static_cast<const uint16_t*>(sw);
    if (K <= 4096)
        hipLaunchKernelGGL((k2_decode<MB, NB, 4, SG, OF>), grid, dim3(DEC_THREADS), 0, st, a, w, sap, swp, out, M, N, K);
    else
        hipLaunchKernelGGL((k2_decode<MB, NB, 6, SG, OF>), grid, dim3(DEC_THREADS), 0, st, a, w, sap, swp, out, M, N, K);
    return hipGetLastError();
}

// Compute units of the current device (cached per device).
int cu_count() {
    static int cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
    if (dev < 64 && cache[dev] > 0) return cache[dev];
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    if (dev < 64) cache[dev] = v;
    return v;
}

// The wide kernel needs the widened activation block and the scales to fit
// in LDS, whole 8-chunk lines per row (swizzle), and at least 4 column blocks
// per CU.
bool wide_fits(int M, int N, int K) {
    const int mb = (M + 15) / 16;
    const int per_cu = ((N + 15) / 16 + cu_count() - 1) / cu_count();
    return M <= 32 && K % 256 == 0 && (int64_t)mb * 16 * K <= WIDE_A_BYTES &&
           (int64_t)(K / 128) * mb * 16 <= WIDE_SCALES && per_cu >= 4 && per_cu <= 8 &&
           (int64_t)(K / 128) * 16 * (per_cu <= 4 ? 4 : per_cu <= 6 ? 6 : 8) <= WIDE_WSCALES;
}

template <int MB, int CBW, bool SG, bool OF>
hipError_t launch_wide_cbw(const int8_t* a, const int8_t* w, const void* sa, const void* sw, void* out,
                           int M, int N, int K, hipStream_t st) {
    constexpr int D = 8;  // groups in flight per wave
    const int ncb = (N + 15) / 16;
    hipLaunchKernelGGL((k2_wide<MB, CBW, D, SG, OF>), dim3((unsigned)((ncb + CBW - 1) / CBW)), dim3(CBW * MB * 64),
                       0, st, a, w, static_cast<const uint16_t*>(sa), static_cast<const uint16_t*>(sw), out, M, N, K);
    return hipGetLastError();
}

template <int MB, bool SG, bool OF>
hipError_t launch_wide(const int8_t* a, const int8_t* w, const void* sa, const void* sw, void* out,
                       int M, int N, int K, hipStream_t st) {
    // Column blocks per workgroup: enough that one workgroup per CU covers N.
    const int per_cu = ((N + 15) / 16 + cu_count() - 1) / cu_count();
    if (per_cu <= 4) return launch_wide_cbw<MB, 4, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    if (per_cu <= 6) return launch_wide_cbw<MB, 6, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    return launch_wide_cbw<MB, 8, SG, OF>(a, w, sa, sw, out, M, N, K, st);
}

template <bool SG, bool OF>
hipError_t dispatch(const int8_t* a, const int8_t* w, const void* sa, const void* sw, void* out,
                    int M, int N, int K, hipStream_t st) {
    // Wide N: waves own column blocks, activations fetched once per CU.
    if (wide_fits(M, N, K)) {
        return M <= 16 ? launch_wide<1, SG, OF>(a, w, sa, sw, out, M, N, K, st)
                       : launch_wide<2, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    }
    // Otherwise 32 columns per workgroup for wide N halves the activation
    // re-reads while still giving every CU several workgroups.
    const bool wide = N >= 16384;
    if (M <= 16) return wide ? launch_decode<1, 2, SG, OF>(a, w, sa, sw, out, M, N, K, st)
                             : launch_decode<1, 1, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    if (M <= 32) return wide ? launch_decode<2, 2, SG, OF>(a, w, sa, sw, out, M, N, K, st)
                             : launch_decode<2, 1, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    if (M <= 48) return launch_decode<3, 1, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    if (M <= 64) return launch_decode<4, 1, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    return k2_prefill_launch(a, w, sa, sw, SG, out, OF, M, N, K, st);
}

}  // namespace
}  // namespace nv4

extern "C" int nv4_w4a4_linear(const void* x, const int8_t* signs, const int8_t* w, const void* sw,
                               void* out, int8_t* a_packed, void* a_scale,
                               int64_t M, int64_t N, int64_t K, void* stream) {
    using namespace nv4;
    if (!x || !signs || !w || !sw || !out || !a_packed || !a_scale) return NV4_E_NULL;
    if (K != 4096 && K != 12288) return NV4_E_SHAPE;
    const int rc = nv4_rht_quant_pack(x, signs, a_packed, a_scale, M, K, NV4_LAYOUT_REFERENCE, stream);
    if (rc != NV4_OK) return rc;
    return nv4_w4a4_gemm(a_packed, w, a_scale, sw, 1, out, 0, M, N, K, stream);
}

extern "C" int nv4_w4a4_gemm(const int8_t* a, const int8_t* w, const void* sa, const void* sw,
                             int sw_grouped, void* out, int out_fp32,
                             int64_t M, int64_t N, int64_t K, void* stream) {
    using namespace nv4;
    if (!a || !w || !sa || !sw || !out) return NV4_E_NULL;
    if (M < 1 || N < 1 || K < 128 || K % 128 || N % 8) return NV4_E_SHAPE;
    if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > (1LL << 20)) return NV4_E_SHAPE;
    if (M * (K / 128) > 0x7fffffffLL || N * (K / 128) > 0x7fffffffLL) return NV4_E_SHAPE;
    if (((M + 127) / 128) * ((N + 127) / 128) > 0x7fffffffLL) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(a) % 16 || reinterpret_cast<uintptr_t>(w) % 16 ||
        reinterpret_cast<uintptr_t>(sa) % 2 || reinterpret_cast<uintptr_t>(sw) % 2 ||
        reinterpret_cast<uintptr_t>(out) % (out_fp32 ? 4 : 2))
        return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int m = (int)M, n = (int)N, k = (int)K;
    hipError_t e;
    if (sw_grouped) {
        e = out_fp32 ? dispatch<true, true>(a, w, sa, sw, out, m, n, k, st)
                     : dispatch<true, false>(a, w, sa, sw, out, m, n, k, st);
    } else {
        e = out_fp32 ? dispatch<false, true>(a, w, sa, sw, out, m, n, k, st)
                     : dispatch<false, false>(a, w, sa, sw, out, m, n, k, st);
    }
    return (int)e;
}
