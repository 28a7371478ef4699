// LM head of the decode step: logits[M, N] = h[M, K] . W[N, K]^T in bf16 with
// fp32 sums, for M <= 32 rows (one per sequence) and the vocabulary-sized N.
// Replaces ParallelLMHead.forward's F.linear (nanovllm/layers/embed_head.py:56-61)
// in the decode step; prefill-sized calls keep the library GEMM.
//
// The product reads W once (1.24 GB for Qwen3-8B) and is bound by HBM.  One
// workgroup (4 waves) per 16 rows of W: wave w sums the K-quarter
// [K/4 w, K/4 (w+1)) on the matrix cores (v_mfma_f32_16x16x32_bf16, A = W
// rows, B = h rows as columns), and the four quarter sums are added in LDS in
// wave order.  Small workgroups keep the tail of the grid short (the
// hardware hands them to CUs as others finish).
//
// K order inside a quarter: per step of 128, lane (r, q) = (l % 16, l / 16)
// loads 64 contiguous bytes of its row, k = 32q .. 32q + 31, and feeds them
// to four products, 8 values each; the h operand is read the same way, so
// each product pairs equal k.  A wave keeps three steps of loads in flight.
#include "nv4_common.h"

namespace nv4 {
namespace {

constexpr int LM_ROWS = 16;   // rows of W per workgroup
constexpr int LM_STEP = 128;  // k per step of one wave
constexpr int LM_RING = 3;    // steps of loads in flight

template <int MT, int STEPS>
__global__ void __launch_bounds__(256)
lm_head_k(const uint16_t* __restrict__ h, int64_t h_row, const uint16_t* __restrict__ w,
          uint16_t* __restrict__ out, int64_t out_row, int M, int N, int K) {
    __shared__ __align__(16) v4f red[4][MT][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, q = lane >> 4;
    const int n0 = blockIdx.x * LM_ROWS;
    const int kq = STEPS * LM_STEP;  // the wave's K-quarter (K = 4 kq)
    // Rows past the matrix edge repeat its last row (never stored).
    // Product j of a step takes k = 32 j + 8 q .. + 7 (lane group q): a row's
    // four lanes read 64 contiguous bytes per load.
    const uint16_t* pw = w + (int64_t)min(n0 + r, N - 1) * K + wave * kq + 8 * q;
    const uint16_t* ph[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) ph[mt] = h + (int64_t)min(16 * mt + r, M - 1) * h_row + wave * kq + 8 * q;

    // A fixed step count: every load and wait is placed at compile time, the
    // wait before step s leaves the loads of the next steps in flight.
    v4u a[LM_RING][4], b[LM_RING][MT][4];
    auto issue = [&](int slot, int s) {
#pragma unroll
        for (int j = 0; j < 4; ++j) a[slot][j] = *reinterpret_cast<const v4u*>(pw + s * LM_STEP + 32 * j);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int j = 0; j < 4; ++j) b[slot][mt][j] = *reinterpret_cast<const v4u*>(ph[mt] + s * LM_STEP + 32 * j);
    };
    v4f acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
    // (The scheduling barriers keep the compiler from trading the ring for
    // registers: every step's loads go out as one group.)
    static_for<0, (LM_RING < STEPS ? LM_RING : STEPS)>([&](auto s) { issue(s.value, s.value); });
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, STEPS>([&](auto sc) {
        constexpr int s = sc.value, u = s % LM_RING;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a[u][j]),
                                                                  __builtin_bit_cast(v8bf, b[u][mt][j]), acc[mt], 0,
                                                                  0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (s + LM_RING < STEPS) issue(u, s + LM_RING);
        __builtin_amdgcn_sched_barrier(0);
    });
    // Quarter sums in wave order: ((w0 + w1) + w2) + w3.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[wave][mt][lane] = acc[mt];
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            v4f t = red[0][mt][lane];
#pragma unroll
            for (int ww = 1; ww < 4; ++ww) t += red[ww][mt][lane];
            const int m = 16 * mt + r;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int n = n0 + 4 * q + i;  // lane holds rows 4q + i of the tile, column r
                if (m < M && n < N) out[(int64_t)m * out_row + n] = (uint16_t)f32_to_bf16_rne(t[i]);
            }
        }
    }
}

// 17..32 rows: 32 rows of W per workgroup on v_mfma_f32_32x32x16_bf16 (all
// 32 h rows as the columns of one product), so every byte of W meets the h
// operand bytes once instead of twice.  Lane (r, hh) = (l % 32, l / 32) loads
// k = 32 hh .. 32 hh + 31 of its row per step of 64 and feeds four products;
// the result lane l holds C[8 (i / 4) + 4 hh + i % 4][l % 32], i = 0..15.
template <int STEPS>
__global__ void __launch_bounds__(256)
lm_head_k32(const uint16_t* __restrict__ h, int64_t h_row, const uint16_t* __restrict__ w,
            uint16_t* __restrict__ out, int64_t out_row, int M, int N, int K) {
    constexpr int STEP = 64;
    __shared__ __align__(16) v16f red[4][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 31, hh = lane >> 5;
    const int n0 = blockIdx.x * 32;
    const int kq = STEPS * STEP;  // the wave's K-quarter
    // Product j of a step takes k = 16 j + 8 hh .. + 7: a row's two lanes read
    // 32 contiguous bytes per load.
    const uint16_t* pw = w + (int64_t)min(n0 + r, N - 1) * K + wave * kq + 8 * hh;
    const uint16_t* ph = h + (int64_t)min(r, M - 1) * h_row + wave * kq + 8 * hh;
    v4u a[LM_RING][4], b[LM_RING][4];
    auto issue = [&](int slot, int s) {
#pragma unroll
        for (int j = 0; j < 4; ++j) a[slot][j] = *reinterpret_cast<const v4u*>(pw + s * STEP + 16 * j);
#pragma unroll
        for (int j = 0; j < 4; ++j) b[slot][j] = *reinterpret_cast<const v4u*>(ph + s * STEP + 16 * j);
    };
    v16f acc = {};
    static_for<0, (LM_RING < STEPS ? LM_RING : STEPS)>([&](auto s) { issue(s.value, s.value); });
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, STEPS>([&](auto sc) {
        constexpr int s = sc.value, u = s % LM_RING;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a[u][j]),
                                                          __builtin_bit_cast(v8bf, b[u][j]), acc, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (s + LM_RING < STEPS) issue(u, s + LM_RING);
        __builtin_amdgcn_sched_barrier(0);
    });
    red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
        v16f t = red[0][lane];
#pragma unroll
        for (int ww = 1; ww < 4; ++ww) t += red[ww][lane];
        const int m = r;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int n = n0 + 8 * (i >> 2) + 4 * hh + (i & 3);
            if (m < M && n < N) out[(int64_t)m * out_row + n] = (uint16_t)f32_to_bf16_rne(t[i]);
        }
    }
}

// 17..32 rows, one workgroup of 16 waves per CU over a balanced share of the
// rows (16-row tiles), in two passes over K.  Wave w of pass p owns the
// K-slice p K/2 + w K/32 .. +K/32: its h operand (both 16-row halves of h) is
// loaded once per pass and kept in registers, so h is read from L2 once per
// CU and pass instead of once per tile.  Every tile, each wave multiplies its
// slice of the tile's W rows, the 16 partial sums go through LDS, and waves
// tile % 16 and (tile + 8) % 16 add them in wave order for the two 16-row
// halves of h (pass 0 kept in registers, pass 1 added to it, then rounded and
// stored).  All waves take the same tiles, so
// the one barrier per tile is reached by every wave the same number of times.
// Lane (r, q) = (l % 16, l / 16) of a slice of KS = 32 KSTEPS values feeds
// product j the 8 values at 32 j + 8 q of its row, so the four lanes of a row
// read 64 contiguous bytes per load; the h operand is read the same way.
constexpr int LMP_WAVES = 16;
constexpr int LMP_RING = 2;      // tiles of W loads in flight per wave
constexpr int LMP_MAX_TILES = 48;  // tiles per workgroup (3 per wave to reduce)

template <int KSTEPS>
__global__ void __launch_bounds__(1024)
lm_head_p(const uint16_t* __restrict__ h, int64_t h_row, const uint16_t* __restrict__ w,
          uint16_t* __restrict__ out, int64_t out_row, int M, int N, int K) {
    __shared__ __align__(16) v4f part[2][LMP_WAVES][2][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, q = lane >> 4;
    const int T = (N + 15) >> 4;
    if ((int64_t)T * (blockIdx.x + 1) / gridDim.x == (int64_t)T * blockIdx.x / gridDim.x) return;  // no tile
    const int t0 = (int)((int64_t)T * blockIdx.x / gridDim.x), t1 = (int)((int64_t)T * (blockIdx.x + 1) / gridDim.x);
    const int nt = t1 - t0;  // <= LMP_MAX_TILES (checked by the launcher)
    const bool vec_out = (out_row & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 7) == 0;
    constexpr int KS = 32 * KSTEPS;
    v4f carry[3][2];  // pass-0 sums this wave reduces: [tile / 16][half of h]
    for (int pass = 0; pass < 2; ++pass) {
        // MFMA step j takes k = 32 j + 8 q .. + 7 of the wave's slice for lane
        // group q (any assignment of k to steps gives the same dot product),
        // so the four lanes of a row read 64 contiguous bytes per load: one
        // cache line per row and instruction instead of two.
        const int k0 = pass * (K >> 1) + wave * KS + q * 8;
        v4u b[2][KSTEPS];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int j = 0; j < KSTEPS; ++j)
                b[mt][j] = *reinterpret_cast<const v4u*>(h + (int64_t)min(16 * mt + r, M - 1) * h_row + k0 + 32 * j);
        auto wrow = [&](int t) { return w + (int64_t)min(16 * (t0 + t) + r, N - 1) * K + k0; };
        v4u a[LMP_RING][KSTEPS];
        auto issue = [&](int slot, int t) {
            const uint16_t* p = wrow(min(t, nt - 1));
#pragma unroll
            for (int j = 0; j < KSTEPS; ++j) a[slot][j] = *reinterpret_cast<const v4u*>(p + 32 * j);
        };
        // The ring always holds LMP_RING tiles (past the last tile it reloads
        // the last one), so the loop body has one fixed form.
#pragma unroll
        for (int u = 0; u < LMP_RING; ++u) issue(u, u);
        __builtin_amdgcn_sched_barrier(0);
        for (int t = 0; t < nt; t += LMP_RING) {
#pragma unroll
            for (int u = 0; u < LMP_RING; ++u) {
                const int tt = t + u;  // uniform
                if (tt < nt) {
                    v4f acc[2] = {v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
                    for (int j = 0; j < KSTEPS; ++j)
#pragma unroll
                        for (int mt = 0; mt < 2; ++mt)
                            acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a[u][j]),
                                                                              __builtin_bit_cast(v8bf, b[mt][j]),
                                                                              acc[mt], 0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                    issue(u, tt + LMP_RING);
                    __builtin_amdgcn_sched_barrier(0);
                    part[tt & 1][wave][0][lane] = acc[0];
                    part[tt & 1][wave][1][lane] = acc[1];
                    __syncthreads();
                    // Wave tt % 16 reduces the tile's first 16 h rows, wave
                    // (tt + 8) % 16 the second.
                    const int mt = ((tt & 15) == wave) ? 0 : (((tt + 8) & 15) == wave ? 1 : -1);
                    if (mt >= 0) {
                        const int c = tt >> 4;  // 0..2
                        v4f sum = part[tt & 1][0][mt][lane];
#pragma unroll
                        for (int ww = 1; ww < LMP_WAVES; ++ww) sum += part[tt & 1][ww][mt][lane];
                        if (pass == 0) {
#pragma unroll
                            for (int cc = 0; cc < 3; ++cc)
#pragma unroll
                                for (int hm = 0; hm < 2; ++hm)
                                    if (cc == c && hm == mt) carry[cc][hm] = sum;
                        } else {
                            v4f tot = sum;
#pragma unroll
                            for (int cc = 0; cc < 3; ++cc)
#pragma unroll
                                for (int hm = 0; hm < 2; ++hm)
                                    if (cc == c && hm == mt) tot = carry[cc][hm] + sum;
                            const int n0 = 16 * (t0 + tt), m = 16 * mt + r;
                            uint16_t* o = out + (int64_t)m * out_row + n0 + 4 * q;
                            if (m < M) {
                                if (vec_out && n0 + 16 <= N) {  // the lane's 4 columns in one 8-byte store
                                    *reinterpret_cast<uint2*>(o) =
                                        make_uint2(f32_to_bf16_rne(tot[0]) | (f32_to_bf16_rne(tot[1]) << 16),
                                                   f32_to_bf16_rne(tot[2]) | (f32_to_bf16_rne(tot[3]) << 16));
                                } else {
#pragma unroll
                                    for (int i = 0; i < 4; ++i)
                                        if (n0 + 4 * q + i < N) o[i] = (uint16_t)f32_to_bf16_rne(tot[i]);
                                }
                            }
                        }
                    }
                }
            }
        }
        // Drain the ring's extra loads before the next pass reuses it.
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
    }
}

}  // namespace
}  // namespace nv4

extern "C" int nv4_lm_head(const void* h, int64_t h_row_stride, const void* w, void* out, int64_t out_row_stride,
                           int64_t M, int64_t N, int64_t K, void* stream) {
    using namespace nv4;
    if (!h || !w || !out) return NV4_E_NULL;
    // K in {2048, 4096, 5120} (the hidden sizes of the Qwen3 family up to 14B).
    if (M < 1 || M > 32 || N < 1 || N > ((int64_t)1 << 30) || (K != 2048 && K != 4096 && K != 5120) ||
        h_row_stride < K || out_row_stride < N)
        return NV4_E_SHAPE;
    // 16-byte loads of W rows and h rows.
    if (reinterpret_cast<uintptr_t>(h) % 16 || reinterpret_cast<uintptr_t>(w) % 16 || h_row_stride % 8 ||
        reinterpret_cast<uintptr_t>(out) % 2)
        return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const auto* hp = static_cast<const uint16_t*>(h);
    const auto* wp = static_cast<const uint16_t*>(w);
    auto* op = static_cast<uint16_t*>(out);
    // One row, or a share per CU too large for the per-CU form: 16-row
    // workgroups of the 16 x 16 product up to 16 rows, 32-row workgroups of
    // the 32 x 32 product above.
    auto go16 = [&](auto steps) {
        hipLaunchKernelGGL((lm_head_k<1, decltype(steps)::value>), dim3((unsigned)((N + LM_ROWS - 1) / LM_ROWS)),
                           dim3(256), 0, st, hp, h_row_stride, wp, op, out_row_stride, (int)M, (int)N, (int)K);
    };
    auto go32 = [&](auto steps) {
        hipLaunchKernelGGL((lm_head_k32<decltype(steps)::value>), dim3((unsigned)((N + 31) / 32)), dim3(256), 0, st,
                           hp, h_row_stride, wp, op, out_row_stride, (int)M, (int)N, (int)K);
    };
    // 2..32 rows: one 16-wave workgroup per CU when every CU's share is at
    // most LMP_MAX_TILES tiles (N <= 196608 on 256 CUs) and K is 2048 or
    // 4096.
    const int cus = device_cu_count();
    const bool persistent = M > 1 && ((N + 15) / 16 + cus - 1) / cus <= LMP_MAX_TILES;
    auto gop = [&](auto ksteps) {
        hipLaunchKernelGGL((lm_head_p<decltype(ksteps)::value>), dim3((unsigned)cus), dim3(1024), 0, st, hp,
                           h_row_stride, wp, op, out_row_stride, (int)M, (int)N, (int)K);
    };
    using std::integral_constant;
    switch (K) {
        case 2048:
            persistent ? gop(integral_constant<int, 2>{})
                       : (M <= 16 ? go16(integral_constant<int, 4>{}) : go32(integral_constant<int, 8>{}));
            break;
        case 4096:
            persistent ? gop(integral_constant<int, 4>{})
                       : (M <= 16 ? go16(integral_constant<int, 8>{}) : go32(integral_constant<int, 16>{}));
            break;
        default:  // 5120 (the per-CU form would spill registers)
            M <= 16 ? go16(integral_constant<int, 10>{}) : go32(integral_constant<int, 20>{});
            break;
    }
    return (int)hipGetLastError();
}
