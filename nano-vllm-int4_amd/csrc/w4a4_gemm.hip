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
// Two kernels, no split-K, no atomics:
//  * k2_skinny (M <= 64, decode): one workgroup per 16 output columns, all M
//    rows.  Its four waves take every fourth K-group, compute exact int32
//    group dots with v_mfma_i32_16x16x64_i8, and hand them to the whole
//    workgroup through LDS, which runs the fp32 epilogue in group order.
//    The weight stream (N*K/2 bytes) dominates, so this kernel is HBM-bound.
//  * k2_tiled (prefill): 128x128 output tile per workgroup, 2x2 waves of
//    64x64 (2x2 v_mfma_i32_32x32x32_i8 blocks each), per-group epilogue in
//    registers with the activation/weight scale tiles staged in LDS.
#include "nv4_common.h"

namespace nv4 {
namespace {

__device__ __forceinline__ uint16_t ld_u16(const uint16_t* p) { return *p; }

template <bool OUT_F32>
__device__ __forceinline__ void store_out(void* out, int64_t idx, float v) {
    if constexpr (OUT_F32) {
        static_cast<float*>(out)[idx] = v;
    } else {
        static_cast<uint16_t*>(out)[idx] = (uint16_t)f32_to_bf16_rne(v);
    }
}

// ----------------------------------------------------------------------------
// Skinny kernel.  Output tile: all M (<= 16*MB) rows x 16 columns.
// MFMA 16x16x64 i8 layout used here (verified by the parity tests):
//   A operand: lane l supplies row l%16, B operand: lane l supplies column l%16;
//   the 16 bytes a lane supplies are one "k-slot" set shared by A and B.
//   Result: lane l holds C[4*(l/16) + i][l%16], i = 0..3.
// Each lane loads 16 packed bytes (32 k values) per group for its row/column:
// bytes [16*(l/16), 16*(l/16)+16) of the group's 64 bytes, split over two MFMAs.
// ----------------------------------------------------------------------------
template <int MB, bool SW_GROUPED, bool OUT_F32>
__global__ void __launch_bounds__(256)
k2_skinny(const int8_t* __restrict__ a, const int8_t* __restrict__ w,
          const uint16_t* __restrict__ sa, const uint16_t* __restrict__ sw,
          void* __restrict__ out, int M, int N, int K) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * 16;
    const int G = K >> 7;
    const int64_t KB = K >> 1;  // packed bytes per row
    // dots[buffer][group slot][m-block][lane*4 + i]
    __shared__ int dots[2][4][MB][256];

    const int rc = lane & 15;   // row (A) / column (W) within the 16-block
    const int part = lane >> 4; // which 16-byte quarter of the group's 64 bytes
    const int ncol = min(n0 + rc, N - 1);
    const int8_t* __restrict__ wp = w + (int64_t)ncol * KB + part * 16;
    const int8_t* ap[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int r = min(mb * 16 + rc, M - 1);
        ap[mb] = a + (int64_t)r * KB + part * 16;
    }

    // Epilogue ownership: entry e = threadIdx.x of every m-block.
    const int e_lane = threadIdx.x >> 2, e_i = threadIdx.x & 3;
    const int e_col = e_lane & 15;
    const int e_row0 = 4 * (e_lane >> 4) + e_i;
    const int on = n0 + e_col;
    float total[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) total[mb] = 0.0f;

    const int rounds = (G + 3) >> 2;
    for (int rd = 0; rd < rounds; ++rd) {
        const int g = rd * 4 + wave;
        const int buf = rd & 1;
        if (g < G) {
            const uint4 wv = *reinterpret_cast<const uint4*>(wp + (int64_t)g * 64);
            const v4i w0 = unpack8_x16(wv.x, wv.y);
            const v4i w1 = unpack8_x16(wv.z, wv.w);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const uint4 av = *reinterpret_cast<const uint4*>(ap[mb] + (int64_t)g * 64);
                v4i acc = {0, 0, 0, 0};
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack8_x16(av.x, av.y), w0, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack8_x16(av.z, av.w), w1, acc, 0, 0, 0);
                int4 d;
                d.x = acc[0] >> 8; d.y = acc[1] >> 8; d.z = acc[2] >> 8; d.w = acc[3] >> 8;
                *reinterpret_cast<int4*>(&dots[buf][wave][mb][lane * 4]) = d;
            }
        }
        __syncthreads();
#pragma unroll
        for (int gi = 0; gi < 4; ++gi) {
            const int gg = rd * 4 + gi;
            if (gg < G) {
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    const int om = mb * 16 + e_row0;
                    const int omc = min(om, M - 1);
                    const float d = (float)dots[buf][gi][mb][threadIdx.x];
                    const float s_a = bf16_to_f32(ld_u16(sa + (int64_t)omc * G + gg));
                    if constexpr (SW_GROUPED) {
                        const float s_w = bf16_to_f32(ld_u16(sw + (int64_t)min(on, N - 1) * G + gg));
                        const float s = s_a * s_w;
                        total[mb] = __builtin_fmaf(d, s, total[mb]);
                    } else {
                        total[mb] = __builtin_fmaf(d, s_a, total[mb]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int om = mb * 16 + e_row0;
        if (om < M && on < N) {
            float v = total[mb];
            if constexpr (!SW_GROUPED) v = v * bf16_to_f32(ld_u16(sw + on));
            store_out<OUT_F32>(out, (int64_t)om * N + on, v);
        }
    }
}

// ----------------------------------------------------------------------------
// Tiled kernel.  Workgroup tile 128 (M) x 128 (N); wave (wm, wn) owns rows
// 64*wm.., columns 64*wn..; 2x2 blocks of 32x32.
// MFMA 32x32x32 i8 layout: lane l supplies row (A) / column (W) l%32 and the
// k-slots of half l/32.  Result: lane l holds C[8*(i/4) + 4*(l/32) + i%4][l%32].
// Per group each lane reads 32 packed bytes (half l/32 of the 64-byte group)
// for each of its rows/columns; MFMA j (0..3) takes bytes 8j..8j+7 of those.
// ----------------------------------------------------------------------------
constexpr int TBM = 128, TBN = 128;

template <bool SW_GROUPED, bool OUT_F32>
__global__ void __launch_bounds__(256)
k2_tiled(const int8_t* __restrict__ a, const int8_t* __restrict__ w,
         const uint16_t* __restrict__ sa, const uint16_t* __restrict__ sw,
         void* __restrict__ out, int M, int N, int K) {
    extern __shared__ uint16_t smem[];  // sa tile [G][TBM], then sw tile [G][TBN]
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * TBM, n0 = blockIdx.x * TBN;
    const int G = K >> 7;
    const int64_t KB = K >> 1;
    uint16_t* sa_t = smem;
    uint16_t* sw_t = smem + G * TBM;

    // Stage the scale tiles (transposed to [g][row]) once.
    for (int i = threadIdx.x; i < G * TBM; i += 256) {
        const int r = i / G, g = i - r * G;
        const int m = m0 + r;
        sa_t[g * TBM + r] = m < M ? sa[(int64_t)m * G + g] : (uint16_t)0;
    }
    if constexpr (SW_GROUPED) {
        for (int i = threadIdx.x; i < G * TBN; i += 256) {
            const int c = i / G, g = i - c * G;
            const int n = n0 + c;
            sw_t[g * TBN + c] = n < N ? sw[(int64_t)n * G + g] : (uint16_t)0;
        }
    }
    __syncthreads();

    const int rc = lane & 31, half = lane >> 5;
    const int8_t* ap[2];
    const int8_t* wp[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = min(m0 + wm * 64 + i * 32 + rc, M - 1);
        ap[i] = a + (int64_t)r * KB + half * 32;
        const int c = min(n0 + wn * 64 + i * 32 + rc, N - 1);
        wp[i] = w + (int64_t)c * KB + half * 32;
    }

    float total[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) total[i][j][v] = 0.0f;

    for (int g = 0; g < G; ++g) {
        uint4 av[2][2], wv[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            av[i][0] = *reinterpret_cast<const uint4*>(ap[i] + (int64_t)g * 64);
            av[i][1] = *reinterpret_cast<const uint4*>(ap[i] + (int64_t)g * 64 + 16);
            wv[i][0] = *reinterpret_cast<const uint4*>(wp[i] + (int64_t)g * 64);
            wv[i][1] = *reinterpret_cast<const uint4*>(wp[i] + (int64_t)g * 64 + 16);
        }
        v16i acc[2][2];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            v4i ao[2], wo[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint4 q = av[i][s >> 1];
                ao[i] = (s & 1) ? unpack8_x16(q.z, q.w) : unpack8_x16(q.x, q.y);
                const uint4 r = wv[i][s >> 1];
                wo[i] = (s & 1) ? unpack8_x16(r.z, r.w) : unpack8_x16(r.x, r.y);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ao[i], wo[j], acc[i][j], 0, 0, 0);
        }
        // Epilogue for group g.
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int cl = wn * 64 + j * 32 + rc;  // column within the tile
            float s_w = 0.0f;
            if constexpr (SW_GROUPED) s_w = bf16_to_f32(sw_t[g * TBN + cl]);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int rl = wm * 64 + i * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                    const float s_a = bf16_to_f32(sa_t[g * TBM + rl]);
                    const float d = (float)(acc[i][j][v] >> 8);
                    if constexpr (SW_GROUPED) {
                        const float s = s_a * s_w;
                        total[i][j][v] = __builtin_fmaf(d, s, total[i][j][v]);
                    } else {
                        total[i][j][v] = __builtin_fmaf(d, s_a, total[i][j][v]);
                    }
                }
            }
        }
    }

#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 64 + j * 32 + rc;
        float swn = 1.0f;
        if constexpr (!SW_GROUPED) swn = bf16_to_f32(sw[min(n, N - 1)]);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                if (m < M && n < N) {
                    float val = total[i][j][v];
                    if constexpr (!SW_GROUPED) val = val * swn;
                    store_out<OUT_F32>(out, (int64_t)m * N + n, val);
                }
            }
    }
}

template <int MB, bool SG, bool OF>
hipError_t launch_skinny(const int8_t* a, const int8_t* w, const void* sa, const void* sw, void* out,
                         int M, int N, int K, hipStream_t st) {
    hipLaunchKernelGGL((k2_skinny<MB, SG, OF>), dim3((unsigned)((N + 15) / 16)), dim3(256), 0, st, a, w,
                       static_cast<const uint16_t*>(sa), static_cast<const uint16_t*>(sw), out, M, N, K);
    return hipGetLastError();
}

template <bool SG, bool OF>
hipError_t launch_tiled(const int8_t* a, const int8_t* w, const void* sa, const void* sw, void* out,
                        int M, int N, int K, hipStream_t st) {
    const int G = K / 128;
    const size_t lds = (size_t)G * (TBM + TBN) * sizeof(uint16_t);
    dim3 grid((unsigned)((N + TBN - 1) / TBN), (unsigned)((M + TBM - 1) / TBM));
    hipLaunchKernelGGL((k2_tiled<SG, OF>), grid, dim3(256), lds, st, a, w, static_cast<const uint16_t*>(sa),
                       static_cast<const uint16_t*>(sw), out, M, N, K);
    return hipGetLastError();
}

template <bool SG, bool OF>
hipError_t dispatch(const int8_t* a, const int8_t* w, const void* sa, const void* sw, void* out,
                    int M, int N, int K, hipStream_t st) {
    if (M <= 16) return launch_skinny<1, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    if (M <= 32) return launch_skinny<2, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    if (M <= 48) return launch_skinny<3, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    if (M <= 64) return launch_skinny<4, SG, OF>(a, w, sa, sw, out, M, N, K, st);
    return launch_tiled<SG, OF>(a, w, sa, sw, out, M, N, K, st);
}

}  // namespace
}  // namespace nv4

extern "C" int nv4_w4a4_gemm(const int8_t* a, const int8_t* w, const void* sa, const void* sw,
                             int sw_grouped, void* out, int out_fp32,
                             int64_t M, int64_t N, int64_t K, void* stream) {
    using namespace nv4;
    if (!a || !w || !sa || !sw || !out) return NV4_E_NULL;
    if (M < 1 || N < 1 || K < 128 || K % 128 || N % 8) return NV4_E_SHAPE;
    if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > (1LL << 20)) return NV4_E_SHAPE;
    if (M * (K / 128) > 0x7fffffffLL || N * (K / 128) > 0x7fffffffLL) return NV4_E_SHAPE;
    if ((M + 127) / 128 > 65535) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(a) % 16 || reinterpret_cast<uintptr_t>(w) % 16 ||
        reinterpret_cast<uintptr_t>(sa) % 2 || reinterpret_cast<uintptr_t>(sw) % 2 ||
        reinterpret_cast<uintptr_t>(out) % (out_fp32 ? 4 : 2))
        return NV4_E_ALIGN;
    // The tiled kernel stages G*(128+128) bf16 scales in LDS (<= 64 KiB).
    if (M > 64 && (K / 128) * (TBM + TBN) * 2 > 64 * 1024) return NV4_E_SHAPE;
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
