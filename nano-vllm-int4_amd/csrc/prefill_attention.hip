// Prefill (causal) attention for the Qwen3 decoder, gfx950.  Replaces
// flash_attn_varlen_func in the reference's prefill branch
// (nanovllm/layers/attention.py:64-70): for every packed sequence b (rows
// cu[b] .. cu[b+1]-1 of q, k, v), query head h and query row i,
//   o[i] = softmax_j<=i(scale * q[i] . k[j]) v[j]
// with GQA (query head h reads KV head h / G), head_dim 128, bf16 in and out.
//
// Layout: one workgroup of NW = 8 waves (4 when that grid would leave CUs
// idle: short prompts, G <= 4) per (sequence, KV head, block of QW = 32 NW/G
// query rows); wave w takes query head w % G of the group and the 32 query
// rows 32 (w / G) .. of the block, so the G heads of a KV head share every
// staged key and value.  Keys run in blocks of KB (128 in the 8-wave form,
// 64 in the 4-wave form) up to the block's last query row; each block is
// staged in LDS once for the workgroup (K as rows, V transposed), with the
// next block's loads in flight during the current one's arithmetic and one
// barrier per block.  Workgroups of the longest causal extent are dispatched
// first.
//
// Matrix cores (v_mfma_f32_32x32x16_bf16; operand lane l supplies row /
// column l%32 and the 8 k-slots 8(l/32) .. +7, result lane l holds
// C[8(i/4) + 4(l/32) + i%4][l%32], i = 0..15):
//  * scores S^T[key][query] = K . Q^T: A = 16 bytes of a K row from LDS,
//    B = 16 bytes of this lane's query row (kept in registers), eight 16-dim
//    steps per 32-key tile.  Lane l thus holds scores of one query (l%32)
//    and 16 keys per tile: the online softmax is per lane, with one exchange
//    between lanes l and l^32 for the running max;
//  * output O^T[dim][query] += V^T . P^T: B = P^T straight from the score
//    registers (bf16, as flash attention rounds P for its P.V product), whose
//    k-slot e of lane half hh is key 16t + 8(e/4) + 4hh + e%4 of step t; A =
//    the same keys of one dim row of V^T, two 8-byte LDS reads.  Every
//    output accumulator of a lane belongs to its own query, so the softmax
//    rescale is a per-lane factor (skipped when no running max moved).
//
// LDS per stage: K[KB][136] bf16 (a 272-byte row stride: the 16-byte reads
// of 16 consecutive rows fall in distinct bank groups) and V^T[128][KB + 4]
// bf16 (rows of 136 or 264 bytes, 8 times an odd number: the 8-byte reads of
// 32 consecutive rows are conflict-free); two stages: 134 KiB for one
// 8-wave workgroup per CU, 68 KiB for two 4-wave ones.  All global loads are
// clamped into the sequence and unconditional; rows past a sequence are
// never stored.
#include "nv4_common.h"

namespace nv4 {
namespace {

constexpr int FA_D = 128;                                   // head dim
constexpr int FA_KS = FA_D + 8;                             // K row stride (bf16)
// V^T row stride and bf16 per stage for KB-key blocks.
constexpr int fa_vs(int KB) { return KB + 4; }
constexpr int fa_stage(int KB) { return KB * FA_KS + FA_D * fa_vs(KB); }
static_assert(2 * fa_stage(64) * 2 == 69632 && 2 * fa_stage(128) * 2 == 137216, "68 / 134 KiB of LDS");

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

template <int G, int NW, int FA_KB>
__global__ void __launch_bounds__(NW * 64, FA_KB == 64 ? 8 / NW : 1)
fa_prefill(const uint16_t* __restrict__ q, int64_t q_row, const uint16_t* __restrict__ k, int64_t k_row,
           const uint16_t* __restrict__ v, int64_t v_row, uint16_t* __restrict__ out, int64_t o_row,
           const int32_t* __restrict__ cu, int Hkv, int nqb, float qscale) {
    constexpr int T = NW * 64;
    constexpr int FA_VS = fa_vs(FA_KB), FA_STAGE = fa_stage(FA_KB);
    constexpr int NC = FA_KB / 32;    // 32-key tiles per block
    constexpr int QT = NW / G;        // 32-row query tiles per workgroup
    constexpr int QW = 32 * QT;       // query rows per workgroup
    constexpr int KU = FA_KB * FA_D / 8 / T, VU = FA_KB / 2 * FA_D / 8 / T;  // staging units per thread
    static_assert(QT >= 1 && KU * T * 8 == FA_KB * FA_D && VU * T * 16 == FA_KB * FA_D, "staging split");
    __shared__ __align__(16) uint16_t lds[2 * FA_STAGE];

    const int b = blockIdx.y;
    const int kvh = (int)(blockIdx.x % (unsigned)Hkv);
    const int qb = nqb - 1 - (int)(blockIdx.x / (unsigned)Hkv);  // longest causal extent first
    const int start = cu[b], L = cu[b + 1] - start;
    const int q0 = qb * QW;
    if (q0 >= L) return;

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int hq = kvh * G + wave % G, qt = wave / G;
    const int rc = lane & 31, hh = lane >> 5;
    const int qr = q0 + 32 * qt + rc;    // this lane's query row (rows >= L are computed, not stored)
    const int lim = min(qr, L - 1);      // last key this row attends to
    const int wave_q0 = q0 + 32 * qt;    // the wave's first query row

    // Q^T operands, 16-dim step s: dims 16 s + 8 hh .. +7 of the lane's row.
    v4u qv[8];
    {
        const uint16_t* qp = q + (int64_t)(start + lim) * q_row + (int64_t)hq * FA_D + 8 * hh;
#pragma unroll
        for (int s = 0; s < 8; ++s) qv[s] = *reinterpret_cast<const v4u*>(qp + 16 * s);
    }

    // Staging.  K: chunks c = t + T i of the block (key c / 16, dims
    // 8 (c % 16) ..).  V: units u = t + T i, keys 2 kp, 2 kp + 1 (kp =
    // u % (KB/2)), dims 8 dc .. (dc = u / (KB/2)), written transposed as
    // bf16 pairs.
    const uint16_t* kbase = k + (int64_t)start * k_row + (int64_t)kvh * FA_D;
    const uint16_t* vbase = v + (int64_t)start * v_row + (int64_t)kvh * FA_D;
    v4u kr[KU], vr[VU][2];
    auto load = [&](int kb) {
        const int key0 = kb * FA_KB;
#pragma unroll
        for (int i = 0; i < KU; ++i) {
            const int c = t + T * i;
            kr[i] = *reinterpret_cast<const v4u*>(kbase + (int64_t)min(key0 + (c >> 4), L - 1) * k_row + (c & 15) * 8);
        }
#pragma unroll
        for (int i = 0; i < VU; ++i) {
            const int u = t + T * i, kp = u % (FA_KB / 2), dc = u / (FA_KB / 2);
            vr[i][0] = *reinterpret_cast<const v4u*>(vbase + (int64_t)min(key0 + 2 * kp, L - 1) * v_row + 8 * dc);
            vr[i][1] = *reinterpret_cast<const v4u*>(vbase + (int64_t)min(key0 + 2 * kp + 1, L - 1) * v_row + 8 * dc);
        }
    };
    auto store = [&](int stage) {
        uint16_t* Ks = lds + stage * FA_STAGE;
        uint16_t* Vt = Ks + FA_KB * FA_KS;
#pragma unroll
        for (int i = 0; i < KU; ++i) {
            const int c = t + T * i;
            *reinterpret_cast<v4u*>(Ks + (c >> 4) * FA_KS + (c & 15) * 8) = kr[i];
        }
#pragma unroll
        for (int i = 0; i < VU; ++i) {
            const int u = t + T * i, kp = u % (FA_KB / 2), dc = u / (FA_KB / 2);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t lo = __builtin_amdgcn_perm(vr[i][1][j], vr[i][0][j], 0x05040100u);  // dim 2j
                const uint32_t hi = __builtin_amdgcn_perm(vr[i][1][j], vr[i][0][j], 0x07060302u);  // dim 2j + 1
                *reinterpret_cast<uint32_t*>(Vt + (8 * dc + 2 * j) * FA_VS + 2 * kp) = lo;
                *reinterpret_cast<uint32_t*>(Vt + (8 * dc + 2 * j + 1) * FA_VS + 2 * kp) = hi;
            }
        }
    };

    float m = -__builtin_inff(), l = 0.0f;
    v16f o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = v16f{};

    auto compute = [&](int kb) {
        const uint16_t* Ks = lds + (kb & 1) * FA_STAGE;
        const uint16_t* Vt = Ks + FA_KB * FA_KS;
        v16f sc[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            sc[c] = v16f{};
            const uint16_t* kp_row = Ks + (32 * c + rc) * FA_KS + 8 * hh;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const v4u a = *reinterpret_cast<const v4u*>(kp_row + 16 * s);
                sc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a),
                                                                __builtin_bit_cast(v8bf, qv[s]), sc[c], 0, 0, 0);
            }
        }
        // Causal and sequence-end mask, only in blocks that reach past the
        // wave's first query row or the sequence (uniform over the wave).
        const int key0 = kb * FA_KB;
        if (key0 + FA_KB - 1 > wave_q0 || key0 + FA_KB > L) {
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = key0 + 32 * c + 8 * (i >> 2) + 4 * hh + (i & 3);
                    if (key > lim) sc[c][i] = -__builtin_inff();
                }
        }
        float mx = -__builtin_inff();
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sc[c][i]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);  // finite from the first block on (key 0 is never masked)
        const float off = -mn * qscale;
        const float corr = __builtin_amdgcn_exp2f(__builtin_fmaf(m, qscale, off));
        m = mn;
        // P^T operands: step t of tile c takes values 8t .. 8t + 7.
        v4u pw[NC][2];
        float ls = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[c][2 * j], qscale, off));
                const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[c][2 * j + 1], qscale, off));
                ls += p0 + p1;
                pw[c][j >> 2][j & 3] = __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f){p0, p1}, v2bf));
            }
        l = l * corr + ls;
        if (__builtin_amdgcn_ballot_w64(corr != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[dt][i] *= corr;
        }
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const int kofs = 32 * c + 16 * st + 4 * hh;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    const uint16_t* vp = Vt + (32 * dt + rc) * FA_VS + kofs;
                    const uint2 lo = *reinterpret_cast<const uint2*>(vp);
                    const uint2 hi = *reinterpret_cast<const uint2*>(vp + 8);
                    const v4u a = {lo.x, lo.y, hi.x, hi.y};
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a),
                                                                    __builtin_bit_cast(v8bf, pw[c][st]), o[dt], 0,
                                                                    0, 0);
                }
            }
    };

    const int kend = min(L, q0 + QW);
    const int nkb = (kend + FA_KB - 1) / FA_KB;
    load(0);
    store(0);
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb) {
        // The next block's loads fly during this block's arithmetic; past the
        // last block they reload it into the unused stage.
        load(min(kb + 1, nkb - 1));
        compute(kb);
        store((kb + 1) & 1);
        __syncthreads();
    }

    l += __shfl_xor(l, 32);
    const float inv = 1.0f / l;
    if (qr < L) {
        uint16_t* op = out + (int64_t)(start + qr) * o_row + (int64_t)hq * FA_D + 4 * hh;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const v2bf a = __builtin_convertvector((v2f){o[dt][4 * j] * inv, o[dt][4 * j + 1] * inv}, v2bf);
                const v2bf c2 = __builtin_convertvector((v2f){o[dt][4 * j + 2] * inv, o[dt][4 * j + 3] * inv}, v2bf);
                *reinterpret_cast<uint2*>(op + 32 * dt + 8 * j) =
                    make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, c2));
            }
    }
}

// Eight waves per workgroup (G heads x 8/G query tiles) when the grid fills
// the CUs; otherwise four (short prompts: twice the workgroups).
template <int G>
hipError_t launch_fa(const uint16_t* q, int64_t q_row, const uint16_t* k, int64_t k_row, const uint16_t* v,
                     int64_t v_row, uint16_t* out, int64_t o_row, const int32_t* cu, int B, int64_t max_seqlen,
                     int Hkv, float qscale, hipStream_t st) {
    constexpr int NW = G > 4 ? 8 : 4;
    const int64_t nqb8 = (max_seqlen + 32 * (8 / G) - 1) / (32 * (8 / G));
    if (G > 4 || nqb8 * Hkv * B >= device_cu_count()) {
        const int nqb = (int)nqb8;
        hipLaunchKernelGGL((fa_prefill<G, 8, 128>), dim3((unsigned)(nqb * Hkv), (unsigned)B), dim3(512), 0, st, q, q_row,
                           k, k_row, v, v_row, out, o_row, cu, Hkv, nqb, qscale);
    } else {
        const int nqb = (int)((max_seqlen + 32 * (NW / G) - 1) / (32 * (NW / G)));
        hipLaunchKernelGGL((fa_prefill<G, NW, 64>), dim3((unsigned)(nqb * Hkv), (unsigned)B), dim3(NW * 64), 0, st, q,
                           q_row, k, k_row, v, v_row, out, o_row, cu, Hkv, nqb, qscale);
    }
    return hipGetLastError();
}

}  // namespace
}  // namespace nv4

extern "C" int nv4_prefill_attention(const void* q, int64_t q_row, const void* k, int64_t k_row, const void* v,
                                     int64_t v_row, void* out, int64_t o_row, const int32_t* cu_seqlens, int64_t B,
                                     int64_t max_seqlen, int64_t Hq, int64_t Hkv, int64_t D, float scale,
                                     void* stream) {
    using namespace nv4;
    if (!q || !k || !v || !out || !cu_seqlens) return NV4_E_NULL;
    if (D != FA_D || Hkv < 1 || Hq < Hkv || Hq % Hkv || !(scale > 0.0f) || scale > 3.0e38f) return NV4_E_SHAPE;
    const int64_t G = Hq / Hkv;
    if (G != 1 && G != 2 && G != 4 && G != 8) return NV4_E_SHAPE;
    if (B < 1 || B > 65535 || max_seqlen < 1 || max_seqlen > (1LL << 24) || Hkv > 4096) return NV4_E_SHAPE;
    if (q_row < Hq * D || o_row < Hq * D || k_row < Hkv * D || v_row < Hkv * D) return NV4_E_SHAPE;
    if (q_row % 8 || k_row % 8 || v_row % 8 || o_row % 8) return NV4_E_ALIGN;
    if (reinterpret_cast<uintptr_t>(q) % 16 || reinterpret_cast<uintptr_t>(k) % 16 ||
        reinterpret_cast<uintptr_t>(v) % 16 || reinterpret_cast<uintptr_t>(out) % 16 ||
        reinterpret_cast<uintptr_t>(cu_seqlens) % 4)
        return NV4_E_ALIGN;
    const int64_t nqb = (max_seqlen + 31) / 32;  // the most query blocks any form launches
    if (nqb * Hkv > 0x7fffffffLL) return NV4_E_SHAPE;
    const float qscale = scale * 1.44269504088896340736f;  // scores in base-2 units
    const auto* qp = static_cast<const uint16_t*>(q);
    const auto* kp = static_cast<const uint16_t*>(k);
    const auto* vp = static_cast<const uint16_t*>(v);
    auto* op = static_cast<uint16_t*>(out);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int b = (int)B, hk = (int)Hkv;
    const int64_t n = max_seqlen;
    hipError_t e;
    switch (G) {
        case 1: e = launch_fa<1>(qp, q_row, kp, k_row, vp, v_row, op, o_row, cu_seqlens, b, n, hk, qscale, st); break;
        case 2: e = launch_fa<2>(qp, q_row, kp, k_row, vp, v_row, op, o_row, cu_seqlens, b, n, hk, qscale, st); break;
        case 4: e = launch_fa<4>(qp, q_row, kp, k_row, vp, v_row, op, o_row, cu_seqlens, b, n, hk, qscale, st); break;
        default: e = launch_fa<8>(qp, q_row, kp, k_row, vp, v_row, op, o_row, cu_seqlens, b, n, hk, qscale, st); break;
    }
    return (int)e;
}
