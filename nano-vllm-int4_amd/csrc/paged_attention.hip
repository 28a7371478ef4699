// Paged decode attention for the Qwen3 decoder (GQA, head_dim 128, bf16 KV
// cache), gfx950.  Replaces flash_attn_with_kvcache in the reference's
// decode branch (nanovllm/layers/attention.py:72-74): for every sequence b
// and query head h, o = softmax(scale * q . K^T) V over the first
// context_lens[b] cache slots of the sequence, found through its block table.
//
// Decode attention reads the whole KV context of every sequence once per
// step, so it is bound by HBM bandwidth; the kernel is laid out for streaming:
//  * pass 1: one workgroup (4 waves) per (sequence, KV head, split of
//    PA_SPLIT context tokens).  Wave w takes a quarter of the split; within a
//    wave, lane group g (16 lanes) owns PA_SPLIT/16 consecutive tokens, and
//    lane j of a group owns head dims 8j..8j+7, so every K and V row
//    of a token (256 contiguous bytes per KV head) is read as one coalesced
//    piece.  The G query heads that share the KV head stay in registers,
//    pre-multiplied by scale * log2(e), so the softmax runs in base 2.
//    A group issues all its K and V loads before any arithmetic (its slot
//    offsets come from one block-table read when block_size % 16 == 0),
//    reduces its scores over its 16 lanes with DPP, and keeps one softmax
//    state (max m, sum l, output o) per head.
//    The 16 group states of the workgroup are merged through LDS and written
//    to the split workspace (or, for a single split, normalised into out).
//  * pass 2: one wave per (sequence, query head) merges the splits: lane s
//    reads split s's (m, l), M = max m_s, w_s = 2^(m_s - M) (broadcast with
//    lane reads), o = sum w_s o_s / sum w_s l_s with lane i owning dims 2i,
//    2i+1 and every split's loads issued before the sums.
#include "nv4_common.h"

namespace nv4 {
namespace {

constexpr int PA_D = 128;        // head dim
constexpr int PA_SPLIT = 256;    // context tokens per pass-1 workgroup
constexpr int PA_TPG = PA_SPLIT / 16;    // tokens per lane group (16 lane groups per workgroup)
constexpr int PA_THREADS = 256;  // 4 waves x 64 tokens

constexpr int DPP_QUAD_XOR1 = 0xB1;
constexpr int DPP_QUAD_XOR2 = 0x4E;
constexpr int DPP_HALF_MIRROR = 0x141;
constexpr int DPP_MIRROR = 0x140;

template <int CTRL>
__device__ __forceinline__ float pa_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// Sum over the 16 lanes of a DPP row (every lane gets the sum).
__device__ __forceinline__ float row16_sum(float v) {
    v += pa_dpp<DPP_QUAD_XOR1>(v);
    v += pa_dpp<DPP_QUAD_XOR2>(v);
    v += pa_dpp<DPP_HALF_MIRROR>(v);
    v += pa_dpp<DPP_MIRROR>(v);
    return v;
}

__device__ __forceinline__ void bf16x8_to_f32(const v4u& w, float (&f)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = __uint_as_float(w[i] << 16);
        f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}

template <int G, bool BLK16>
__global__ void __launch_bounds__(PA_THREADS)
pa_split(const uint16_t* __restrict__ q, int64_t q_row, const uint16_t* __restrict__ kc,
         const uint16_t* __restrict__ vc, const int32_t* __restrict__ block_tables, int max_blocks,
         const int32_t* __restrict__ context_lens, uint16_t* __restrict__ out, float* __restrict__ part_o,
         float* __restrict__ part_ml, int Hkv, int bs, int S, int max_ctx, float qscale) {
    const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int Hq = Hkv * G;
    const int ctx = min(context_lens[b], max_ctx);  // never past the block table's row
    const int start = s * PA_SPLIT;
    if (start >= ctx) return;  // nothing of this sequence here; pass 2 skips the split
    const int end = min(start + PA_SPLIT, ctx);
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int g = lane >> 4, j = lane & 15;

    __shared__ float sm_m[16][G], sm_l[16][G];
    __shared__ float sm_o[16][G][PA_D];

    const int32_t* bt = block_tables + (int64_t)b * max_blocks;
    const int tok0 = start + (wave * 4 + g) * PA_TPG;  // this group's first token
    // Element offsets of the group's token rows for this KV head and lane,
    // clamped into the sequence so every load stays in its own valid slots.
    // With block_size % 16 == 0 the group's 16 tokens (16-aligned) share one
    // block: a single block-table read serves them all.
    int64_t off[PA_TPG];
    if constexpr (BLK16) {
        const int c0 = min(tok0, ctx - 1);
        const int64_t base = ((int64_t)bt[c0 / bs] * bs + c0 % bs) * Hkv + kvh;
#pragma unroll
        for (int i = 0; i < PA_TPG; ++i) off[i] = (base + (int64_t)(min(tok0 + i, ctx - 1) - c0) * Hkv) * PA_D + 8 * j;
    } else {
#pragma unroll
        for (int i = 0; i < PA_TPG; ++i) {
            const int c = min(tok0 + i, ctx - 1);
            off[i] = (((int64_t)bt[c / bs] * bs + c % bs) * Hkv + kvh) * PA_D + 8 * j;
        }
    }
    // Every K row, then every V row, of the group in flight at once.
    v4u kb[PA_TPG], vb[PA_TPG];
#pragma unroll
    for (int i = 0; i < PA_TPG; ++i) kb[i] = *reinterpret_cast<const v4u*>(kc + off[i]);
#pragma unroll
    for (int i = 0; i < PA_TPG; ++i) vb[i] = *reinterpret_cast<const v4u*>(vc + off[i]);

    // Query heads kvh*G .. kvh*G+G-1, dims 8j..8j+7, scaled into base 2.
    float qv[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const v4u w = *reinterpret_cast<const v4u*>(q + (int64_t)b * q_row + (int64_t)(kvh * G + h) * PA_D + 8 * j);
        float f[8];
        bf16x8_to_f32(w, f);
#pragma unroll
        for (int d = 0; d < 8; ++d) qv[h][d] = f[d] * qscale;
    }

    // Scores of the group's tokens (reduced over its 16 lanes), then one
    // softmax state per head: m = max, l = sum 2^(s - m), o = sum 2^(s - m) v.
    float sc[PA_TPG][G];
#pragma unroll
    for (int i = 0; i < PA_TPG; ++i) {
        float kf[8];
        bf16x8_to_f32(kb[i], kf);
        const bool live = tok0 + i < end;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            float p = 0.0f;
#pragma unroll
            for (int d = 0; d < 8; ++d) p = __builtin_fmaf(qv[h][d], kf[d], p);
            p = row16_sum(p);
            sc[i][h] = live ? p : -__builtin_inff();
        }
    }
    float m[G], l[G], o[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float mx = sc[0][h];
#pragma unroll
        for (int i = 1; i < PA_TPG; ++i) mx = fmaxf(mx, sc[i][h]);
        m[h] = mx;
        l[h] = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; ++d) o[h][d] = 0.0f;
        // a group whose tokens are all past the end keeps m = -inf, l = 0, o = 0
        const bool any = mx != -__builtin_inff();
#pragma unroll
        for (int i = 0; i < PA_TPG; ++i) sc[i][h] = any ? __builtin_amdgcn_exp2f(sc[i][h] - mx) : 0.0f;
#pragma unroll
        for (int i = 0; i < PA_TPG; ++i) l[h] += sc[i][h];
    }
#pragma unroll
    for (int i = 0; i < PA_TPG; ++i) {
        float vf[8];
        bf16x8_to_f32(vb[i], vf);
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int d = 0; d < 8; ++d) o[h][d] = __builtin_fmaf(sc[i][h], vf[d], o[h][d]);
    }

    // Merge the 16 group states of the workgroup.
    const int gs = wave * 4 + g;
#pragma unroll
    for (int h = 0; h < G; ++h) {
        if (j == 0) {
            sm_m[gs][h] = m[h];
            sm_l[gs][h] = l[h];
        }
#pragma unroll
        for (int d = 0; d < 8; ++d) sm_o[gs][h][8 * j + d] = o[h][d];
    }
    __syncthreads();
    for (int e = t; e < G * PA_D; e += PA_THREADS) {
        const int h = e / PA_D, d = e % PA_D;
        float M = -__builtin_inff();
#pragma unroll
        for (int k = 0; k < 16; ++k) M = fmaxf(M, sm_m[k][h]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const float w = sm_m[k][h] == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(sm_m[k][h] - M);
            L = __builtin_fmaf(w, sm_l[k][h], L);
            O = __builtin_fmaf(w, sm_o[k][h][d], O);
        }
        const int hq = kvh * G + h;
        if (S == 1) {
            out[((int64_t)b * Hq + hq) * PA_D + d] = (uint16_t)f32_to_bf16_rne(O / L);
        } else {
            const int64_t ps = ((int64_t)b * Hq + hq) * S + s;
            part_o[ps * PA_D + d] = O;
            if (d == 0) {
                part_ml[ps * 2] = M;
                part_ml[ps * 2 + 1] = L;
            }
        }
    }
}

__global__ void __launch_bounds__(64)
pa_merge(const int32_t* __restrict__ context_lens, const float* __restrict__ part_o,
         const float* __restrict__ part_ml, uint16_t* __restrict__ out, int Hq, int S, int max_ctx) {
    const int hq = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
    const int n = min(S, (min(context_lens[b], max_ctx) + PA_SPLIT - 1) / PA_SPLIT);
    const int64_t base = ((int64_t)b * Hq + hq) * S;
    float O0 = 0.0f, O1 = 0.0f, L = 0.0f;
    // Splits in chunks of 64 (one per lane); the running max M rescales
    // earlier chunks when a later one raises it.
    float M = -__builtin_inff();
    for (int c0 = 0; c0 < n; c0 += 64) {
        const int sidx = c0 + lane;
        float ms = -__builtin_inff(), ls = 0.0f;
        if (sidx < n) {
            const float2 ml = *reinterpret_cast<const float2*>(part_ml + (base + sidx) * 2);
            ms = ml.x;
            ls = ml.y;
        }
        float cm = ms;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) cm = fmaxf(cm, __shfl_xor(cm, off));
        const float Mn = fmaxf(M, cm);
        const float corr = M == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(M - Mn);
        O0 *= corr;
        O1 *= corr;
        L *= corr;
        M = Mn;
        const float w = sidx < n ? __builtin_amdgcn_exp2f(ms - M) : 0.0f;
        float wl = w * ls;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) wl += __shfl_xor(wl, off);
        L += wl;
        const int cnt = min(64, n - c0);
        constexpr int U = 8;
        for (int k0 = 0; k0 < cnt; k0 += U) {
            float2 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int k = min(k0 + u, cnt - 1);
                v[u] = *reinterpret_cast<const float2*>(part_o + (base + c0 + k) * PA_D + 2 * lane);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (k0 + u < cnt) {
                    const float wk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w),
                                                                                         k0 + u));
                    O0 = __builtin_fmaf(wk, v[u].x, O0);
                    O1 = __builtin_fmaf(wk, v[u].y, O1);
                }
            }
        }
    }
    uint16_t* o = out + ((int64_t)b * Hq + hq) * PA_D + 2 * lane;
    *reinterpret_cast<uint32_t*>(o) = f32_to_bf16_rne(O0 / L) | (f32_to_bf16_rne(O1 / L) << 16);
}

template <int G>
hipError_t pa_launch(const void* q, int64_t q_row, const void* kc, const void* vc, const int32_t* bt, int max_blocks,
                     const int32_t* cl, void* out, float* ws, int B, int Hkv, int bs, int S, int max_ctx,
                     float qscale, hipStream_t st) {
    float* part_o = ws;
    float* part_ml = ws + (int64_t)B * Hkv * G * S * PA_D;
    const dim3 grid((unsigned)S, (unsigned)Hkv, (unsigned)B);
    if (bs % 16 == 0)
        hipLaunchKernelGGL((pa_split<G, true>), grid, dim3(PA_THREADS), 0, st, static_cast<const uint16_t*>(q), q_row,
                           static_cast<const uint16_t*>(kc), static_cast<const uint16_t*>(vc), bt, max_blocks, cl,
                           static_cast<uint16_t*>(out), part_o, part_ml, Hkv, bs, S, max_ctx, qscale);
    else
        hipLaunchKernelGGL((pa_split<G, false>), grid, dim3(PA_THREADS), 0, st, static_cast<const uint16_t*>(q),
                           q_row, static_cast<const uint16_t*>(kc), static_cast<const uint16_t*>(vc), bt, max_blocks,
                           cl, static_cast<uint16_t*>(out), part_o, part_ml, Hkv, bs, S, max_ctx, qscale);
    if (S > 1)
        hipLaunchKernelGGL(pa_merge, dim3((unsigned)(Hkv * G), (unsigned)B), dim3(64), 0, st, cl, part_o, part_ml,
                           static_cast<uint16_t*>(out), Hkv * G, S, max_ctx);
    return hipGetLastError();
}

}  // namespace
}  // namespace nv4

extern "C" int nv4_paged_decode_attention(const void* q, int64_t q_row_stride, const void* k_cache,
                                          const void* v_cache, const int32_t* block_tables, int64_t max_blocks,
                                          const int32_t* context_lens, void* out, float* workspace,
                                          int64_t workspace_bytes, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                          int64_t block_size, int64_t max_context, float scale, void* stream) {
    using namespace nv4;
    if (!q || !k_cache || !v_cache || !block_tables || !context_lens || !out || !workspace) return NV4_E_NULL;
    if (D != PA_D || B < 1 || Hkv < 1 || Hq < 1 || Hq % Hkv || block_size < 1 || max_blocks < 1 ||
        max_context < 1 || max_context > max_blocks * block_size || B > 65535 || Hkv > 65535 ||
        q_row_stride < Hq * D)
        return NV4_E_SHAPE;
    const int64_t G = Hq / Hkv;
    if (G != 1 && G != 2 && G != 4) return NV4_E_SHAPE;  // the merge keeps 16 x G x 128 fp32 in LDS
    const int64_t S = (max_context + PA_SPLIT - 1) / PA_SPLIT;
    if (workspace_bytes < B * Hq * S * (D + 2) * 4) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(q) % 16 || reinterpret_cast<uintptr_t>(k_cache) % 16 ||
        reinterpret_cast<uintptr_t>(v_cache) % 16 || reinterpret_cast<uintptr_t>(out) % 4 ||
        reinterpret_cast<uintptr_t>(workspace) % 8 || q_row_stride % 8)
        return NV4_E_ALIGN;
    const float qscale = scale * 1.4426950408889634f;  // log2(e): softmax in base 2
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int b = (int)B, hkv = (int)Hkv, bs = (int)block_size, s = (int)S, mb = (int)max_blocks;
    switch (G) {
        case 1: return (int)pa_launch<1>(q, q_row_stride, k_cache, v_cache, block_tables, mb, context_lens, out,
                                         workspace, b, hkv, bs, s, (int)max_context, qscale, st);
        case 2: return (int)pa_launch<2>(q, q_row_stride, k_cache, v_cache, block_tables, mb, context_lens, out,
                                         workspace, b, hkv, bs, s, (int)max_context, qscale, st);
        default: return (int)pa_launch<4>(q, q_row_stride, k_cache, v_cache, block_tables, mb, context_lens, out,
                                          workspace, b, hkv, bs, s, (int)max_context, qscale, st);
    }
}
