// Temperature sampling of the next token (gfx950), one launch per step.
//
// The reference's Sampler (nanovllm/layers/sampler.py:5-12) draws
//   argmax_v softmax(l / T)[v] / max(E_v, 1e-10),   E_v ~ Exp(1) i.i.d.,
// the Gumbel-max form of sampling from softmax(l / T).  Dividing by a
// positive row constant and taking logs keep the argmax, so this kernel draws
//   argmax_v  l[v] / T - log(max(E_v, 1e-10)),       E_v = -log U_v,
// the same distribution, in one pass over the logits: one workgroup per row,
// no probabilities materialised.  The split form (nv4_gumbel_sample_ws)
// spreads a row over several workgroups whose (score, index) partials a
// second launch merges: the same scores, the same tie rule, the same token.  U_v = (top 24 bits of a Philox4x32-10 word
// + 0.5) * 2^-24 lies in (0, 1); the generator is counter based (Salmon et
// al., "Parallel random numbers: as easy as 1, 2, 3", SC 2011): key = the
// 64-bit seed, counter = (column / 4, row, 64-bit offset), one 128-bit block
// per 4 columns, so a (seed, offset) pair fixes every draw of the step.  Ties
// resolve to the smallest index (torch.argmax's rule).
#include "nv4_common.h"

namespace nv4 {

struct Philox4 {
    uint32_t v[4];
};

// Philox4x32 with 10 rounds: multipliers 0xD2511F53 / 0xCD9E8D57, Weyl key
// increments 0x9E3779B9 / 0xBB67AE85 (the published parameters).
__host__ __device__ inline Philox4 philox4x32_10(Philox4 c, uint32_t k0, uint32_t k1) {
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c.v[0];
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c.v[2];
        const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        const uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        Philox4 n;
        n.v[0] = hi1 ^ c.v[1] ^ k0;
        n.v[1] = lo1;
        n.v[2] = hi0 ^ c.v[3] ^ k1;
        n.v[3] = lo0;
        c = n;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return c;
}

namespace {

constexpr int SMP_T = 1024;
constexpr int SMP_PT = 256;         // threads per partial workgroup
constexpr int SMP_TARGET_WG = 2048;  // partial workgroups aimed at over the batch

__device__ __forceinline__ float gumbel_score(float l, float temp, uint32_t bits) {
    const float u = ((float)(bits >> 8) + 0.5f) * 0x1p-24f;
    const float e = fmaxf(-logf(u), 1e-10f);
    return l / temp - logf(e);
}

// Scores of quad q (columns 4q .. 4q+3) of a row folded into the running
// (best, besti); columns rise within a thread, so the first maximum stays.
template <bool BF16, bool VEC>
__device__ __forceinline__ void score_quad(const void* __restrict__ logits, int64_t row_stride, int row, int q, int V,
                                           float temp, uint32_t seed_lo, uint32_t seed_hi, uint32_t off_lo,
                                           uint32_t off_hi, float& best, int& besti) {
    float l[4];
    const int c0 = q * 4;
    if constexpr (BF16) {
        const uint16_t* lr = static_cast<const uint16_t*>(logits) + row * row_stride;
        if (VEC && c0 + 3 < V) {
            const uint2 w = *reinterpret_cast<const uint2*>(lr + c0);
            l[0] = bf16_to_f32(w.x & 0xffffu);
            l[1] = bf16_to_f32(w.x >> 16);
            l[2] = bf16_to_f32(w.y & 0xffffu);
            l[3] = bf16_to_f32(w.y >> 16);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) l[i] = c0 + i < V ? bf16_to_f32(lr[c0 + i]) : -INFINITY;
        }
    } else {
        const float* lr = static_cast<const float*>(logits) + row * row_stride;
#pragma unroll
        for (int i = 0; i < 4; ++i) l[i] = c0 + i < V ? lr[c0 + i] : -INFINITY;
    }
    Philox4 c;
    c.v[0] = (uint32_t)q;
    c.v[1] = (uint32_t)row;
    c.v[2] = off_lo;
    c.v[3] = off_hi;
    const Philox4 r = philox4x32_10(c, seed_lo, seed_hi);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (c0 + i < V) {
            const float sc = gumbel_score(l[i], temp, r.v[i]);
            if (sc > best) {
                best = sc;
                besti = c0 + i;
            }
        }
    }
}

// Larger score wins; equal scores go to the smaller index.
__device__ __forceinline__ void argmax_merge(float& best, int& besti, float os, int oi) {
    if (os > best || (os == best && oi < besti)) {
        best = os;
        besti = oi;
    }
}

template <int T>
__device__ __forceinline__ void block_argmax(float& best, int& besti, float* red_s, int* red_i) {
    const int t = threadIdx.x;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) argmax_merge(best, besti, __shfl_xor(best, off), __shfl_xor(besti, off));
    if ((t & 63) == 0) {
        red_s[t >> 6] = best;
        red_i[t >> 6] = besti;
    }
    __syncthreads();
    if (t == 0) {
        for (int w = 1; w < T / 64; ++w) argmax_merge(best, besti, red_s[w], red_i[w]);
    }
}

template <bool BF16, bool VEC>
__global__ void __launch_bounds__(SMP_T)
gumbel_sample(const void* __restrict__ logits, int64_t row_stride, const float* __restrict__ temps, int V,
              uint32_t seed_lo, uint32_t seed_hi, uint32_t off_lo, uint32_t off_hi, int64_t* __restrict__ out) {
    __shared__ float red_s[SMP_T / 64];
    __shared__ int red_i[SMP_T / 64];
    const int row = blockIdx.x;
    const float temp = temps[row];
    float best = -INFINITY;
    int besti = 0x7fffffff;
    const int nq = (V + 3) >> 2;  // 4-column quads
    for (int q = threadIdx.x; q < nq; q += SMP_T)
        score_quad<BF16, VEC>(logits, row_stride, row, q, V, temp, seed_lo, seed_hi, off_lo, off_hi, best, besti);
    block_argmax<SMP_T>(best, besti, red_s, red_i);
    if (threadIdx.x == 0) out[row] = besti == 0x7fffffff ? 0 : besti;
}

// Pass 1 of the split form: workgroup (chunk, row) scans quads
// chunk*qpc .. +qpc of the row and writes its (score, index) to the workspace.
template <bool BF16, bool VEC>
__global__ void __launch_bounds__(SMP_PT)
gumbel_partial(const void* __restrict__ logits, int64_t row_stride, const float* __restrict__ temps, int V,
               uint32_t seed_lo, uint32_t seed_hi, uint32_t off_lo, uint32_t off_hi, int qpc, int P,
               float* __restrict__ ws_s, int* __restrict__ ws_i) {
    __shared__ float red_s[SMP_PT / 64];
    __shared__ int red_i[SMP_PT / 64];
    const int chunk = blockIdx.x, row = blockIdx.y;
    const float temp = temps[row];
    float best = -INFINITY;
    int besti = 0x7fffffff;
    const int nq = (V + 3) >> 2;
    const int q1 = min(nq, (chunk + 1) * qpc);
    for (int q = chunk * qpc + (int)threadIdx.x; q < q1; q += SMP_PT)
        score_quad<BF16, VEC>(logits, row_stride, row, q, V, temp, seed_lo, seed_hi, off_lo, off_hi, best, besti);
    block_argmax<SMP_PT>(best, besti, red_s, red_i);
    if (threadIdx.x == 0) {
        ws_s[row * P + chunk] = best;
        ws_i[row * P + chunk] = besti;
    }
}

// Pass 2: one wave per row merges the row's P partials.
__global__ void __launch_bounds__(64)
gumbel_final(const float* __restrict__ ws_s, const int* __restrict__ ws_i, int P, int64_t* __restrict__ out) {
    const int row = blockIdx.x, lane = threadIdx.x;
    float best = -INFINITY;
    int besti = 0x7fffffff;
    for (int p = lane; p < P; p += 64) argmax_merge(best, besti, ws_s[row * P + p], ws_i[row * P + p]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) argmax_merge(best, besti, __shfl_xor(best, off), __shfl_xor(besti, off));
    if (lane == 0) out[row] = besti == 0x7fffffff ? 0 : besti;
}

}  // namespace
}  // namespace nv4

extern "C" int nv4_gumbel_sample(const void* logits, int64_t row_stride, int logits_dtype, const float* temperatures,
                                 int64_t B, int64_t V, uint64_t seed, uint64_t offset, int64_t* out, void* stream) {
    using namespace nv4;
    if (!logits || !temperatures || !out) return NV4_E_NULL;
    if (B < 1 || B > 0x7fffffffLL || V < 1 || V > 0x7ffffff0LL || row_stride < V) return NV4_E_SHAPE;
    if (logits_dtype != NV4_BF16 && logits_dtype != NV4_FP32) return NV4_E_DTYPE;
    if (reinterpret_cast<uintptr_t>(logits) % (logits_dtype == NV4_BF16 ? 2 : 4)) return NV4_E_ALIGN;
    // bf16 rows read 4 columns per 8-byte load when every row start allows it
    const bool vec = reinterpret_cast<uintptr_t>(logits) % 8 == 0 && row_stride % 4 == 0;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const uint32_t s0 = (uint32_t)seed, s1 = (uint32_t)(seed >> 32);
    const uint32_t o0 = (uint32_t)offset, o1 = (uint32_t)(offset >> 32);
    if (logits_dtype == NV4_BF16 && vec)
        hipLaunchKernelGGL((gumbel_sample<true, true>), dim3((unsigned)B), dim3(SMP_T), 0, st, logits, row_stride,
                           temperatures, (int)V, s0, s1, o0, o1, out);
    else if (logits_dtype == NV4_BF16)
        hipLaunchKernelGGL((gumbel_sample<true, false>), dim3((unsigned)B), dim3(SMP_T), 0, st, logits, row_stride,
                           temperatures, (int)V, s0, s1, o0, o1, out);
    else
        hipLaunchKernelGGL((gumbel_sample<false, false>), dim3((unsigned)B), dim3(SMP_T), 0, st, logits,
                           row_stride, temperatures, (int)V, s0, s1, o0, o1, out);
    return (int)hipGetLastError();
}

extern "C" int64_t nv4_gumbel_sample_chunks(int64_t B, int64_t V) {
    if (B < 1 || V < 1) return 0;
    const int64_t nq = (V + 3) / 4;
    const int64_t by_batch = (nv4::SMP_TARGET_WG + B - 1) / B;
    const int64_t by_vocab = (nq + nv4::SMP_PT - 1) / nv4::SMP_PT;
    return by_batch < by_vocab ? by_batch : by_vocab;
}

extern "C" int nv4_gumbel_sample_ws(const void* logits, int64_t row_stride, int logits_dtype,
                                    const float* temperatures, int64_t B, int64_t V, uint64_t seed, uint64_t offset,
                                    void* workspace, int64_t workspace_bytes, int64_t* out, void* stream) {
    using namespace nv4;
    if (!logits || !temperatures || !out || !workspace) return NV4_E_NULL;
    if (B < 1 || B > 65535 || V < 1 || V > 0x7ffffff0LL || row_stride < V) return NV4_E_SHAPE;
    if (logits_dtype != NV4_BF16 && logits_dtype != NV4_FP32) return NV4_E_DTYPE;
    if (reinterpret_cast<uintptr_t>(logits) % (logits_dtype == NV4_BF16 ? 2 : 4) ||
        reinterpret_cast<uintptr_t>(workspace) % 4)
        return NV4_E_ALIGN;
    const int64_t P = nv4_gumbel_sample_chunks(B, V);
    if (workspace_bytes < 8 * B * P) return NV4_E_SHAPE;
    const int64_t nq = (V + 3) / 4;
    const int qpc = (int)((nq + P - 1) / P);
    const bool vec = reinterpret_cast<uintptr_t>(logits) % 8 == 0 && row_stride % 4 == 0;
    float* ws_s = static_cast<float*>(workspace);
    int* ws_i = reinterpret_cast<int*>(ws_s + B * P);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const uint32_t s0 = (uint32_t)seed, s1 = (uint32_t)(seed >> 32);
    const uint32_t o0 = (uint32_t)offset, o1 = (uint32_t)(offset >> 32);
    const dim3 grid((unsigned)P, (unsigned)B);
    if (logits_dtype == NV4_BF16 && vec)
        hipLaunchKernelGGL((gumbel_partial<true, true>), grid, dim3(SMP_PT), 0, st, logits, row_stride, temperatures,
                           (int)V, s0, s1, o0, o1, qpc, (int)P, ws_s, ws_i);
    else if (logits_dtype == NV4_BF16)
        hipLaunchKernelGGL((gumbel_partial<true, false>), grid, dim3(SMP_PT), 0, st, logits, row_stride,
                           temperatures, (int)V, s0, s1, o0, o1, qpc, (int)P, ws_s, ws_i);
    else
        hipLaunchKernelGGL((gumbel_partial<false, false>), grid, dim3(SMP_PT), 0, st, logits, row_stride,
                           temperatures, (int)V, s0, s1, o0, o1, qpc, (int)P, ws_s, ws_i);
    hipLaunchKernelGGL(gumbel_final, dim3((unsigned)B), dim3(64), 0, st, ws_s, ws_i, (int)P, out);
    return (int)hipGetLastError();
}

extern "C" void nv4_philox4x32_10(const uint32_t* counter, const uint32_t* key, uint32_t* out) {
    nv4::Philox4 c;
    for (int i = 0; i < 4; ++i) c.v[i] = counter[i];
    const nv4::Philox4 r = nv4::philox4x32_10(c, key[0], key[1]);
    for (int i = 0; i < 4; ++i) out[i] = r.v[i];
}
