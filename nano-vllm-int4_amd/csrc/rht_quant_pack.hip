// K1: fused randomized Hadamard transform + group-128 INT4 quantization +
// nibble packing, for gfx950.  The reference-layout row transforms live in
// k1_row.h; this file holds the kernels and the C ABI entry points,
// including K1 with the producer of its input fused in front (add+RMSNorm
// for the qkv and gate_up inputs, SiLU-mul for the down input): the row is
// computed, rounded to bf16 as the separate op would store it, and fed to the
// transform without the round trip through memory.
#include "k1_row.h"
#include "norm_ops.h"

namespace nv4 {
namespace {

// Row sources: load(row, c0, raw) issues the loads of one thread's 16
// columns c0..c0+15 of a row; values(raw, row, c0, v) turns them into the
// fp32 values the transform takes: the bf16 input itself, or the output of
// the fused producer rounded to bf16 as the separate op would store it.
struct RowX {  // bf16 rows of width K
    const uint16_t* __restrict__ x;
    int K;
    struct Raw { v4u a, b; };
    __device__ __forceinline__ void load(int64_t row, int c0, Raw& r) const {
        const uint16_t* p = x + row * K + c0;
        r.a = *reinterpret_cast<const v4u*>(p);
        r.b = *reinterpret_cast<const v4u*>(p + 8);
    }
    __device__ __forceinline__ void values(const Raw& r, int64_t, int, float (&v)[16]) const {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t xw = i < 8 ? r.a[(i & 7) >> 1] : r.b[(i & 7) >> 1];
            v[i] = bf16_to_f32((xw >> (16 * (i & 1))) & 0xffffu);
        }
    }
};

struct RowSilu {  // SiLU(gate) * up of [M, 2K] gate/up rows
    const uint16_t* __restrict__ gu;
    int K;
    struct Raw { v4u g0, g1, u0, u1; };
    __device__ __forceinline__ void load(int64_t row, int c0, Raw& r) const {
        const uint16_t* g = gu + row * 2 * K + c0;
        r.g0 = *reinterpret_cast<const v4u*>(g);
        r.g1 = *reinterpret_cast<const v4u*>(g + 8);
        r.u0 = *reinterpret_cast<const v4u*>(g + K);
        r.u1 = *reinterpret_cast<const v4u*>(g + K + 8);
    }
    __device__ __forceinline__ void values(const Raw& r, int64_t, int, float (&v)[16]) const {
        silu_mul16(r.g0, r.g1, r.u0, r.u1, v);
    }
};

// add + RMSNorm of 4096-wide rows (K4_THREADS = 256 threads; thread t's unit
// is columns 16t..16t+15, the unit nv4_rmsnorm's thread t owns, so the sum
// of squares runs in nv4_rmsnorm's order).  The caller sets the thread's
// norm weights w0/w1 (loaded ahead of the row) and red (4 floats of LDS).
template <bool RESID>
struct RowRms {
    const uint16_t* x;
    const uint16_t* res_in;
    uint16_t* res_out;
    float eps;
    v4u w0, w1;
    float* red;
    struct Raw { v4u x0, x1, r0, r1; };
    __device__ __forceinline__ void load(int64_t row, int c0, Raw& r) const {
        const int64_t off = row * 4096 + c0;
        r.x0 = *reinterpret_cast<const v4u*>(x + off);
        r.x1 = *reinterpret_cast<const v4u*>(x + off + 8);
        r.r0 = RESID ? *reinterpret_cast<const v4u*>(res_in + off) : v4u{0u, 0u, 0u, 0u};
        r.r1 = RESID ? *reinterpret_cast<const v4u*>(res_in + off + 8) : v4u{0u, 0u, 0u, 0u};
    }
    __device__ __forceinline__ void values(const Raw& r, int64_t row, int c0, float (&v)[16]) const {
        float h[16], ss = 0.0f;
        rms_h16<RESID>(r.x0, r.x1, r.r0, r.r1, RESID ? res_out + row * 4096 + c0 : nullptr, h, ss);
        rms_apply16(h, rms_rsqrt256(ss, red, 4096, eps), w0, w1, v);
    }
};

// Prefetch tail of decode-sized launches.  At M <= 32 K1 keeps one
// workgroup per row busy (32 of the CUs) for a few microseconds while HBM
// idles.  Workgroups past the M rows read `bytes` of a buffer -- the weights
// of the GEMM that consumes these codes -- and discard them, so that the
// GEMM launched next finds them in the memory-side Infinity Cache instead of
// HBM.  Nothing is written, and no result depends on it.
struct Prefetch {
    const int8_t* p = nullptr;
    int64_t bytes = 0;  // a multiple of 16
};
constexpr int PF_LOADS = 8;  // 16-byte loads per thread of a prefetch workgroup

// True for a prefetch workgroup, one past the `rows` K1 workgroups (which has
// then issued its loads).  The loads are unconditional (offsets clamped into
// the buffer), so none waits alone.
template <int T>
__device__ __forceinline__ bool prefetch_tail(int rows, const int8_t* __restrict__ p, int64_t bytes) {
    if ((int)blockIdx.x < rows) return false;
    const int64_t base = (int64_t)(blockIdx.x - rows) * (T * 16 * PF_LOADS);
    v4u v[PF_LOADS];
#pragma unroll
    for (int i = 0; i < PF_LOADS; ++i) {
        const int64_t off = min(base + (int64_t)(i * T + threadIdx.x) * 16, bytes - 16);
        v[i] = *reinterpret_cast<const v4u*>(p + off);
    }
    __builtin_amdgcn_sched_barrier(0);  // all loads in flight before the first use
    v4u acc = v[0];
#pragma unroll
    for (int i = 1; i < PF_LOADS; ++i) acc ^= v[i];
    asm volatile("" ::"v"(acc[0] ^ acc[1] ^ acc[2] ^ acc[3]));  // keep the loads
    return true;
}

inline unsigned prefetch_grid(int M, const Prefetch& pf, int threads) {
    const int64_t per = (int64_t)threads * 16 * PF_LOADS;
    return (unsigned)(M + (pf.bytes > 0 ? (pf.bytes + per - 1) / per : 0));
}

// K = 4096: one workgroup of K4_THREADS threads per row.  RT: the codes go
// to the row-tiled layout (packed_dst) instead of [M][K/2].
template <bool RT, class Src>
__device__ __forceinline__ void k1_k4096_body(const Src& src, const int8_t* __restrict__ signs,
                                              int8_t* __restrict__ packed, uint16_t* __restrict__ scale,
                                              float* buf) {
    const v4u sv = k1_signs4096(signs);
    const int64_t row = blockIdx.x;
    const int c0 = 16 * threadIdx.x;
    typename Src::Raw raw;
    src.load(row, c0, raw);
    k1_row4096([&](int, float (&v)[16]) { src.values(raw, row, c0, v); }, sv,
               packed_dst<RT>(packed, row, threadIdx.x, 4096), scale + row * 32, buf);
}

// The K1 kernels take plain scalars and pointers, the row count and the
// row's inputs first: the first 14 argument dwords are preloaded into SGPRs
// when the waves launch (a struct argument would end the preload there), so
// a row's loads issue without a round trip to the kernel-argument buffer.
// The prefetch workgroups' arguments come last and are loaded as usual.
template <class Src, bool RT>
__global__ void __launch_bounds__(K4_THREADS)
k1_k4096(int rows, const uint16_t* __restrict__ src_p, const int8_t* __restrict__ signs,
         int8_t* __restrict__ packed, uint16_t* __restrict__ scale, const int8_t* __restrict__ pf_p,
         int64_t pf_bytes) {
    __shared__ float buf[K4_LDS];
    if (prefetch_tail<K4_THREADS>(rows, pf_p, pf_bytes)) return;
    k1_k4096_body<RT>(Src{src_p, 4096}, signs, packed, scale, buf);
}

// add + RMSNorm in front: the norm weights are loaded ahead of the row.
template <bool RESID, bool RT>
__global__ void __launch_bounds__(K4_THREADS)
k1_k4096_rms(int rows, float eps, const uint16_t* x, const uint16_t* res_in, uint16_t* res_out,
             const uint16_t* __restrict__ nw, const int8_t* __restrict__ signs, int8_t* __restrict__ packed,
             uint16_t* __restrict__ scale, const int8_t* __restrict__ pf_p, int64_t pf_bytes) {
    __shared__ float buf[K4_LDS];
    __shared__ float red[4];
    if (prefetch_tail<K4_THREADS>(rows, pf_p, pf_bytes)) return;
    const RowRms<RESID> src{x, res_in, res_out, eps, *reinterpret_cast<const v4u*>(nw + 16 * threadIdx.x),
                            *reinterpret_cast<const v4u*>(nw + 16 * threadIdx.x + 8), red};
    k1_k4096_body<RT>(src, signs, packed, scale, buf);
}

// K = 12288: one workgroup of 1024 threads per row.  Waves 12-15 hold no
// columns in the butterfly phases (they join the H12 stage); their loads
// repeat the row's last 16 columns, so that every load is unconditional.
template <class Src, bool RT>
__global__ void __launch_bounds__(K12_THREADS)
k1_k12288(int rows, const uint16_t* __restrict__ src_p, const int8_t* __restrict__ signs,
          int8_t* __restrict__ packed, uint16_t* __restrict__ scale, const int8_t* __restrict__ pf_p,
          int64_t pf_bytes) {
    __shared__ float buf[K12_LDS];
    if (prefetch_tail<K12_THREADS>(rows, pf_p, pf_bytes)) return;
    const Src src{src_p, 12288};
    const v4u sv = k1_signs12288(signs);
    const int64_t row = blockIdx.x;
    const int c0 = 16 * min((int)threadIdx.x, 767);
    typename Src::Raw raw;
    src.load(row, c0, raw);
    k1_row12288([&](int, float (&v)[16]) { src.values(raw, row, c0, v); }, sv,
                packed_dst<RT>(packed, row, min((int)threadIdx.x, 767), 12288), scale + row * 96, buf);
}

template <class Src>
hipError_t launch_k4096(const uint16_t* src_p, const int8_t* signs, int8_t* packed, uint16_t* scale, int M, bool rt,
                        Prefetch pf, hipStream_t st) {
    const dim3 grid(prefetch_grid(M, pf, K4_THREADS));
    if (rt)
        hipLaunchKernelGGL((k1_k4096<Src, true>), grid, dim3(K4_THREADS), 0, st, M, src_p, signs, packed, scale,
                           pf.p, pf.bytes);
    else
        hipLaunchKernelGGL((k1_k4096<Src, false>), grid, dim3(K4_THREADS), 0, st, M, src_p, signs, packed, scale,
                           pf.p, pf.bytes);
    return hipGetLastError();
}

template <class Src>
hipError_t launch_k12288(const uint16_t* src_p, const int8_t* signs, int8_t* packed, uint16_t* scale, int M,
                         bool rt, Prefetch pf, hipStream_t st) {
    const dim3 grid(prefetch_grid(M, pf, K12_THREADS));
    if (rt)
        hipLaunchKernelGGL((k1_k12288<Src, true>), grid, dim3(K12_THREADS), 0, st, M, src_p, signs, packed, scale,
                           pf.p, pf.bytes);
    else
        hipLaunchKernelGGL((k1_k12288<Src, false>), grid, dim3(K12_THREADS), 0, st, M, src_p, signs, packed, scale,
                           pf.p, pf.bytes);
    return hipGetLastError();
}

template <bool RESID>
hipError_t launch_rms4096(const uint16_t* x, const uint16_t* res_in, uint16_t* res_out, float eps,
                          const uint16_t* nw, const int8_t* signs, int8_t* packed, uint16_t* scale, int M, bool rt,
                          Prefetch pf, hipStream_t st) {
    const dim3 grid(prefetch_grid(M, pf, K4_THREADS));
    if (rt)
        hipLaunchKernelGGL((k1_k4096_rms<RESID, true>), grid, dim3(K4_THREADS), 0, st, M, eps, x, res_in, res_out,
                           nw, signs, packed, scale, pf.p, pf.bytes);
    else
        hipLaunchKernelGGL((k1_k4096_rms<RESID, false>), grid, dim3(K4_THREADS), 0, st, M, eps, x, res_in, res_out,
                           nw, signs, packed, scale, pf.p, pf.bytes);
    return hipGetLastError();
}

// block128 layout: every aligned 128-block gets its own 128-point Sylvester
// transform, then x RN(1/sqrt 128).  Each thread owns 16 contiguous values
// (butterfly bits 0-3 in registers); bits 4-6 are lanes xor 1, 2, 4.
__global__ void __launch_bounds__(256)
k1_block128(const uint16_t* __restrict__ x, const int8_t* __restrict__ signs,
            int8_t* __restrict__ packed, uint16_t* __restrict__ scale, int64_t units, int K) {
    const int64_t uu = (int64_t)blockIdx.x * 256 + threadIdx.x;
    // units is a multiple of 8, so the 8-lane groups that exchange values
    // below are either wholly in range or wholly out.
    if (uu >= units) return;
    const int kcol = (int)((uu * 16) % K);
    float a[16];
    {
        const uint4 xv = *reinterpret_cast<const uint4*>(x + uu * 16);
        const uint4 xv2 = *reinterpret_cast<const uint4*>(x + uu * 16 + 8);
        const uint4 sv = *reinterpret_cast<const uint4*>(signs + kcol);
        const uint32_t xw[8] = {xv.x, xv.y, xv.z, xv.w, xv2.x, xv2.y, xv2.z, xv2.w};
        const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint32_t h = (xw[i >> 1] >> (16 * (i & 1))) & 0xffffu;
            const int sg = (int)(int8_t)((sw[i >> 2] >> (8 * (i & 3))) & 0xffu);
            a[i] = bf16_to_f32(h) * (float)sg;
        }
    }
#pragma unroll
    for (int rb = 1; rb < 16; rb <<= 1)
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if ((r & rb) == 0) {
                const float lo = a[r], hi = a[r + rb];
                a[r] = lo + hi;
                a[r + rb] = lo - hi;
            }
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int lb = 1; lb < 8; lb <<= 1) {
        const bool upper = (lane & lb) != 0;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float other = __shfl_xor(a[r], lb);
            a[r] = upper ? (other - a[r]) : (a[r] + other);
        }
    }
    const float norm = 0x1.6a09e6p-4f;  // RN(1/sqrt 128)
#pragma unroll
    for (int i = 0; i < 16; ++i) a[i] = a[i] * norm;
    quantize16_store(a, packed + uu * 8, scale + (uu >> 3), (lane & 7) == 0);
}

}  // namespace
}  // namespace nv4

namespace nv4 {
namespace {

// Prefetch arguments: NULL / 0 for none; otherwise bytes a positive multiple
// of 16 (at most 2^40) and the buffer 16-byte aligned.
int check_prefetch(const void* p, int64_t bytes) {
    if (bytes == 0) return NV4_OK;
    if (!p) return NV4_E_NULL;
    if (bytes < 16 || bytes % 16 || bytes > (1LL << 40)) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(p) % 16) return NV4_E_ALIGN;
    return NV4_OK;
}

int quant_pack_impl(const void* x, const int8_t* signs, int8_t* packed, void* scale, int64_t M, int64_t K,
                    int layout, bool rt, Prefetch pf, void* stream) {
    if (!x || !signs || !packed || !scale) return NV4_E_NULL;
    if (M < 1 || M > 0x7fffffffLL) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(packed) % 8 ||
        reinterpret_cast<uintptr_t>(scale) % 2 || reinterpret_cast<uintptr_t>(signs) % 16)
        return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (layout == NV4_LAYOUT_REFERENCE) {
        const auto* xp = static_cast<const uint16_t*>(x);
        auto* sp = static_cast<uint16_t*>(scale);
        if (K == 4096) return (int)launch_k4096<RowX>(xp, signs, packed, sp, (int)M, rt, pf, st);
        if (K == 12288) return (int)launch_k12288<RowX>(xp, signs, packed, sp, (int)M, rt, pf, st);
        return NV4_E_SHAPE;
    }
    if (layout == NV4_LAYOUT_BLOCK128 && !rt) {
        if (K < 128 || K % 128 || K > 65536) return NV4_E_SHAPE;
        const int64_t units = M * (K / 16);
        const int64_t blocks = (units + 255) / 256;
        if (blocks > 0x7fffffffLL) return NV4_E_SHAPE;
        hipLaunchKernelGGL(k1_block128, dim3((unsigned)blocks), dim3(256), 0, st,
                           static_cast<const uint16_t*>(x), signs, packed, static_cast<uint16_t*>(scale),
                           units, (int)K);
        return (int)hipGetLastError();
    }
    return NV4_E_LAYOUT;
}

int rmsnorm_quant_impl(const void* x, const void* residual_in, void* residual_out, const void* norm_weight,
                       float eps, const int8_t* signs, int8_t* packed, void* scale, int64_t M, int64_t K, bool rt,
                       Prefetch pf, void* stream) {
    if (!x || !norm_weight || !signs || !packed || !scale || (!residual_in) != (!residual_out)) return NV4_E_NULL;
    if (M < 1 || M > 0x7fffffffLL || K != 4096) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(residual_in) % 16 ||
        reinterpret_cast<uintptr_t>(residual_out) % 16 || reinterpret_cast<uintptr_t>(norm_weight) % 16 ||
        reinterpret_cast<uintptr_t>(packed) % 8 || reinterpret_cast<uintptr_t>(scale) % 2 ||
        reinterpret_cast<uintptr_t>(signs) % 16)
        return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const auto* xp = static_cast<const uint16_t*>(x);
    const auto* wp = static_cast<const uint16_t*>(norm_weight);
    auto* sp = static_cast<uint16_t*>(scale);
    if (residual_in)
        return (int)launch_rms4096<true>(xp, static_cast<const uint16_t*>(residual_in),
                                         static_cast<uint16_t*>(residual_out), eps, wp, signs, packed, sp, (int)M, rt,
                                         pf, st);
    return (int)launch_rms4096<false>(xp, nullptr, nullptr, eps, wp, signs, packed, sp, (int)M, rt, pf, st);
}

int silu_quant_impl(const void* gate_up, const int8_t* signs, int8_t* packed, void* scale, int64_t M, int64_t K,
                    bool rt, Prefetch pf, void* stream) {
    if (!gate_up || !signs || !packed || !scale) return NV4_E_NULL;
    if (M < 1 || M > 0x7fffffffLL || (K != 4096 && K != 12288)) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(gate_up) % 16 || reinterpret_cast<uintptr_t>(packed) % 8 ||
        reinterpret_cast<uintptr_t>(scale) % 2 || reinterpret_cast<uintptr_t>(signs) % 16)
        return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const auto* gp = static_cast<const uint16_t*>(gate_up);
    auto* sp = static_cast<uint16_t*>(scale);
    if (K == 4096) return (int)launch_k4096<RowSilu>(gp, signs, packed, sp, (int)M, rt, pf, st);
    return (int)launch_k12288<RowSilu>(gp, signs, packed, sp, (int)M, rt, pf, st);
}

}  // namespace
}  // namespace nv4

extern "C" int nv4_rht_quant_pack(const void* x, const int8_t* signs, int8_t* packed, void* scale,
                                  int64_t M, int64_t K, int layout, void* stream) {
    return nv4::quant_pack_impl(x, signs, packed, scale, M, K, layout, false, nv4::Prefetch{}, stream);
}

extern "C" int nv4_rht_quant_pack_rowtiled(const void* x, const int8_t* signs, int8_t* packed_rt, void* scale,
                                           int64_t M, int64_t K, const void* prefetch, int64_t prefetch_bytes,
                                           void* stream) {
    const int rc = nv4::check_prefetch(prefetch, prefetch_bytes);
    if (rc != NV4_OK) return rc;
    return nv4::quant_pack_impl(x, signs, packed_rt, scale, M, K, NV4_LAYOUT_REFERENCE, true,
                                nv4::Prefetch{static_cast<const int8_t*>(prefetch), prefetch_bytes}, stream);
}

extern "C" int nv4_rmsnorm_rht_quant_pack(const void* x, const void* residual_in, void* residual_out,
                                          const void* norm_weight, float eps, const int8_t* signs, int8_t* packed,
                                          void* scale, int64_t M, int64_t K, void* stream) {
    return nv4::rmsnorm_quant_impl(x, residual_in, residual_out, norm_weight, eps, signs, packed, scale, M, K, false,
                                   nv4::Prefetch{}, stream);
}

extern "C" int nv4_rmsnorm_rht_quant_pack_rowtiled(const void* x, const void* residual_in, void* residual_out,
                                                   const void* norm_weight, float eps, const int8_t* signs,
                                                   int8_t* packed_rt, void* scale, int64_t M, int64_t K,
                                                   const void* prefetch, int64_t prefetch_bytes, void* stream) {
    const int rc = nv4::check_prefetch(prefetch, prefetch_bytes);
    if (rc != NV4_OK) return rc;
    return nv4::rmsnorm_quant_impl(x, residual_in, residual_out, norm_weight, eps, signs, packed_rt, scale, M, K,
                                   true, nv4::Prefetch{static_cast<const int8_t*>(prefetch), prefetch_bytes},
                                   stream);
}

extern "C" int nv4_silu_mul_rht_quant_pack(const void* gate_up, const int8_t* signs, int8_t* packed, void* scale,
                                           int64_t M, int64_t K, void* stream) {
    return nv4::silu_quant_impl(gate_up, signs, packed, scale, M, K, false, nv4::Prefetch{}, stream);
}

extern "C" int nv4_silu_mul_rht_quant_pack_rowtiled(const void* gate_up, const int8_t* signs, int8_t* packed_rt,
                                                    void* scale, int64_t M, int64_t K, const void* prefetch,
                                                    int64_t prefetch_bytes, void* stream) {
    const int rc = nv4::check_prefetch(prefetch, prefetch_bytes);
    if (rc != NV4_OK) return rc;
    return nv4::silu_quant_impl(gate_up, signs, packed_rt, scale, M, K, true,
                                nv4::Prefetch{static_cast<const int8_t*>(prefetch), prefetch_bytes}, stream);
}
