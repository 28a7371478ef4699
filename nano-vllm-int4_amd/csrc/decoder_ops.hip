// Fused elementwise / normalisation ops of the Qwen3 decoder around the
// quantized linears (gfx950).  In the reference these are several
// torch.compile'd PyTorch ops each; here each is one launch, with the
// reference's rounding points kept:
//  * nv4_rmsnorm (nanovllm/layers/layernorm.py:16-40): x = float(x) [+
//    float(residual), residual_out = bf16(x)]; y = bf16(bf16(x * rsqrt(mean(x^2)
//    + eps)) * weight).  One workgroup per row; the sum of squares is taken in
//    fp32 in the fixed order of norm_ops.h (not torch's), which the fused K1
//    prologue shares.
//  * nv4_qk_norm_rope_store (nanovllm/models/qwen3.py:78-94 with
//    layers/rotary_embedding.py:6-48 and the KV store of
//    layers/attention.py:10-40): for every token of the fused qkv row, the
//    query and key heads get the per-head RMSNorm, then the rotary embedding
//    y1 = bf16(x1*cos - x2*sin), y2 = bf16(x2*cos + x1*sin) (fp32, each product
//    and the sum rounded separately) on the bf16 normalised values; queries go
//    to q_out, keys and values to their cache slot (and, when given, to
//    k_out / v_out).  Slots outside [0, num_slots) -- the reference's -1 --
//    are not stored; positions outside the cos/sin table read its row 0.
//    Sixteen lanes per (token, head): lane j owns dims 4j .. 4j+3 and their
//    rotation partners 64 + 4j .. 64 + 4j+3, in 8-byte accesses.
//  * nv4_silu_mul (nanovllm/layers/activation.py:8-11): bf16(bf16(silu(g)) * u)
//    with silu(g) = g / (1 + exp(-g)) in fp32.
#include "norm_ops.h"
#include "qk_ops.h"

namespace nv4 {
namespace {

// rows x H (H % 16 == 0, H <= 8192); 256 threads per row, thread t owning
// the 16-value units t and t + 256 (the fixed reduction order of
// norm_ops.h, shared with the fused K1 prologue).
template <bool RESID>
__global__ void __launch_bounds__(256)
rmsnorm_rows(const uint16_t* x, const uint16_t* resid_in, uint16_t* resid_out,
             const uint16_t* __restrict__ w, uint16_t* y, int H, float eps) {
    constexpr int MAXU = 2;
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const int t = threadIdx.x;
    const int nu = H / 16;
    float h[MAXU][16];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < MAXU; ++j) {
        const int u = t + j * 256;
        if (u < nu) {
            const int64_t off = row * H + u * 16;
            rms_load16<RESID>(x + off, RESID ? resid_in + off : nullptr, RESID ? resid_out + off : nullptr, h[j],
                              ss);
        }
    }
    const float r = rms_rsqrt256(ss, red, H, eps);
#pragma unroll
    for (int j = 0; j < MAXU; ++j) {
        const int u = t + j * 256;
        if (u < nu) {
            float v[16];
            rms_apply16(h[j], r, w + u * 16, v);
            v4u o0, o1;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                o0[k] = f32_to_bf16_rne(v[2 * k]) | (f32_to_bf16_rne(v[2 * k + 1]) << 16);
                o1[k] = f32_to_bf16_rne(v[8 + 2 * k]) | (f32_to_bf16_rne(v[8 + 2 * k + 1]) << 16);
            }
            *reinterpret_cast<v4u*>(y + row * H + u * 16) = o0;
            *reinterpret_cast<v4u*>(y + row * H + u * 16 + 8) = o1;
        }
    }
}

// Sixteen lanes per (token, head) of the fused qkv row [T, (Hq + 2 Hkv) * 128]
// (four per wave): lane j of an item holds dims 4j .. 4j + 3 and their rotary
// partners 64 + 4j .. 64 + 4j + 3, so every access is 8 bytes (16 for the
// cos/sin table) and the head's sum of squares is a 16-lane reduction.
__global__ void __launch_bounds__(256)
qk_norm_rope_store(const uint16_t* __restrict__ qkv, int64_t qkv_row, int T, int Hq, int Hkv,
                   const uint16_t* __restrict__ qw, const uint16_t* __restrict__ kw,
                   const float* __restrict__ cos_sin, const int64_t* __restrict__ positions,
                   int64_t max_position, const int32_t* __restrict__ slots, int64_t num_slots,
                   uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
                   uint16_t* __restrict__ k_out, uint16_t* __restrict__ v_out, float eps) {
    const int heads = Hq + 2 * Hkv;
    const int64_t item = (int64_t)blockIdx.x * (blockDim.x >> 4) + (threadIdx.x >> 4);
    if (item >= (int64_t)T * heads) return;  // whole 16-lane groups
    const int64_t tok = item / heads;
    const int h = (int)(item % heads);
    const int j4 = (threadIdx.x & 15) * 4;
    const uint16_t* src = qkv + tok * qkv_row + (int64_t)h * 128;
    // Every load that depends on no other load is written first; the cos/sin
    // row needs the position.
    const bool is_q = h < Hq;
    const uint16_t* wt = is_q ? qw : kw;
    int64_t pos = positions[tok];
    const int64_t slot = slots[tok];
    const uint2 xa = *reinterpret_cast<const uint2*>(src + j4), xb = *reinterpret_cast<const uint2*>(src + 64 + j4);
    const uint2 wa = *reinterpret_cast<const uint2*>(wt + j4), wb = *reinterpret_cast<const uint2*>(wt + 64 + j4);
    if (pos < 0 || pos >= max_position) pos = 0;  // out-of-table positions: never read outside the table
    const float* cs = cos_sin + pos * 128;
    const v4f c = *reinterpret_cast<const v4f*>(cs + j4), s = *reinterpret_cast<const v4f*>(cs + 64 + j4);
    if (h >= Hq + Hkv) {  // value head: copy to its slot (and v_out)
        const int kvh = h - Hq - Hkv;
        if (slot >= 0 && slot < num_slots) {
            uint16_t* dst = v_cache + (slot * Hkv + kvh) * 128;
            *reinterpret_cast<uint2*>(dst + j4) = xa;
            *reinterpret_cast<uint2*>(dst + 64 + j4) = xb;
        }
        if (v_out) {
            uint16_t* dst = v_out + (tok * Hkv + kvh) * 128;
            *reinterpret_cast<uint2*>(dst + j4) = xa;
            *reinterpret_cast<uint2*>(dst + 64 + j4) = xb;
        }
        return;
    }
    uint2 o1, o2;
    qk_head16(xa, xb, wa, wb, c, s, eps, o1, o2);
    if (is_q) {
        uint16_t* dst = q_out + (tok * Hq + h) * 128;
        *reinterpret_cast<uint2*>(dst + j4) = o1;
        *reinterpret_cast<uint2*>(dst + 64 + j4) = o2;
    } else {
        const int kvh = h - Hq;
        if (slot >= 0 && slot < num_slots) {
            uint16_t* dst = k_cache + (slot * Hkv + kvh) * 128;
            *reinterpret_cast<uint2*>(dst + j4) = o1;
            *reinterpret_cast<uint2*>(dst + 64 + j4) = o2;
        }
        if (k_out) {
            uint16_t* dst = k_out + (tok * Hkv + kvh) * 128;
            *reinterpret_cast<uint2*>(dst + j4) = o1;
            *reinterpret_cast<uint2*>(dst + 64 + j4) = o2;
        }
    }
}

__global__ void __launch_bounds__(256)
silu_mul(const uint16_t* __restrict__ gu, uint16_t* __restrict__ y, int64_t rows, int I) {
    const int64_t n8 = rows * (I / 8);
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= n8) return;
    const int64_t row = idx / (I / 8), c = idx % (I / 8);
    const v4u g = *reinterpret_cast<const v4u*>(gu + row * 2 * I + c * 8);
    const v4u u = *reinterpret_cast<const v4u*>(gu + row * 2 * I + I + c * 8);
    v4u out;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t pair = 0;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float gf = bf16_to_f32((g[k] >> (16 * e)) & 0xffffu);
            const float uf = bf16_to_f32((u[k] >> (16 * e)) & 0xffffu);
            pair |= f32_to_bf16_rne(silu_mul1(gf, uf)) << (16 * e);
        }
        out[k] = pair;
    }
    *reinterpret_cast<v4u*>(y + row * I + c * 8) = out;
}

}  // namespace
}  // namespace nv4

extern "C" int nv4_rmsnorm(const void* x, const void* residual_in, void* residual_out, const void* weight, void* y,
                           int64_t rows, int64_t H, float eps, void* stream) {
    using namespace nv4;
    if (!x || !weight || !y || (residual_in && !residual_out) || (!residual_in && residual_out)) return NV4_E_NULL;
    if (rows < 1 || rows > 0x7fffffffLL || H < 16 || H % 16 || H > 8192) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(weight) % 16 ||
        reinterpret_cast<uintptr_t>(y) % 16 || reinterpret_cast<uintptr_t>(residual_in) % 16 ||
        reinterpret_cast<uintptr_t>(residual_out) % 16)
        return NV4_E_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const auto* xp = static_cast<const uint16_t*>(x);
    const auto* wp = static_cast<const uint16_t*>(weight);
    auto* yp = static_cast<uint16_t*>(y);
    if (residual_in)
        hipLaunchKernelGGL(rmsnorm_rows<true>, dim3((unsigned)rows), dim3(256), 0, st, xp,
                           static_cast<const uint16_t*>(residual_in), static_cast<uint16_t*>(residual_out), wp, yp,
                           (int)H, eps);
    else
        hipLaunchKernelGGL(rmsnorm_rows<false>, dim3((unsigned)rows), dim3(256), 0, st, xp, nullptr, nullptr, wp, yp,
                           (int)H, eps);
    return (int)hipGetLastError();
}

extern "C" int nv4_qk_norm_rope_store(const void* qkv, int64_t qkv_row_stride, int64_t T, int64_t Hq, int64_t Hkv,
                                      const void* q_norm_w, const void* k_norm_w, const float* cos_sin,
                                      int64_t max_position, const int64_t* positions,
                                      const int32_t* slot_mapping, int64_t num_slots, void* q_out, void* k_cache,
                                      void* v_cache, void* k_out, void* v_out, float eps, void* stream) {
    using namespace nv4;
    if (!qkv || !q_norm_w || !k_norm_w || !cos_sin || !positions || !slot_mapping || !q_out || !k_cache || !v_cache)
        return NV4_E_NULL;
    if (T < 1 || Hq < 1 || Hkv < 1 || max_position < 1 || num_slots < 0 ||
        qkv_row_stride < (Hq + 2 * Hkv) * 128 || T * (Hq + 2 * Hkv) > 0x7fffffffLL * 16)
        return NV4_E_SHAPE;
    // 8-byte accesses to bf16 data, 16-byte reads of the cos/sin table.
    auto a8 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 8 == 0; };
    if (qkv_row_stride % 4 || !a8(qkv) || !a8(q_norm_w) || !a8(k_norm_w) || !a8(q_out) || !a8(k_cache) ||
        !a8(v_cache) || (k_out && !a8(k_out)) || (v_out && !a8(v_out)) ||
        reinterpret_cast<uintptr_t>(cos_sin) % 16)
        return NV4_E_ALIGN;
    const int64_t items = T * (Hq + 2 * Hkv);
    // Decode-sized calls: one wave (4 items) per workgroup, to spread over the
    // CUs; otherwise 256 threads (16 items).
    const int per = T <= 256 ? 4 : 16;
    hipLaunchKernelGGL(qk_norm_rope_store, dim3((unsigned)((items + per - 1) / per)), dim3(per * 16), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(qkv), qkv_row_stride, (int)T,
                       (int)Hq, (int)Hkv, static_cast<const uint16_t*>(q_norm_w),
                       static_cast<const uint16_t*>(k_norm_w), cos_sin, positions, max_position, slot_mapping,
                       num_slots,
                       static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
                       static_cast<uint16_t*>(k_out), static_cast<uint16_t*>(v_out), eps);
    return (int)hipGetLastError();
}

extern "C" int nv4_silu_mul(const void* gate_up, void* y, int64_t rows, int64_t I, void* stream) {
    using namespace nv4;
    if (!gate_up || !y) return NV4_E_NULL;
    if (rows < 1 || I < 8 || I % 8) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(gate_up) % 16 || reinterpret_cast<uintptr_t>(y) % 16) return NV4_E_ALIGN;
    const int64_t n8 = rows * (I / 8);
    if ((n8 + 255) / 256 > 0x7fffffffLL) return NV4_E_SHAPE;
    hipLaunchKernelGGL(silu_mul, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(gate_up), static_cast<uint16_t*>(y), rows, (int)I);
    return (int)hipGetLastError();
}
