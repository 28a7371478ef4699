/*
 * oracle.c -- CPU restatement of Nano-vLLM-INT4's quantized-linear numerics.
 *
 * TEST INFRASTRUCTURE ONLY.  The tests compare the HIP kernels of
 * nano-vllm-int4_amd/csrc against this file, and bench.py times it as the
 * CPU baseline beside them.  Nothing in the product path links, loads or calls it; the product
 * raises when its HIP library is missing instead of falling back here.
 *
 * Every function restates the reference's algorithm in plain C, with the
 * exact fp32 operation order the reference's CUDA execution uses.  Citations
 * are relative to the reference repository root.
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off, no fast-math: every fp32
 * operation below is a single IEEE round-to-nearest-even operation, fmaf is a
 * true fused multiply-add, and subnormals are kept).
 *
 * Pinning (what checks each function; tests/test_oracle_*.py):
 *   orc_rht_rows        impulse responses (closed form), dense float64
 *                       Kronecker products for K in {16,24,48,4096,12288},
 *                       exact-rational replay of the butterfly order on tiny
 *                       K, H12 orthogonality, inverse/norm preservation.
 *   orc_quantize_rows   the reference known-answer list (ties, clip-7/0.9,
 *                       BF16-scale-before-codes boundary, zero and 1e-40
 *                       groups), brute force over all codes of a group.
 *   orc_weight_quantize equals orc_quantize_rows at clip 0.9 with the CUDA
 *                       division; the reference self-test's zero row; exact
 *                       dyadic groups (codes recovered, zero error); every code
 *                       a nearest grid point of its bf16 scale; the scale
 *                       within half a bf16 ulp of mx*clip/7; torch's own CPU
 *                       evaluation of the reference expression for the CPU
 *                       division; ragged last group; two planted mistakes.
 *   orc_weight_dequantize exact products against float64.
 *   orc_pack_int4       the reference packed-byte vector 98 ba dc fe 10 32 54 76.
 *   orc_w4a4_gemm       brute-force integer dots with exact-rational FMA
 *                       replay, constant-dyadic-scale reductions, float64
 *                       relative-RMSE bound.
 *   orc_w4a16_gemm      closed-form dequantization of hand-built codes, float64
 *                       dense product.  The reference's own W4A16 kernel sums
 *                       in a nondeterministic split-K order and no reference
 *                       test covers it: its summation order is parity
 *                       unpinned, the 1e-2 relative bar applies.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_OK 0
#define ORC_EINVAL (-1)

/* ---------------------------------------------------------------- helpers */

static inline float f32_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t bits_from_f32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static inline float bf16_to_f32(uint16_t h) { return f32_from_bits((uint32_t)h << 16); }

/* fp32 -> bf16, round to nearest even; NaN stays NaN (quieted). */
static inline uint16_t f32_to_bf16(float f) {
    uint32_t u = bits_from_f32(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* IEEE binary16 -> fp32 (exact). */
static inline float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return f32_from_bits(sign);
        float v = ldexpf((float)man, -24);           /* subnormal: man * 2^-24, exact */
        return sign ? -v : v;
    }
    if (exp == 31) return f32_from_bits(sign | 0x7f800000u | (man << 13));
    return f32_from_bits(sign | ((exp + 112u) << 23) | (man << 13));
}

/* fp32 -> binary16, round to nearest even (used for the FP16-activation
 * W4A16 dequantization). */
static inline uint16_t f32_to_f16(float f) {
    uint32_t u = bits_from_f32(f);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);    /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {                                        /* below 2^-14: subnormal */
        float v = f32_from_bits(a);
        float q = nearbyintf(v * 16777216.0f);                    /* units of 2^-24, exact scale */
        return (uint16_t)(sign | (uint32_t)q);
    }
    uint32_t e = (a >> 23) - 112u, m = a & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rest = m & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

/* The fp32 constants of the reference quantizer (nanovllm/kernels/
 * rht_a4_tilelang.py:98,123-126; benchmarks/a4_group_quant.py:68 under CUDA,
 * where tensor/python-scalar division is a multiply by the fp32 reciprocal). */
static inline float c_clip(void)     { return (float)0.9; }            /* 0x1.ccccccp-1 */
static inline float c_inv7(void)     { return 1.0f / 7.0f; }           /* 0x1.24924ap-3 */
static inline float c_inv_sqrt12(void) { return (float)(1.0 / sqrt(12.0)); } /* 0x1.279a74p-2 */
static inline float c_tiny(void)     { return f32_from_bits(0x00800000u); } /* 2^-126 */

/* Paley H12 sign (benchmarks/rht_reference.py:15-23; kernel form
 * nanovllm/kernels/rht_a4_tilelang.py:93-95): entry [source][destination]. */
static inline int paley_positive(int s, int d) {
    if (s == 0 || d == 0) return 1;
    int delta = ((d - s) % 11 + 11) % 11;
    return delta == 1 || delta == 3 || delta == 4 || delta == 5 || delta == 9;
}

int orc_paley_sign(int s, int d) { return paley_positive(s, d) ? 1 : -1; }

static int is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

/* In-place Sylvester butterflies on a[0..F), strides 1,2,...,F/2 in increasing
 * order; the pair (i, i+h) with bit h clear in i becomes (lo+hi, lo-hi).
 * benchmarks/rht_reference.py:33-38; nanovllm/kernels/rht_a4_tilelang.py:62-84. */
static void fwht_f32(float* a, int64_t F) {
    for (int64_t h = 1; h < F; h <<= 1) {
        for (int64_t base = 0; base < F; base += 2 * h) {
            for (int64_t i = base; i < base + h; ++i) {
                float lo = a[i], hi = a[i + h];
                a[i] = lo + hi;
                a[i + h] = lo - hi;
            }
        }
    }
}

/* Mutation hooks: tests plant a known mistake here to show the pinning checks
 * reject it.  0 = faithful restatement. */
static int g_mutation = 0;
int orc_set_mutation(int m) { int old = g_mutation; g_mutation = m; return old; }

static void fwht_f32_descending(float* a, int64_t F) {
    for (int64_t h = F >> 1; h >= 1; h >>= 1) {
        for (int64_t base = 0; base < F; base += 2 * h) {
            for (int64_t i = base; i < base + h; ++i) {
                float lo = a[i], hi = a[i + h];
                a[i] = lo + hi;
                a[i + h] = lo - hi;
            }
        }
    }
}

/*
 * Rotate one row in place: a[k] (already x[k]*sign[k]) -> X D H.
 * layout 0 ("row_DH_paley12_kron_sylvester_v1", the reference layout):
 *   K = F (power of two): F-point Sylvester FWHT then x RN(1/sqrt F).
 *   K = 12*F: F-point FWHT per chunk s (k = s*F + c), x RN(1/sqrt F), then
 *   out[d] = RN(1/sqrt 12) * sum_{s=0..11} (+/-) a[s], summed from 0.0f in
 *   source order.  nanovllm/kernels/rht_a4_tilelang.py:58-100;
 *   benchmarks/rht_reference.py:42-54; benchmarks/a4_group_quant.py:47-56.
 * layout 1 ("block128"): 128-point FWHT on every aligned 128-block, then
 *   x RN(1/sqrt 128) = 0x1.6a09e6p-4; no H12 stage.  Not a reference layout:
 *   the literal "Hadamard-128 per 128-wide block" text of the configs.
 */
static int rotate_row(float* a, int64_t K, int layout, float* scratch12) {
    if (layout == 1) {
        if (K % 128) return ORC_EINVAL;
        const float norm = (float)(1.0 / sqrt(128.0));
        for (int64_t b = 0; b < K; b += 128) {
            fwht_f32(a + b, 128);
            for (int64_t i = 0; i < 128; ++i) a[b + i] = a[b + i] * norm;
        }
        return ORC_OK;
    }
    if (layout != 0) return ORC_EINVAL;
    int64_t F, C;
    if (is_pow2(K)) { F = K; C = 1; }
    else if (K % 12 == 0 && is_pow2(K / 12)) { F = K / 12; C = 12; }
    else return ORC_EINVAL;
    const float norm = (float)(1.0 / sqrt((double)F));
    for (int64_t s = 0; s < C; ++s) {
        if (g_mutation == 1) fwht_f32_descending(a + s * F, F);
        else fwht_f32(a + s * F, F);
        for (int64_t i = 0; i < F; ++i) a[s * F + i] = a[s * F + i] * norm;
    }
    if (C == 12) {
        const float inv12 = c_inv_sqrt12();
        for (int64_t c = 0; c < F; ++c) {
            for (int d = 0; d < 12; ++d) {
                float t = 0.0f;
                for (int s = 0; s < 12; ++s) {
                    float v = a[s * F + c];
                    int pos = paley_positive(s, d);
                    if (g_mutation == 2) pos = paley_positive(d, s);   /* transposed H12 */
                    t = t + (pos ? v : -v);
                }
                scratch12[d] = t * inv12;
            }
            for (int d = 0; d < 12; ++d) a[d * F + c] = scratch12[d];
        }
    }
    return ORC_OK;
}

/* x: bf16 bits [M,K]; signs [K] (+/-1); rotated: fp32 [M,K]. */
int orc_rht_rows(const uint16_t* x, const int8_t* signs, float* rotated,
                 int64_t M, int64_t K, int layout, int threads) {
    if (!x || !signs || !rotated || M < 0 || K < 1) return ORC_EINVAL;
    int err = ORC_OK;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static) reduction(min:err)
#endif
    for (int64_t m = 0; m < M; ++m) {
        float s12[12];
        float* a = rotated + m * K;
        /* a = fp32(x) * fp32(sign): exact (rht_a4_tilelang.py:58-60). */
        for (int64_t k = 0; k < K; ++k) a[k] = bf16_to_f32(x[m * K + k]) * (float)signs[k];
        int e = rotate_row(a, K, layout, s12);
        if (e < err) err = e;
    }
    (void)threads;
    return err;
}

/* Group-128 scale and codes of one group of fp32 values.
 * nanovllm/kernels/rht_a4_tilelang.py:101-131; benchmarks/a4_group_quant.py:60-70:
 *   mx = max|r|; t = RN(RN(mx*0.9f) * RN(1/7)); scale = mx==0 ? 1 : bf16(max(t, 2^-126));
 *   q = clamp(rint_even(r / fp32(scale)), -7, 7), IEEE division. */
static void quantize_group(const float* r, int8_t* q, uint16_t* scale_bits, int64_t G) {
    float mx = 0.0f;
    for (int64_t i = 0; i < G; ++i) { float v = fabsf(r[i]); if (v > mx) mx = v; }
    uint16_t sb;
    if (mx == 0.0f) {
        sb = f32_to_bf16(1.0f);
    } else {
        float t = mx * c_clip();
        t = t * c_inv7();
        if (g_mutation == 3) t = (mx * c_clip()) / 7.0f;              /* true division */
        if (t < c_tiny()) t = c_tiny();
        sb = f32_to_bf16(t);
    }
    float s = bf16_to_f32(sb);
    if (g_mutation == 4) s = mx == 0.0f ? 1.0f : fmaxf(mx * c_clip() * c_inv7(), c_tiny()); /* unrounded scale */
    for (int64_t i = 0; i < G; ++i) {
        float v = rintf(r[i] / s);
        if (v > 7.0f) v = 7.0f;
        if (v < -7.0f) v = -7.0f;
        q[i] = (int8_t)v;
    }
    *scale_bits = sb;
}

/* rotated fp32 [M,K] -> codes int8 [M,K] in [-7,7], scales bf16 [M,K/group]. */
int orc_quantize_rows(const float* r, int8_t* codes, uint16_t* scales,
                      int64_t M, int64_t K, int64_t group, int threads) {
    if (!r || !codes || !scales || M < 0 || group < 1 || K % group) return ORC_EINVAL;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
    for (int64_t m = 0; m < M; ++m)
        for (int64_t g = 0; g < K / group; ++g)
            quantize_group(r + m * K + g * group, codes + m * K + g * group,
                           scales + m * (K / group) + g, group);
    (void)threads;
    return ORC_OK;
}

/* Round-to-nearest weight quantizer with static groups along K (RTN-G128).
 * benchmarks/rht_gptq_grouped.py:27-34 (quantize_groups: each K-slice of
 * `group` columns, the last one possibly shorter, through
 * benchmarks/rht_reference.py:70-77 quantize_rows) and
 * benchmarks/kernel_bench_common.py:36-42 (grouped_quantize with a clip):
 *   mx = max|w| over the group; t = RN(mx * clip) then t / 7;
 *   scale = mx == 0 ? 1 : bf16(max(t, 2^-126));
 *   q = clamp(rint_even(w / fp32(scale)), -7, 7), IEEE division.
 * The reference evaluates these lines with torch, whose `tensor / 7` is an
 * IEEE division on the CPU but RN(t * RN(1/7)) on a CUDA device (division by
 * a host scalar becomes a multiplication by its fp32 reciprocal), so the
 * device the reference ran on is an argument: reciprocal = 0 for CPU tensors,
 * 1 for CUDA tensors.  quantize_rows is clip = 1 (RN(mx * 1) = mx) and
 * group = K.  w fp32 [N,K] -> codes int8 [N,K], scales bf16 [N,ceil(K/group)]. */
int orc_weight_quantize(const float* w, int8_t* codes, uint16_t* scales, int64_t N, int64_t K,
                        int64_t group, float clip, int reciprocal, int threads) {
    if (!w || !codes || !scales || N < 0 || K < 1 || group < 1 || !(clip > 0.0f)) return ORC_EINVAL;
    const int64_t G = (K + group - 1) / group;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t g = 0; g < G; ++g) {
            const int64_t k0 = g * group, len = (k0 + group <= K) ? group : K - k0;
            const float* r = w + n * K + k0;
            float mx = 0.0f;
            for (int64_t i = 0; i < len; ++i) { float v = fabsf(r[i]); if (v > mx) mx = v; }
            uint16_t sb;
            if (mx == 0.0f) {
                sb = f32_to_bf16(1.0f);
            } else {
                float t = mx * clip;
                t = reciprocal ? t * c_inv7() : t / 7.0f;
                if (g_mutation == 6) t = reciprocal ? t / 7.0f : t * c_inv7();   /* the other device's division */
                if (t < c_tiny()) t = c_tiny();
                sb = f32_to_bf16(t);
            }
            const float s = bf16_to_f32(sb);
            for (int64_t i = 0; i < len; ++i) {
                float v = rintf(r[i] / s);
                if (g_mutation == 7) v = truncf(r[i] / s);                     /* toward zero */
                if (v > 7.0f) v = 7.0f;
                if (v < -7.0f) v = -7.0f;
                codes[n * K + k0 + i] = (int8_t)v;
            }
            scales[n * G + g] = sb;
        }
    }
    (void)threads;
    return ORC_OK;
}

/* codes [N,K] x bf16 scales [N,ceil(K/group)] -> fp32 [N,K]: the product of a
 * code in [-8,7] and a bf16 value is exact in fp32
 * (benchmarks/rht_gptq_grouped.py:37-39). */
int orc_weight_dequantize(const int8_t* codes, const uint16_t* scales, float* out, int64_t N, int64_t K,
                          int64_t group) {
    if (!codes || !scales || !out || N < 0 || K < 1 || group < 1) return ORC_EINVAL;
    const int64_t G = (K + group - 1) / group;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k)
            out[n * K + k] = (float)codes[n * K + k] * bf16_to_f32(scales[n * G + k / group]);
    return ORC_OK;
}

/* Two signed nibbles per byte, even k in the low nibble
 * (benchmarks/rht_reference.py:80-83; rht_a4_bench_common.py:31). */
int orc_pack_int4(const int8_t* codes, int8_t* packed, int64_t n) {
    if (!codes || !packed || n % 2) return ORC_EINVAL;
    for (int64_t i = 0; i < n / 2; ++i)
        packed[i] = (int8_t)(uint8_t)(((uint8_t)codes[2 * i] & 15u) | (((uint8_t)codes[2 * i + 1] & 15u) << 4));
    return ORC_OK;
}

int orc_unpack_int4(const int8_t* packed, int8_t* codes, int64_t n) {
    if (!codes || !packed || n % 2) return ORC_EINVAL;
    for (int64_t i = 0; i < n / 2; ++i) {
        int lo = (uint8_t)packed[i] & 15, hi = ((uint8_t)packed[i] >> 4) & 15;
        codes[2 * i] = (int8_t)(lo >= 8 ? lo - 16 : lo);
        codes[2 * i + 1] = (int8_t)(hi >= 8 ? hi - 16 : hi);
    }
    return ORC_OK;
}

/* The whole K1 contract: bf16 X[M,K] -> packed int8 [M,K/2], bf16 scale [M,K/128]
 * (benchmarks/rht_a4_bench_common.py:19-36 contract; reference_parts :85-90). */
int orc_rht_quant_pack(const uint16_t* x, const int8_t* signs, int8_t* packed, uint16_t* scales,
                       int64_t M, int64_t K, int layout, int threads) {
    if (!x || !signs || !packed || !scales || M < 0 || K < 128 || K % 128) return ORC_EINVAL;
    int err = ORC_OK;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel reduction(min:err)
#endif
    {
        float* a = (float*)malloc((size_t)K * sizeof(float));
        int8_t* q = (int8_t*)malloc((size_t)K);
        float s12[12];
        if (!a || !q) { err = ORC_EINVAL; }
        else {
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
            for (int64_t m = 0; m < M; ++m) {
                for (int64_t k = 0; k < K; ++k) a[k] = bf16_to_f32(x[m * K + k]) * (float)signs[k];
                int e = rotate_row(a, K, layout, s12);
                if (e < err) err = e;
                for (int64_t g = 0; g < K / 128; ++g)
                    quantize_group(a + g * 128, q + g * 128, scales + m * (K / 128) + g, 128);
                orc_pack_int4(q, packed + m * (K / 2), K);
            }
        }
        free(a); free(q);
    }
    (void)threads;
    return err;
}

/*
 * Grouped INT4 GEMM, the numerical contract of nanovllm/kernels/
 * w4a4_grouped_kernel.py:64-90 with benchmarks/verify_w4a4_aw_grouped.py:13-29
 * (2-D weight scales) and benchmarks/verify_w4a4_grouped.py:17-25 (1-D):
 *   for g in order: d = sum_{k in g} qa*qw (exact int32);
 *   2-D: total = fmaf((float)d, fp32(sa[m,g]) * fp32(sw[n,g]), total); C = bf16(total)
 *   1-D: total = fmaf((float)d, fp32(sa[m,g]), total);  C = bf16(total * fp32(sw[n]))
 * out_fp32 != 0 writes the fp32 value before the final bf16 rounding.
 */
int orc_w4a4_gemm(const int8_t* a_packed, const int8_t* w_packed, const uint16_t* sa,
                  const uint16_t* sw, int sw_grouped, void* out, int out_fp32,
                  int64_t M, int64_t N, int64_t K, int threads) {
    if (!a_packed || !w_packed || !sa || !sw || !out || M < 0 || N < 0 || K < 128 || K % 128)
        return ORC_EINVAL;
    const int64_t G = K / 128;
    int8_t* qa = (int8_t*)malloc((size_t)(M * K > 0 ? M * K : 1));
    int8_t* qw = (int8_t*)malloc((size_t)(N * K > 0 ? N * K : 1));
    if (!qa || !qw) { free(qa); free(qw); return ORC_EINVAL; }
    orc_unpack_int4(a_packed, qa, M * K);
    orc_unpack_int4(w_packed, qw, N * K);
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static) collapse(2)
#endif
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            const int8_t* ar = qa + m * K;
            const int8_t* wr = qw + n * K;
            float total = 0.0f;
            for (int64_t g = 0; g < G; ++g) {
                int32_t d = 0;
                for (int64_t k = g * 128; k < g * 128 + 128; ++k) d += (int32_t)ar[k] * (int32_t)wr[k];
                float sag = bf16_to_f32(sa[m * G + g]);
                if (sw_grouped) {
                    float s = sag * bf16_to_f32(sw[n * G + g]);
                    total = g_mutation == 5 ? total + (float)d * s : fmaf((float)d, s, total);
                } else {
                    total = fmaf((float)d, sag, total);
                }
            }
            if (!sw_grouped) total = total * bf16_to_f32(sw[n]);
            if (out_fp32) ((float*)out)[m * N + n] = total;
            else ((uint16_t*)out)[m * N + n] = f32_to_bf16(total);
        }
    }
    free(qa); free(qw);
    (void)threads;
    return ORC_OK;
}

/* Integer group dots only: d[m, n, g] (the part the kernels must match bit for bit). */
int orc_w4a4_group_dots(const int8_t* a_packed, const int8_t* w_packed, int32_t* dots,
                        int64_t M, int64_t N, int64_t K) {
    if (!a_packed || !w_packed || !dots || K % 128) return ORC_EINVAL;
    const int64_t G = K / 128;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n)
            for (int64_t g = 0; g < G; ++g) {
                int32_t d = 0;
                for (int64_t j = g * 64; j < g * 64 + 64; ++j) {
                    uint8_t pa = (uint8_t)a_packed[m * K / 2 + j], pw = (uint8_t)w_packed[n * K / 2 + j];
                    int alo = pa & 15, ahi = pa >> 4, wlo = pw & 15, whi = pw >> 4;
                    alo -= alo >= 8 ? 16 : 0; ahi -= ahi >= 8 ? 16 : 0;
                    wlo -= wlo >= 8 ? 16 : 0; whi -= whi >= 8 ? 16 : 0;
                    d += alo * wlo + ahi * whi;
                }
                dots[(m * N + n) * G + g] = d;
            }
    return ORC_OK;
}

/*
 * W4A16 dequantization (nanovllm/layers/linear_w4a16.py:45-55, GPTQ "v1"
 * zero convention):  q = nibble k%8 of qweight[k/8, n]; z = nibble n%8 of
 * qzeros[k/group, n/8]; s = scales[k/group, n] (fp16).
 *   x_dtype 0 (bf16, the reference): deq = bf16(fp32(bf16(q - z - 1)) * fp32(bf16(s)))
 *   x_dtype 1 (fp16):                deq = fp16(fp32(q - z - 1) * fp32(s))
 * deq_out: fp32 [K, N] holding the rounded dequantized weights.
 */
int orc_w4a16_dequant(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                      float* deq_out, int64_t N, int64_t K, int64_t group, int x_dtype) {
    if (!qweight || !qzeros || !scales || !deq_out || K % 8 || N % 8 || group < 8 || K % group)
        return ORC_EINVAL;
    for (int64_t k = 0; k < K; ++k) {
        for (int64_t n = 0; n < N; ++n) {
            uint32_t word = (uint32_t)qweight[(k / 8) * N + n];
            int q = (int)((word >> (4 * (k % 8))) & 15u);
            uint32_t zw = (uint32_t)qzeros[(k / group) * (N / 8) + n / 8];
            int z = (int)((zw >> (4 * (n % 8))) & 15u);
            uint16_t s = scales[(k / group) * N + n];
            float v;
            if (x_dtype == 0) {
                float sb = bf16_to_f32(f32_to_bf16(f16_to_f32(s)));
                v = bf16_to_f32(f32_to_bf16((float)(q - z - 1) * sb));
            } else {
                v = f16_to_f32(f32_to_f16((float)(q - z - 1) * f16_to_f32(s)));
            }
            deq_out[k * N + n] = v;
        }
    }
    return ORC_OK;
}

/* y[m,n] = sum_k fp32(x[m,k]) * deq[k,n], accumulated in float64 (the
 * reference accumulates in fp32 per split and adds eight BF16 partials with
 * atomics, an unpinnable order; the oracle gives the exact-sum baseline). */
int orc_w4a16_gemm(const uint16_t* x, int x_dtype, const int32_t* qweight, const int32_t* qzeros,
                   const uint16_t* scales, double* out, int64_t M, int64_t N, int64_t K,
                   int64_t group, int threads) {
    if (!x || !out || M < 0) return ORC_EINVAL;
    float* deq = (float*)malloc((size_t)(K * N) * sizeof(float));
    if (!deq) return ORC_EINVAL;
    int e = orc_w4a16_dequant(qweight, qzeros, scales, deq, N, K, group, x_dtype);
    if (e) { free(deq); return e; }
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
    for (int64_t m = 0; m < M; ++m) {
        double* row = out + m * N;
        for (int64_t n = 0; n < N; ++n) row[n] = 0.0;
        for (int64_t k = 0; k < K; ++k) {
            double xv = x_dtype == 0 ? (double)bf16_to_f32(x[m * K + k]) : (double)f16_to_f32(x[m * K + k]);
            const float* dr = deq + k * N;
            for (int64_t n = 0; n < N; ++n) row[n] += xv * (double)dr[n];
        }
    }
    free(deq);
    (void)threads;
    return ORC_OK;
}

/* Conversions exposed for the tests. */
void orc_f32_to_bf16(const float* in, uint16_t* out, int64_t n) { for (int64_t i = 0; i < n; ++i) out[i] = f32_to_bf16(in[i]); }
void orc_bf16_to_f32(const uint16_t* in, float* out, int64_t n) { for (int64_t i = 0; i < n; ++i) out[i] = bf16_to_f32(in[i]); }
void orc_f32_to_f16(const float* in, uint16_t* out, int64_t n) { for (int64_t i = 0; i < n; ++i) out[i] = f32_to_f16(in[i]); }
void orc_f16_to_f32(const uint16_t* in, float* out, int64_t n) { for (int64_t i = 0; i < n; ++i) out[i] = f16_to_f32(in[i]); }

/* The quantizer constants, for the tests that pin their bit patterns. */
uint32_t orc_constant_bits(int which) {
    switch (which) {
        case 0: return bits_from_f32(c_clip());
        case 1: return bits_from_f32(c_inv7());
        case 2: return bits_from_f32(c_inv_sqrt12());
        case 3: return bits_from_f32((float)(1.0 / sqrt(128.0)));
        default: return 0;
    }
}

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
