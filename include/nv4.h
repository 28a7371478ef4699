/*
 * nv4.h -- C ABI of the MI355X (gfx950) quantized-linear library libnv4.so.
 *
 * Plain pointers and sizes only.  bf16/fp16 buffers are passed as void*;
 * `stream` is a hipStream_t (NULL = the null stream) passed as void* so this
 * header needs no HIP headers.  The caller owns every buffer; no entry point
 * allocates, frees or synchronises.  Launches are asynchronous on `stream`
 * and may be captured into a HIP graph.  Inputs are never modified and
 * nothing outside the output ranges is written.
 *
 * Return value: NV4_OK (0); a negative NV4_E* code when the arguments are
 * rejected (nothing is launched); or a positive hipError_t from the launch.
 * Nothing aborts or prints.
 *
 * Entry points replace, one for one, the kernels behind the reference's
 * Python operators (paths relative to the reference repository):
 *   nv4_rht_quant_pack  <- nanovllm/kernels/rht_a4_tilelang.py:150 rht_quant_pack
 *                          (kernel :37-136)
 *   nv4_w4a4_gemm       <- nanovllm/kernels/w4a4_grouped_kernel.py:104 w4a4_grouped_gemm
 *                          and :32 compile_grouped_gemm(..., output_fp32, weight_grouped)
 *   nv4_w4a4_linear     <- nanovllm/layers/linear_w4a4.py:27-35 W4A4Linear.forward
 *                          (rht_quant_pack + w4a4_grouped_gemm)
 *   nv4_w4a4_gemm_tiled, nv4_w4a4_linear_tiled, nv4_w4a4_tile_weights,
 *   nv4_w4a4_untile_weights <- the same two operators on weights stored in an
 *                          MFMA-tiled order (no counterpart in the reference,
 *                          whose kernels read [N,K/2]; W4A4Linear keeps the
 *                          reference layout in its state dict)
 *   nv4_w4a4_gemm_f8    <- w4a4_grouped_gemm (w4a4_grouped_kernel.py:104) for
 *                          prefill-sized M: the same operator on the fp8 matrix
 *                          cores, with a caller workspace for the e4m3 operands
 *   nv4_w4a4_gemm_f6, nv4_w4a4_gemm_f6_workspace <- the same, on the fp6 matrix
 *                          cores (e3m2 operands in 128-row tiles)
 *   nv4_w4a4_weights_to_f6, nv4_w4a4_weights_f6_bytes <- no counterpart in the
 *                          reference: the weight half of that conversion, done
 *                          once per layer and kept beside the INT4 weights
 *   nv4_w4a16_gemm, nv4_w4a16_gemm_ws, nv4_w4a16_dequant <- nanovllm/layers/linear_w4a16.py:11
 *                          tl_dequant_matmul_w4a16 (called from W4A16Linear.forward
 *                          :128-148; the reference splits K 8 ways with bf16 atomics,
 *                          the _ws form splits K into 1024-deep fp32 partials, and
 *                          prefill-sized M dequantizes once for a library GEMM)
 *   nv4_prefill_attention <- flash_attn_varlen_func in the prefill branch of
 *                          nanovllm/layers/attention.py:64-70 (causal, no prefix cache)
 *   nv4_paged_decode_attention <- flash_attn_with_kvcache in the decode branch of
 *                          nanovllm/layers/attention.py:72-74 (caller of the hot path)
 *   nv4_rmsnorm         <- RMSNorm.rms_forward / add_rms_forward,
 *                          nanovllm/layers/layernorm.py:16-50 (caller of the hot path)
 *   nv4_qk_norm_rope_store <- q_norm/k_norm + rotary_emb in Qwen3Attention.forward,
 *                          nanovllm/models/qwen3.py:78-94, with
 *                          nanovllm/layers/rotary_embedding.py:6-48 and store_kvcache,
 *                          nanovllm/layers/attention.py:10-40 (caller of the hot path)
 *   nv4_silu_mul        <- SiluAndMul.forward, nanovllm/layers/activation.py:8-11
 *                          (caller of the hot path)
 *   nv4_gumbel_sample, nv4_gumbel_sample_ws <- Sampler.forward, nanovllm/layers/sampler.py:5-12
 *                          (caller of the hot path); nv4_philox4x32_10 is its
 *                          generator on the host, for known-answer tests
 *   nv4_rmsnorm_rht_quant_pack, nv4_silu_mul_rht_quant_pack <- the producer of
 *                          W4A4Linear's input fused into rht_quant_pack:
 *                          add+RMSNorm (layernorm.py:28-40) before the qkv and
 *                          gate_up projections, SiluAndMul (activation.py:8-11)
 *                          before down (nanovllm/models/qwen3.py:96-135 with
 *                          nanovllm/layers/linear_w4a4.py:30-34)
 *   nv4_rht_quant_pack_rowtiled, nv4_rmsnorm_rht_quant_pack_rowtiled,
 *   nv4_silu_mul_rht_quant_pack_rowtiled, nv4_w4a4_gemm_rowtiled,
 *   nv4_w4a4_linear_rowtiled <- the same operators for decode-sized M with the
 *                          packed activations in a row-tiled order (no
 *                          counterpart in the reference, whose kernels pass
 *                          [M,K/2] from rht_quant_pack to w4a4_grouped_gemm)
 *   nv4_w4a4_gemm_rowtiled_silu <- the gate_up W4A4Linear followed by
 *                          SiluAndMul (nanovllm/models/qwen3.py:125-129,
 *                          nanovllm/layers/activation.py:8-11) in one launch, for
 *                          decode-sized M (no counterpart call in the reference)
 *   nv4_lm_head         <- F.linear of ParallelLMHead.forward,
 *                          nanovllm/layers/embed_head.py:56-61 (decode-sized M; caller of
 *                          the hot path)
 *   nv4_paged_decode_attention_qkv <- the decode step's q_norm/k_norm +
 *                          rotary_emb + store_kvcache + flash_attn_with_kvcache
 *                          (nanovllm/models/qwen3.py:78-94,
 *                          nanovllm/layers/attention.py:10-40, 72-74) in one call
 *                          (no counterpart call in the reference)
 */
#ifndef NV4_H
#define NV4_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NV4_OK 0
#define NV4_E_NULL (-1)      /* a required pointer is NULL */
#define NV4_E_SHAPE (-2)     /* M/N/K outside what the contract allows */
#define NV4_E_ALIGN (-3)     /* a pointer is not aligned as documented */
#define NV4_E_LAYOUT (-4)    /* unknown rotation layout */
#define NV4_E_DTYPE (-5)     /* unknown dtype code */
#define NV4_E_GROUP (-6)     /* unsupported quantization group size */
#define NV4_E_SCRATCH (-7)   /* needs more device scratch than the allocation-free entry point has */

/* Rotation layouts for nv4_rht_quant_pack. */
#define NV4_LAYOUT_REFERENCE 0 /* "row_DH_paley12_kron_sylvester_v1": full-width
                                  Sylvester H4096, or H12 (Paley) x H1024 for K=12288 */
#define NV4_LAYOUT_BLOCK128 1  /* Hadamard-128 on every aligned 128-block, x RN(1/sqrt 128)
                                  (no reference counterpart) */

/* dtype codes */
#define NV4_BF16 0
#define NV4_FP16 1
#define NV4_FP32 2

/*
 * Fused randomized Hadamard transform + group-128 INT4 quantization + packing.
 * Replaces rht_quant_pack (nanovllm/kernels/rht_a4_tilelang.py:150-163).
 *   x      bf16 [M,K] row-major, 16-byte aligned
 *   signs  int8 [K], values +/-1, 16-byte aligned
 *   packed int8 [M,K/2] out: two's-complement nibbles, even k in the low nibble
 *   scale  bf16 [M,K/128] out: BF16(max|r|*0.9/7) rounded before the codes
 *          (1.0 for an all-zero group, at least 2^-126)
 * layout NV4_LAYOUT_REFERENCE requires K in {4096, 12288};
 * NV4_LAYOUT_BLOCK128 accepts any K that is a positive multiple of 128 up to 65536.
 * M >= 1.
 */
int nv4_rht_quant_pack(const void* x, const int8_t* signs, int8_t* packed, void* scale,
                       int64_t M, int64_t K, int layout, void* stream);

/*
 * Grouped W4A4 GEMM: C[M,N] = sum over 128-groups g (in order) of
 * fmaf(float(dot_g), sa[m,g]*sw[n,g], total), rounded to bf16 at the end.
 * Replaces w4a4_grouped_gemm / compile_grouped_gemm
 * (nanovllm/kernels/w4a4_grouped_kernel.py:32,104-129).
 *   a   int8 [M,K/2] packed activation codes (16-byte aligned)
 *   w   int8 [N,K/2] packed weight codes (16-byte aligned)
 *   sa  bf16 [M,K/128]
 *   sw  bf16 [N,K/128] when sw_grouped != 0 (production), else bf16 [N]
 *       (per-channel: total = sum fmaf(float(dot_g), sa[m,g], total); C = bf16(total*sw[n]))
 *   out bf16 [M,N], or fp32 [M,N] (the value before the final rounding) when out_fp32 != 0
 * M >= 1, N >= 1 with N % 8 == 0, K >= 128 with K % 128 == 0.
 */
int nv4_w4a4_gemm(const int8_t* a, const int8_t* w, const void* sa, const void* sw,
                  int sw_grouped, void* out, int out_fp32,
                  int64_t M, int64_t N, int64_t K, void* stream);

/*
 * W4A4 linear forward: RHT + quantize + pack the activations, then the
 * grouped INT4 GEMM -- the body of W4A4Linear.forward
 * (nanovllm/layers/linear_w4a4.py:27-35: rht_quant_pack then
 * w4a4_grouped_gemm), launched back to back on `stream`; identical to
 * calling nv4_rht_quant_pack (reference layout) and nv4_w4a4_gemm (grouped
 * scales, bf16 output) in sequence, with the same argument rules.
 *   x        bf16 [M,K], K in {4096, 12288}
 *   signs    int8 [K]
 *   w, sw    packed weights int8 [N,K/2] and bf16 scales [N,K/128]
 *   out      bf16 [M,N]
 *   a_packed int8 [M,K/2], a_scale bf16 [M,K/128]: receive the quantized
 *            activations (caller-owned workspace, also an output)
 */
int nv4_w4a4_linear(const void* x, const int8_t* signs, const int8_t* w, const void* sw,
                    void* out, int8_t* a_packed, void* a_scale,
                    int64_t M, int64_t N, int64_t K, void* stream);

/*
 * MFMA-tiled packed weights.  The same N*K/2 bytes as [N,K/2], reordered so
 * that the 16 columns x 128 k of one column block and K group are 1 KiB of
 * consecutive memory in the order the matrix-core lanes consume them:
 *   16-byte unit u = (cb*(K/128) + g)*64 + l  holds packed bytes
 *   64*g + 16*(l/16) .. +15 of column 16*cb + l%16          (l = 0..63).
 * Decode-sized GEMMs then load whole cache lines instead of half lines.
 * N % 16 == 0, K % 128 == 0; both buffers 16-byte aligned and not overlapping.
 */
int nv4_w4a4_tile_weights(const int8_t* w, int8_t* w_tiled, int64_t N, int64_t K, void* stream);
int nv4_w4a4_untile_weights(const int8_t* w_tiled, int8_t* w, int64_t N, int64_t K, void* stream);

/*
 * nv4_w4a4_gemm / nv4_w4a4_linear on MFMA-tiled weights (N % 16 == 0 as well);
 * results are bit-identical to the reference-layout calls on the untiled
 * weights.
 */
int nv4_w4a4_gemm_tiled(const int8_t* a, const int8_t* w_tiled, const void* sa, const void* sw,
                        int sw_grouped, void* out, int out_fp32,
                        int64_t M, int64_t N, int64_t K, void* stream);
int nv4_w4a4_linear_tiled(const void* x, const int8_t* signs, const int8_t* w_tiled, const void* sw,
                          void* out, int8_t* a_packed, void* a_scale,
                          int64_t M, int64_t N, int64_t K, void* stream);

/*
 * Row-tiled packed activations: the packed codes of M rows in 16-row blocks,
 * ceil(M/16) * 16 * K/2 bytes (rows past M in the last block are never
 * written and never change a result).  The 16 rows x 128 k of row block rb
 * and K group g are the 1 KiB at byte (rb*(K/128) + g) * 1024, in the order
 * the matrix-core lanes consume them:
 *   16-byte unit  (rb*(K/128) + g)*64 + l  holds packed bytes
 *   64*g + 16*(l/16) .. +15 of row 16*rb + l%16             (l = 0..63),
 * the activation counterpart of the tiled weight layout.  The decode GEMM then
 * loads every operand as whole cache lines straight into registers.
 * nv4_rht_quant_pack_rowtiled: nv4_rht_quant_pack (reference layout, K in
 *   {4096, 12288}) writing packed_rt in this order; scale stays [M,K/128].
 *   prefetch / prefetch_bytes (NULL / 0 for none; else a 16-byte aligned
 *   buffer and a positive multiple of 16 bytes): workgroups beyond the M rows
 *   of the launch read that many bytes of the buffer and discard them -- at
 *   decode sizes K1 occupies few CUs, so the weights of the GEMM that follows
 *   are read from HBM into the Infinity Cache meanwhile.  Nothing is written
 *   and no result changes.
 * nv4_w4a4_gemm_rowtiled: nv4_w4a4_gemm_tiled for 1 <= M <= 32 on row-tiled
 *   activations (a_rt 16-byte aligned); bit-identical results.
 * nv4_w4a4_linear_rowtiled: nv4_w4a4_linear_tiled for 1 <= M <= 32 with the
 *   row-tiled activation workspace a_packed_rt; its K1 prefetches the first
 *   nv4_w4a4_prefetch_bytes(N, K) bytes of w_tiled.
 * nv4_w4a4_prefetch_bytes: how many bytes of an [N,K] layer's packed weights
 *   a decode-sized K1 reads ahead of the GEMM (0 for invalid shapes).
 */
int nv4_rht_quant_pack_rowtiled(const void* x, const int8_t* signs, int8_t* packed_rt, void* scale,
                                int64_t M, int64_t K, const void* prefetch, int64_t prefetch_bytes, void* stream);
int nv4_w4a4_gemm_rowtiled(const int8_t* a_rt, const int8_t* w_tiled, const void* sa, const void* sw,
                           int sw_grouped, void* out, int out_fp32,
                           int64_t M, int64_t N, int64_t K, void* stream);

/*
 * SiLU-and-mul of a fused gate/up projection on row-tiled activations, in
 * one launch.  w_tiled is the MFMA-tiled weight of N = 2I rows, the gate
 * projection's I rows first, then the up projection's (the reference's
 * merged layout, nanovllm/layers/linear.py:87-93, shard 0 = gate), sw its
 * [N] or [N, K/128] scales.
 * out bf16 [M, I] = bf16(bf16(g / (1 + expf(-g))) * u), g and u the bf16
 * results nv4_w4a4_gemm_rowtiled would store for the paired columns n and
 * I + n: the bits of that GEMM followed by SiLU-and-mul
 * (nanovllm/layers/activation.py:8-11), without the [M, N] round trip.
 * Serves the wide decode kernel's sizes only: 1 <= M <= 32, N % 32 == 0,
 * K % 256 == 0, 4..8 column blocks of 16 per CU, M x K activations and the
 * scales within the kernel's LDS; other sizes return NV4_E_SHAPE (run
 * nv4_w4a4_gemm_rowtiled and nv4_silu_mul_rht_quant_pack_rowtiled instead).
 * No counterpart call in the reference (which runs the GEMM and the
 * activation as two ops); it replaces that pair for decode-sized batches.
 */
int nv4_w4a4_gemm_rowtiled_silu(const int8_t* a_rt, const int8_t* w_tiled, const void* a_scale,
                                const void* w_scale, int w_scale_grouped, void* out, int64_t M, int64_t N,
                                int64_t K, void* stream);
int nv4_w4a4_linear_rowtiled(const void* x, const int8_t* signs, const int8_t* w_tiled, const void* sw,
                             void* out, int8_t* a_packed_rt, void* a_scale,
                             int64_t M, int64_t N, int64_t K, void* stream);
int64_t nv4_w4a4_prefetch_bytes(int64_t N, int64_t K);

/*
 * nv4_w4a4_gemm (w_tiled = 0) / nv4_w4a4_gemm_tiled (w_tiled = 1) for
 * prefill-sized M on the fp8 matrix cores: the INT4 codes of both operands
 * are first written as fp8 (e4m3) bytes, one per code, into the caller's
 * workspace (A [M,K] then W [N,K]; workspace_bytes >= (M + N) * K, 16-byte
 * aligned), then multiplied with v_mfma_f32_32x32x64_f8f6f4.  Every group dot
 * is a small integer, exact in fp32, so the results are bit-identical to
 * nv4_w4a4_gemm.  Same argument rules as nv4_w4a4_gemm, and (M + N)·K/32
 * below 2^32; the workspace is overwritten, and calls sharing one workspace
 * must be stream-ordered.
 */
int nv4_w4a4_gemm_f8(const int8_t* a, const int8_t* w, int w_tiled, const void* sa, const void* sw,
                     int sw_grouped, void* out, int out_fp32, int64_t M, int64_t N, int64_t K,
                     void* workspace, int64_t workspace_bytes, void* stream);

/*
 * The same operator on the fp6 matrix cores: the INT4 codes of both operands
 * are first written as fp6 (e3m2) codes -- every integer of [-8, 8] is exact
 * in e3m2 -- into the caller's workspace, in 128-row tiles of 12 KiB per
 * 128-deep group (nv4_w4a4_gemm_f6_workspace(M, N, K) bytes, 16-byte
 * aligned), then multiplied with v_mfma_scale_f32_32x32x64_f8f6f4 in its
 * 6-bit form.  Every group dot is a small integer, exact in fp32, so the
 * results are bit-identical to nv4_w4a4_gemm.  Same argument rules as
 * nv4_w4a4_gemm_f8; the workspace is overwritten, and calls sharing one
 * workspace must be stream-ordered.  nv4_w4a4_gemm_f6_workspace returns -1
 * for shapes the operator rejects (M, N < 1; K not a positive multiple of 128).
 *   w_form  0: w is packed int8 [N,K/2]; 1: MFMA-tiled (N % 16 == 0);
 *           2: w is the fp6 tile form written by nv4_w4a4_weights_to_f6 for
 *              this N and K -- only A is converted, and the workspace needs
 *              only its A part, ceil(M/128) * (K/128) * 12288 bytes.
 */
int nv4_w4a4_gemm_f6(const int8_t* a, const int8_t* w, int w_form, const void* sa, const void* sw,
                     int sw_grouped, void* out, int out_fp32, int64_t M, int64_t N, int64_t K,
                     void* workspace, int64_t workspace_bytes, void* stream);
int64_t nv4_w4a4_gemm_f6_workspace(int64_t M, int64_t N, int64_t K);

/*
 * Weights converted once for nv4_w4a4_gemm_f6 (w_form 2): packed int8
 * [N,K/2] (w_tiled 0) or MFMA-tiled (w_tiled 1, N % 16 == 0) -> w6, the
 * e3m2 tile blocks the per-call conversion would write for W
 * (nv4_w4a4_weights_f6_bytes(N, K) = ceil(N/128) * (K/128) * 12288 bytes;
 * -1 for N < 1 or K not a positive multiple of 128).  Same shape and
 * alignment rules as nv4_w4a4_gemm_f6; w6 must not overlap w.  A layer keeps
 * w6 for as long as its weights do, so prefill calls convert activations only.
 */
int nv4_w4a4_weights_to_f6(const int8_t* w, int w_tiled, uint8_t* w6, int64_t N, int64_t K,
                           int64_t w6_bytes, void* stream);
int64_t nv4_w4a4_weights_f6_bytes(int64_t N, int64_t K);

/*
 * W4A16 GEMM with GPTQ weights (zero-point convention w = (q - z - 1) * s).
 * Replaces tl_dequant_matmul_w4a16 (nanovllm/layers/linear_w4a16.py:11-59).
 *   x        [M,K] activations, x_dtype NV4_BF16 (reference) or NV4_FP16
 *   qweight  int32 [K/8,N]: nibble k%8 (bits 4*(k%8)) of row k/8 holds q[k,n]
 *   qzeros   int32 [K/group,N/8]: nibble n%8 of [g, n/8] holds z[g,n]
 *   scales   fp16 [K/group,N]
 *   out      [M,N] out, out_dtype NV4_BF16 (reference) or NV4_FP16
 * Dequantization: bf16 activations use deq = bf16(bf16(q-z-1) * bf16(s)) as the
 * reference does; fp16 activations use deq = fp16((q-z-1) * s).  Products are
 * accumulated in fp32 over the whole K (deterministic; no split-K atomics).
 * Decode sizes -- M <= 16 (any K), or M <= 32 with K <= 4096 and
 * ceil(N/32) <= the CU count; K*N/2 < 2^31; qweight 8-byte and scales 4-byte
 * aligned -- run one launch (32 columns per workgroup over the whole K, no
 * workspace) that applies the (bf16-rounded) scale per group to exact sums of
 * biased codes, sum x (q-z-1) s = s (S - (bias+z+1) X), without rounding each
 * dequantized weight: a difference far inside the 1e-2 relative tolerance of
 * the reference's own split-K product.
 * group == 128; K % 128 == 0; N % 8 == 0; M >= 1.  x and out 16-byte aligned.
 */
int nv4_w4a16_gemm(const void* x, int x_dtype, const int32_t* qweight, const int32_t* qzeros,
                   const void* scales, void* out, int out_dtype,
                   int64_t M, int64_t N, int64_t K, int group, void* stream);

/*
 * nv4_w4a16_gemm with a caller-provided fp32 workspace, for decode sizes
 * (M <= 64; larger M runs nv4_w4a16_gemm and ignores the workspace): K is
 * split into 1024-deep slices, each written as an fp32 partial [S, M, N]
 * (S = ceil(K/1024)) and then added in slice order and rounded once, so the
 * result is deterministic (not bit-identical to nv4_w4a16_gemm, whose
 * summation order differs).  workspace_bytes >= S*M*N*4, 16-byte aligned;
 * qweight and x 16-byte aligned, scales and out 8-byte aligned.
 */
int nv4_w4a16_gemm_ws(const void* x, int x_dtype, const int32_t* qweight, const int32_t* qzeros,
                      const void* scales, void* out, int out_dtype, float* workspace, int64_t workspace_bytes,
                      int64_t M, int64_t N, int64_t K, int group, void* stream);

/*
 * Dense dequantization of a GPTQ weight, for prefill-sized M where the
 * product then runs as a library GEMM x[M,K] @ w[K,N]:
 *   w[k][n] = cvt(float(q[k][n] - z[k/128][n] - 1) * s),   w row-major [K, N],
 * with the rounding of nv4_w4a16_gemm: bf16 (w_dtype NV4_BF16) takes the
 * scale rounded to bf16 first, fp16 takes it as is.  qweight, scales and w
 * 16-byte aligned; N % 8 == 0, K % 128 == 0, group 128.
 */
int nv4_w4a16_dequant(const int32_t* qweight, const int32_t* qzeros, const void* scales, void* w, int w_dtype,
                      int64_t N, int64_t K, int group, void* stream);

/*
 * Prefill attention: causal GQA attention over packed sequences.
 * Replaces flash_attn_varlen_func(q, k, v, cu_seqlens_q=cu_seqlens_k=cu_seqlens,
 * softmax_scale, causal=True) in nanovllm/layers/attention.py:64-70 (without a
 * prefix cache: queries and keys are the same rows).
 *   q            bf16 [T, Hq, 128]: rows q_row elements apart (>= Hq*128)
 *   k, v         bf16 [T, Hkv, 128]: rows k_row / v_row elements apart (>= Hkv*128)
 *   out          bf16 [T, Hq, 128]: rows o_row elements apart (>= Hq*128)
 *   cu_seqlens   int32 [B+1]: sequence b is rows cu_seqlens[b] .. cu_seqlens[b+1]-1,
 *                each at most max_seqlen long (longer ones are not fully written)
 * o[i] = softmax_{j <= i}(scale * q[i].k[j]) v[j] per sequence and query head;
 * KV head of query head h: h / (Hq/Hkv), Hq/Hkv in {1, 2, 4, 8}; fp32
 * arithmetic, P rounded to bf16 for the P.V product.  Row strides multiples
 * of 8 elements, tensors 16-byte aligned; scale > 0; B <= 65535.
 */
int nv4_prefill_attention(const void* q, int64_t q_row, const void* k, int64_t k_row, const void* v, int64_t v_row,
                          void* out, int64_t o_row, const int32_t* cu_seqlens, int64_t B, int64_t max_seqlen,
                          int64_t Hq, int64_t Hkv, int64_t D, float scale, void* stream);

/*
 * Paged decode attention (one new token per sequence; GQA).
 * Replaces flash_attn_with_kvcache(q, k_cache, v_cache, cache_seqlens, block_table,
 * softmax_scale, causal=True) in nanovllm/layers/attention.py:72-74.
 *   q             bf16 [B, Hq, 128]: rows q_row_stride elements apart (>= Hq*128, multiple of 8)
 *   k/v_cache     bf16 [num_blocks, block_size, Hkv, 128]
 *   block_tables  int32 [B, max_blocks]: the first ceil(context_lens[b]/block_size)
 *                 entries of row b are valid block indices
 *   context_lens  int32 [B], context_lens[b] <= max_context; a row with
 *                 context_lens[b] <= 0 (empty context) gets an output of zeros
 *   out           bf16 [B, Hq, 128] (contiguous)
 *   workspace     fp32 scratch of at least B*Hq*S*(128+2)*4 bytes, S = ceil(max_context/256)
 * Hq / Hkv in {1, 2, 4}; softmax(scale * q.K^T) V with fp32 arithmetic.
 */
int nv4_paged_decode_attention(const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache,
                               const int32_t* block_tables, int64_t max_blocks, const int32_t* context_lens,
                               void* out, float* workspace, int64_t workspace_bytes, int64_t B, int64_t Hq,
                               int64_t Hkv, int64_t D, int64_t block_size, int64_t max_context, float scale,
                               void* stream);

/*
 * nv4_paged_decode_attention without a workspace argument.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP-graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The split partials go to a device array of the library,
 * NV4_PA_SCRATCH_BYTES (16 MiB) per GPU, held from the first call on that GPU
 * until the process ends; nothing is allocated or freed by the call.  A call
 * needing more than that (B*Hq*S*(128+2)*4 bytes with S =
 * ceil(max_context/256) > 1) returns NV4_E_SCRATCH before launching anything.
 * Every call on one GPU shares that GPU's array: calls that overlap in time on
 * one GPU (different streams without ordering between them) race on it and
 * must not be issued.  Same arguments, rules and results (bit for bit) as
 * nv4_paged_decode_attention.  The first call on a device looks up the array's
 * address (hipGetSymbolAddress) with that device current; make it outside
 * graph capture.
 */
#define NV4_PA_SCRATCH_BYTES (16ll << 20)
int nv4_paged_decode_attention_noalloc(const void* q, int64_t q_row_stride, const void* k_cache,
                                       const void* v_cache, const int32_t* block_tables, int64_t max_blocks,
                                       const int32_t* context_lens, void* out, int64_t B, int64_t Hq, int64_t Hkv,
                                       int64_t D, int64_t block_size, int64_t max_context, float scale,
                                       void* stream);

/*
 * The decode step's nv4_qk_norm_rope_store (one token per sequence, T = B)
 * fused into nv4_paged_decode_attention: one launch less per layer, the same
 * bits in out, k_cache and v_cache as the two calls in sequence (the second
 * with q = the first's q_out).  Replaces, in the decode branch, q_norm/k_norm +
 * rotary_emb (nanovllm/models/qwen3.py:78-94, layers/rotary_embedding.py:6-48),
 * store_kvcache (layers/attention.py:10-40) and flash_attn_with_kvcache
 * (layers/attention.py:72-74).
 *   qkv, qkv_row_stride, q/k_norm_w, cos_sin, max_position, positions,
 *   slot_mapping, num_slots: as nv4_qk_norm_rope_store, with T = B
 *   k/v_cache, block_tables, context_lens, out, workspace, max_context, scale:
 *   as nv4_paged_decode_attention (q = the query heads of qkv)
 * The workgroup that reads a sequence's last context token stores the step's
 * key and value and uses them from registers for that token.  Precondition
 * (the engine's): a step's slots are not in any other sequence's context.
 */
int nv4_paged_decode_attention_qkv(const void* qkv, int64_t qkv_row_stride, const void* q_norm_w,
                                   const void* k_norm_w, const float* cos_sin, int64_t max_position,
                                   const int64_t* positions, const int32_t* slot_mapping, int64_t num_slots,
                                   void* k_cache, void* v_cache, const int32_t* block_tables, int64_t max_blocks,
                                   const int32_t* context_lens, void* out, float* workspace, int64_t workspace_bytes,
                                   int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t block_size,
                                   int64_t max_context, float eps, float scale, void* stream);

/*
 * RMSNorm over rows of H bf16 values (nanovllm/layers/layernorm.py:16-50):
 *   residual_in == NULL:  y = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * weight)
 *   residual_in != NULL:  h = float(x) + float(residual_in); residual_out = bf16(h);
 *                         y = bf16(bf16(h * rsqrt(mean(h^2) + eps)) * weight)
 * x, residual_in, residual_out, y: [rows, H] contiguous, 16-byte aligned; weight [H].
 * residual_in and residual_out are both NULL or both set (they may alias;
 * x and y may alias).  16 <= H <= 8192, H % 16 == 0.  The sum of squares is
 * taken in one fixed order, shared with nv4_rmsnorm_rht_quant_pack.
 */
int nv4_rmsnorm(const void* x, const void* residual_in, void* residual_out, const void* weight, void* y,
                int64_t rows, int64_t H, float eps, void* stream);

/*
 * Per-head q/k RMSNorm, rotary embedding and KV-cache store for T tokens of a
 * fused qkv projection (nanovllm/models/qwen3.py:78-94,
 * nanovllm/layers/rotary_embedding.py:6-48, nanovllm/layers/attention.py:10-40).
 *   qkv          bf16 [T, row]: Hq query heads, Hkv key heads, Hkv value heads of 128
 *                (row = qkv_row_stride >= (Hq + 2*Hkv)*128)
 *   q/k_norm_w   bf16 [128]
 *   cos_sin      fp32 [max_position, 128]: cos in columns 0..63, sin in 64..127
 *   positions    int64 [T]; slot_mapping int32 [T]
 *   q_out        bf16 [T, Hq, 128]: normalised, rotated queries
 *   k/v_cache    bf16 [num_slots, Hkv, 128] (= [num_blocks, block_size, Hkv, 128]):
 *                token t's rotated key and its value go to slot slot_mapping[t];
 *                slots outside [0, num_slots) (the reference's -1) are not stored
 *   k_out/v_out  optional bf16 [T, Hkv, 128] copies of the rotated keys / values
 * Positions outside [0, max_position) read row 0 of the table.  qkv_row_stride
 * a multiple of 4; bf16 tensors 8-byte and cos_sin 16-byte aligned.
 */
int nv4_qk_norm_rope_store(const void* qkv, int64_t qkv_row_stride, int64_t T, int64_t Hq, int64_t Hkv,
                           const void* q_norm_w, const void* k_norm_w, const float* cos_sin, int64_t max_position,
                           const int64_t* positions, const int32_t* slot_mapping, int64_t num_slots, void* q_out,
                           void* k_cache, void* v_cache, void* k_out, void* v_out, float eps, void* stream);

/*
 * LM head for decode-sized batches: out[M, N] = bf16(h[M, K] . w[N, K]^T), fp32
 * sums (replaces ParallelLMHead.forward's F.linear, nanovllm/layers/embed_head.py:56-61,
 * for M <= 32 rows).  h bf16 rows h_row_stride elements apart (a multiple of 8),
 * w bf16 [N, K] contiguous, out bf16 rows out_row_stride apart; h and w 16-byte
 * aligned.  1 <= M <= 32, K in {2048, 4096, 5120}, 1 <= N <= 2^30.  The sum
 * order is fixed (four K-quarters added in order), so results repeat bit for
 * bit; they may differ from another library's GEMM in the last bits.
 */
int nv4_lm_head(const void* h, int64_t h_row_stride, const void* w, void* out, int64_t out_row_stride, int64_t M,
                int64_t N, int64_t K, void* stream);

/*
 * SiLU-and-mul (nanovllm/layers/activation.py:8-11): gate_up bf16 [rows, 2*I]
 * (gate in columns 0..I-1, up in I..2I-1) -> y bf16 [rows, I],
 * y = bf16(bf16(g / (1 + exp(-g))) * u).  I % 8 == 0; 16-byte aligned.
 */
int nv4_silu_mul(const void* gate_up, void* y, int64_t rows, int64_t I, void* stream);

/*
 * Fused prologue + K1: the RMSNorm (or SiLU-mul) output is computed, rounded
 * to bf16 exactly as nv4_rmsnorm (nv4_silu_mul) stores it, and quantized as
 * nv4_rht_quant_pack (reference layout) would quantize that stored tensor,
 * without writing it: packed codes and scales are bit-identical to the
 * two-step sequence.
 * nv4_rmsnorm_rht_quant_pack: x bf16 [M,4096]; residual_in/residual_out as
 *   nv4_rmsnorm (both NULL, or both set; they may alias); norm_weight bf16
 *   [4096]; K == 4096.
 * nv4_silu_mul_rht_quant_pack: gate_up bf16 [M,2K] (gate in columns 0..K-1,
 *   up in K..2K-1); K in {4096, 12288}.
 * signs int8 [K]; packed int8 [M,K/2]; scale bf16 [M,K/128]; alignments as
 * nv4_rht_quant_pack (activations 16 bytes).
 */
int nv4_rmsnorm_rht_quant_pack(const void* x, const void* residual_in, void* residual_out, const void* norm_weight,
                               float eps, const int8_t* signs, int8_t* packed, void* scale, int64_t M, int64_t K,
                               void* stream);
int nv4_silu_mul_rht_quant_pack(const void* gate_up, const int8_t* signs, int8_t* packed, void* scale, int64_t M,
                                int64_t K, void* stream);
/* The same two, writing the codes in the row-tiled order (ceil(M/16)*16*K/2 bytes), with the
 * prefetch arguments of nv4_rht_quant_pack_rowtiled. */
int nv4_rmsnorm_rht_quant_pack_rowtiled(const void* x, const void* residual_in, void* residual_out,
                                        const void* norm_weight, float eps, const int8_t* signs, int8_t* packed_rt,
                                        void* scale, int64_t M, int64_t K, const void* prefetch,
                                        int64_t prefetch_bytes, void* stream);
int nv4_silu_mul_rht_quant_pack_rowtiled(const void* gate_up, const int8_t* signs, int8_t* packed_rt, void* scale,
                                         int64_t M, int64_t K, const void* prefetch, int64_t prefetch_bytes,
                                         void* stream);

/*
 * Next-token sampling at per-row temperatures (nanovllm/layers/sampler.py:5-12):
 * out[b] = argmax_v  l[b,v] / T[b] - log(max(E, 1e-10)),  E = -log U,
 * which has the distribution of the reference's argmax(softmax(l/T) / E).
 * U = ((w >> 8) + 0.5) * 2^-24 for word w = v % 4 of the Philox4x32-10 block
 * with key (seed low, seed high) and counter (v / 4, b, offset low,
 * offset high).  Ties go to the smallest index.
 *   logits  [B, V] rows row_stride elements apart (>= V); logits_dtype NV4_BF16
 *           or NV4_FP32 (element-aligned)
 *   temperatures fp32 [B] (> 0); out int64 [B]
 */
int nv4_gumbel_sample(const void* logits, int64_t row_stride, int logits_dtype, const float* temperatures,
                      int64_t B, int64_t V, uint64_t seed, uint64_t offset, int64_t* out, void* stream);

/*
 * nv4_gumbel_sample split over P = nv4_gumbel_sample_chunks(B, V) workgroups
 * per row (quad-aligned column chunks) plus a merge launch; returns the same
 * token ids.  workspace: at least 8*B*P bytes, 4-byte aligned; B <= 65535.
 */
int64_t nv4_gumbel_sample_chunks(int64_t B, int64_t V);
int nv4_gumbel_sample_ws(const void* logits, int64_t row_stride, int logits_dtype, const float* temperatures,
                         int64_t B, int64_t V, uint64_t seed, uint64_t offset, void* workspace,
                         int64_t workspace_bytes, int64_t* out, void* stream);

/* Philox4x32-10 of one counter block, computed on the host: out = philox(counter[4], key[2]). */
void nv4_philox4x32_10(const uint32_t* counter, const uint32_t* key, uint32_t* out);

/* Library version string. */
/*
 * Measurement probes (no counterpart in the reference; bench.py reports
 * their rates beside the published peaks).
 *   nv4_probe_mfma: `workgroups` workgroups of 4 waves, each wave running
 *     `iters` (rounded up to even) rounds of four independent matrix-core
 *     products: kind 0 = v_mfma_i32_16x16x64_i8 (32768 ops each), kind 1 =
 *     v_mfma_scale_f32_32x32x64_f8f6f4 on fp8 operands, kind 2 = the same on
 *     fp6 (e3m2) operands (131072 ops each).  `sink` is an int
 *     array of at least max(workgroups, 1024) entries (written only on a
 *     value the products practically never take).  1 <= iters <= 2^30,
 *     1 <= workgroups <= 2^20.
 *   nv4_probe_read: reads `bytes` (a multiple of 65536, 16-byte aligned
 *     buffer) once with 16-byte nontemporal loads; same sink rule.
 */
int nv4_probe_mfma(int kind, int64_t iters, int64_t workgroups, int* sink, void* stream);
int nv4_probe_read(const void* buf, int64_t bytes, int* sink, void* stream);
/*
 * nv4_probe_bf16_rne: adds to *mismatches (a device counter the caller
 * zeroes) the number of non-NaN fp32 inputs, out of all 2^32, whose bf16
 * conversion by the kernels (the hardware instruction) differs from integer
 * round-to-nearest-even.  No counterpart in the reference; it pins the
 * rounding every bf16 output and intermediate of this library relies on.
 */
int nv4_probe_bf16_rne(unsigned long long* mismatches, void* stream);

const char* nv4_version(void);

/* Human-readable text for an NV4_E* code (or "hip error" for positive codes). */
const char* nv4_strerror(int code);

#ifdef __cplusplus
}
#endif

#endif /* NV4_H */
