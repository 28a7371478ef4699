"""Fused decoder elementwise operators around the quantized linears (MI355X).

Each is one HIP launch on torch's current stream (graph-capturable), with the
rounding points of the reference's PyTorch formulation:

* ``rmsnorm`` -- RMSNorm.rms_forward / add_rms_forward
  (nanovllm/layers/layernorm.py:16-50), the residual add fused;
* ``qk_norm_rope_store`` -- the per-head q/k RMSNorm, rotary embedding and KV
  store of Qwen3Attention.forward (nanovllm/models/qwen3.py:78-94,
  nanovllm/layers/rotary_embedding.py:6-48, nanovllm/layers/attention.py:10-40);
* ``silu_mul`` -- SiluAndMul (nanovllm/layers/activation.py:8-11);
* ``rmsnorm_rht_quant_pack`` / ``silu_mul_rht_quant_pack`` -- the same two
  producers fused in front of ``rht_quant_pack`` (the quantization of a
  W4A4Linear's input): codes and scales bit-identical to running the
  producer, then ``rht_quant_pack`` on its bf16 output, without writing
  that output.
"""
from __future__ import annotations

import ctypes

import torch

from .. import _lib
from .rht_a4 import prefetch_args


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _check_dev(tensors, dev):
    if any(t is not None and (not t.is_cuda or t.device != dev) for t in tensors):
        raise ValueError("All tensors must be on one CUDA device")


def rmsnorm(x, weight, eps, residual=None, out=None):
    """x bf16 [..., H] -> y (bf16, same shape); with ``residual`` returns
    (y, x + residual rounded to bf16) and writes the sum into ``residual``."""
    H = x.shape[-1]
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16 or tuple(weight.shape) != (H,):
        raise TypeError("RMSNorm expects BF16 activations and a BF16 weight [H]")
    if not x.is_contiguous() or not weight.is_contiguous():
        raise ValueError("RMSNorm expects contiguous tensors")
    if residual is not None and (residual.shape != x.shape or residual.dtype != x.dtype
                                 or not residual.is_contiguous()):
        raise ValueError("residual must match x")
    rows = x.numel() // H
    if out is None:
        out = torch.empty_like(x)
    _check_dev((x, weight, residual, out), x.device)
    lib = _lib.load()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    with torch.cuda.device(x.device):
        rc = lib.nv4_rmsnorm(_ptr(x), _ptr(residual), _ptr(residual), _ptr(weight), _ptr(out), rows, H,
                             ctypes.c_float(eps), ctypes.c_void_p(stream))
    _lib.check(rc, "rmsnorm")
    return out if residual is None else (out, residual)


def qk_norm_rope_store(qkv, num_heads, num_kv_heads, q_norm_w, k_norm_w, cos_sin, positions, eps,
                       slot_mapping=None, k_cache=None, v_cache=None, return_kv=False):
    """qkv bf16 [T, (Hq + 2 Hkv) * 128] (rows may be strided) -> q [T, Hq, 128]
    (and, with ``return_kv``, k [T, Hkv, 128], v [T, Hkv, 128]); rotated keys
    and values go to the cache slots ``slot_mapping`` when caches are given."""
    T = qkv.shape[0]
    D = 128
    if qkv.dtype != torch.bfloat16 or qkv.ndim != 2 or qkv.stride(1) != 1:
        raise TypeError("qkv must be BF16 [T, heads*128] with unit column stride")
    if qkv.shape[1] != (num_heads + 2 * num_kv_heads) * D:
        raise ValueError("qkv width does not match the head counts (head_dim 128)")
    if cos_sin.dtype != torch.float32 or cos_sin.shape[-1] != D or not cos_sin.is_contiguous():
        raise TypeError("cos_sin must be a contiguous FP32 [max_position, 128] table")
    if positions.dtype != torch.int64 or tuple(positions.shape) != (T,):
        raise TypeError("positions must be int64 [T]")
    for w in (q_norm_w, k_norm_w):
        if w.dtype != torch.bfloat16 or tuple(w.shape) != (D,) or not w.is_contiguous():
            raise TypeError("q/k norm weights must be contiguous BF16 [128]")
    max_position = cos_sin.numel() // D
    dev = qkv.device
    q = torch.empty((T, num_heads, D), dtype=torch.bfloat16, device=dev)
    k = v = None
    if return_kv:
        k = torch.empty((T, num_kv_heads, D), dtype=torch.bfloat16, device=dev)
        v = torch.empty((T, num_kv_heads, D), dtype=torch.bfloat16, device=dev)
    store = k_cache is not None and k_cache.numel() > 0
    if store:
        if (k_cache.dtype != torch.bfloat16 or v_cache.shape != k_cache.shape or k_cache.shape[-2:] != (
                num_kv_heads, D) or not k_cache.is_contiguous() or not v_cache.is_contiguous()):
            raise ValueError("caches must be contiguous BF16 [num_blocks, block_size, num_kv_heads, 128]")
        if slot_mapping is None or slot_mapping.dtype != torch.int32 or tuple(slot_mapping.shape) != (T,):
            raise TypeError("slot_mapping must be int32 [T]")
        num_slots = k_cache.numel() // (num_kv_heads * D)
    else:
        # No cache: the kernel stores nothing (num_slots 0); pointers are
        # placeholders that are never dereferenced.
        num_slots, k_cache, v_cache = 0, q, q
        slot_mapping = torch.empty((T,), dtype=torch.int32, device=dev) if slot_mapping is None else slot_mapping
    _check_dev((qkv, q_norm_w, k_norm_w, cos_sin, positions, slot_mapping, k_cache, v_cache), dev)
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    with torch.cuda.device(dev):
        rc = lib.nv4_qk_norm_rope_store(
            _ptr(qkv), qkv.stride(0), T, num_heads, num_kv_heads, _ptr(q_norm_w), _ptr(k_norm_w), _ptr(cos_sin),
            max_position, _ptr(positions), _ptr(slot_mapping), num_slots, _ptr(q), _ptr(k_cache), _ptr(v_cache),
            _ptr(k), _ptr(v), ctypes.c_float(eps), ctypes.c_void_p(stream))
    _lib.check(rc, "qk_norm_rope_store")
    return (q, k, v) if return_kv else q


LM_HEAD_MAX_ROWS = 32
LM_HEAD_K = (2048, 4096, 5120)


def lm_head_fits(h, weight) -> bool:
    """Whether ``lm_head`` takes this call (decode-sized rows, a supported
    hidden size, bf16, 16-byte aligned rows); otherwise use F.linear."""
    return (h.ndim == 2 and weight.ndim == 2 and 1 <= h.shape[0] <= LM_HEAD_MAX_ROWS and h.shape[1] in LM_HEAD_K
            and weight.shape[1] == h.shape[1] and h.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
            and h.stride(1) == 1 and h.stride(0) % 8 == 0 and weight.is_contiguous()
            and h.data_ptr() % 16 == 0 and weight.data_ptr() % 16 == 0 and h.is_cuda and h.device == weight.device)


def lm_head(h, weight, out=None):
    """logits = h @ weight^T (ParallelLMHead's F.linear,
    nanovllm/layers/embed_head.py:56-61) for M <= 32 rows: h bf16 [M, K],
    weight bf16 [N, K] -> bf16 [M, N], fp32 sums (``nv4_lm_head``)."""
    if not lm_head_fits(h, weight):
        raise ValueError("lm_head takes bf16 h [M <= 32, K in (2048, 4096, 5120)] and a contiguous weight [N, K]")
    M, K = h.shape
    N = weight.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=h.device)
    elif (out.dtype != torch.bfloat16 or tuple(out.shape) != (M, N) or out.stride(1) != 1
          or out.device != h.device):
        raise ValueError("out must be bf16 [M, N] with unit column stride on the device of h")
    lib = _lib.load()
    stream = torch.cuda.current_stream(h.device).cuda_stream
    with torch.cuda.device(h.device):
        rc = lib.nv4_lm_head(_ptr(h), h.stride(0), _ptr(weight), _ptr(out), out.stride(0), M, N, K,
                             ctypes.c_void_p(stream))
    _lib.check(rc, "lm_head")
    return out


def silu_mul(gate_up, out=None):
    """gate_up bf16 [..., 2I] -> bf16 [..., I] = silu(gate) * up."""
    I2 = gate_up.shape[-1]
    if gate_up.dtype != torch.bfloat16 or I2 % 16 or not gate_up.is_contiguous():
        raise ValueError("silu_mul expects contiguous BF16 [..., 2I] with I % 8 == 0")
    rows = gate_up.numel() // I2
    if out is None:
        out = torch.empty((*gate_up.shape[:-1], I2 // 2), dtype=torch.bfloat16, device=gate_up.device)
    _check_dev((gate_up, out), gate_up.device)
    lib = _lib.load()
    stream = torch.cuda.current_stream(gate_up.device).cuda_stream
    with torch.cuda.device(gate_up.device):
        rc = lib.nv4_silu_mul(_ptr(gate_up), _ptr(out), rows, I2 // 2, ctypes.c_void_p(stream))
    _lib.check(rc, "silu_mul")
    return out


def _k1_outputs(M, K, dev, out_packed, out_scale, rowtiled=False):
    rows = (M + 15) // 16 * 16 if rowtiled else M
    if out_packed is None:
        out_packed = torch.empty((rows, K // 2), dtype=torch.int8, device=dev)
    if out_scale is None:
        out_scale = torch.empty((M, K // 128), dtype=torch.bfloat16, device=dev)
    if (tuple(out_packed.shape) != (rows, K // 2) or out_packed.dtype != torch.int8 or not out_packed.is_contiguous()
            or tuple(out_scale.shape) != (M, K // 128) or out_scale.dtype != torch.bfloat16
            or not out_scale.is_contiguous()):
        raise ValueError("Outputs must be contiguous INT8 [M,K/2] and BF16 [M,K/128]")
    return out_packed, out_scale


def rmsnorm_rht_quant_pack(x, weight, eps, signs, residual=None, out_packed=None, out_scale=None, rowtiled=False,
                           prefetch=None):
    """x bf16 [M, 4096] -> (packed, scale) of rht_quant_pack(rmsnorm(x)); with
    ``residual`` the norm input is x + residual, whose bf16 rounding is written
    into ``residual`` and returned as a third element.  ``rowtiled``: the codes
    in the row-tiled order of ``rht_quant_pack_rowtiled`` ([ceil(M/16)*16, K/2],
    read by ``w4a4_gemm_rowtiled``), with its ``prefetch`` (the consuming
    GEMM's weights)."""
    if x.ndim != 2 or x.shape[1] != 4096 or x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise ValueError("Expected contiguous BF16 x[M,4096]")
    if weight.dtype != torch.bfloat16 or tuple(weight.shape) != (4096,) or signs.dtype != torch.int8 \
            or tuple(signs.shape) != (4096,):
        raise TypeError("Expected a BF16 norm weight [4096] and int8 signs [4096]")
    if residual is not None and (residual.shape != x.shape or residual.dtype != x.dtype
                                 or not residual.is_contiguous()):
        raise ValueError("residual must match x")
    M, K = x.shape
    dev = x.device
    out_packed, out_scale = _k1_outputs(M, K, dev, out_packed, out_scale, rowtiled)
    _check_dev((x, weight, signs, residual, out_packed, out_scale), dev)
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    extra = prefetch_args(prefetch) if rowtiled else ()
    if not rowtiled and prefetch is not None:
        raise ValueError("prefetch goes with rowtiled=True")
    fn = lib.nv4_rmsnorm_rht_quant_pack_rowtiled if rowtiled else lib.nv4_rmsnorm_rht_quant_pack
    with torch.cuda.device(dev):
        rc = fn(_ptr(x), _ptr(residual), _ptr(residual), _ptr(weight),
                ctypes.c_float(eps), _ptr(signs), _ptr(out_packed), _ptr(out_scale), M, K, *extra,
                ctypes.c_void_p(stream))
    _lib.check(rc, "rmsnorm_rht_quant_pack")
    return (out_packed, out_scale) if residual is None else (out_packed, out_scale, residual)


def silu_mul_rht_quant_pack(gate_up, signs, out_packed=None, out_scale=None, rowtiled=False, prefetch=None):
    """gate_up bf16 [M, 2K] (K = 4096 or 12288) -> (packed, scale) of
    rht_quant_pack(silu_mul(gate_up)); ``rowtiled`` as in
    ``rmsnorm_rht_quant_pack``."""
    if gate_up.ndim != 2 or gate_up.dtype != torch.bfloat16 or not gate_up.is_contiguous() \
            or gate_up.shape[1] not in (8192, 24576):
        raise ValueError("Expected contiguous BF16 gate_up[M,2K], K = 4096 or 12288")
    M, K = gate_up.shape[0], gate_up.shape[1] // 2
    if signs.dtype != torch.int8 or tuple(signs.shape) != (K,):
        raise TypeError("Expected int8 signs [K]")
    dev = gate_up.device
    out_packed, out_scale = _k1_outputs(M, K, dev, out_packed, out_scale, rowtiled)
    _check_dev((gate_up, signs, out_packed, out_scale), dev)
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    extra = prefetch_args(prefetch) if rowtiled else ()
    if not rowtiled and prefetch is not None:
        raise ValueError("prefetch goes with rowtiled=True")
    fn = lib.nv4_silu_mul_rht_quant_pack_rowtiled if rowtiled else lib.nv4_silu_mul_rht_quant_pack
    with torch.cuda.device(dev):
        rc = fn(_ptr(gate_up), _ptr(signs), _ptr(out_packed), _ptr(out_scale), M, K, *extra, ctypes.c_void_p(stream))
    _lib.check(rc, "silu_mul_rht_quant_pack")
    return out_packed, out_scale
