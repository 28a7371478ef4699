"""W4A16 GEMM with GPTQ-packed INT4 weights (MI355X).

Replaces the TileLang kernel ``tl_dequant_matmul_w4a16`` of the reference
(nanovllm/layers/linear_w4a16.py:11-59).  Same packed formats: qweight int32
[K/8, N] (nibble k%8 of row k/8), qzeros int32 [K/128, N/8] (nibble n%8),
fp16 scales [K/128, N]; same zero convention w = (q - z - 1) * s and, for bf16
activations, the same bf16 rounding of the dequantized weight.  Unlike the
reference (split-K 8 with bf16 atomics onto a zeroed output) the HIP kernel
sums all of K in fp32 and writes each output once, so results do not depend
on scheduling.  FP16 activations are accepted as well (output fp16).

Decode sizes: for M <= 16 (any K), and for M <= 32 when K <= 4096 and the
32-column workgroups are at most one per CU (the fused QKV and o_proj of an
8B model), ``nv4_w4a16_gemm`` runs one launch whose 16-wave workgroups own 32
columns over the whole K (each wave takes whole quantisation groups; the
waves' fp32 tiles are added in a fixed order in LDS); no workspace.  Other
M <= 64 (every workgroup of the one-launch form reads all M x K activations,
which at 17..32 rows costs more than splitting K when K is long or the
workgroups are several per CU) take the split-K form
(``nv4_w4a16_gemm_ws``): 64-column workgroups per 1024-deep K slice writing
fp32 partials into a workspace from torch's caching allocator, added in slice
order by a second launch.  Both are deterministic and graph-capturable.  At prefill sizes (M > 64) the weight is dequantized once
into a dense [K, N] tensor (``nv4_w4a16_dequant``, the same per-element
rounding) and the product runs as a library GEMM (torch.mm on hipBLASLt,
fp32 accumulation).
"""
from __future__ import annotations

import ctypes

import torch

from .. import _lib

_DT = {torch.bfloat16: _lib.BF16, torch.float16: _lib.FP16}
SLICE_K = 1024  # K per partial of the decode-size split
ONE_LAUNCH_MAX_M = 32  # nv4_w4a16_gemm runs one launch up to this M (see one_launch)


def dequant_w4a16(qweight, qzeros, scales, dtype=torch.bfloat16, group_size=128):
    """GPTQ weight -> dense [K, N] in ``dtype`` (bf16 or fp16), rounded as the
    W4A16 GEMMs round each dequantized weight."""
    if qweight.dtype != torch.int32 or qzeros.dtype != torch.int32 or scales.dtype != torch.float16:
        raise TypeError("Expected int32 qweight/qzeros and fp16 scales")
    if dtype not in _DT or qweight.ndim != 2:
        raise ValueError("Expected qweight [K/8, N] and a BF16 or FP16 target dtype")
    K, N = qweight.shape[0] * 8, qweight.shape[1]
    if group_size != 128 or K % 128 or N % 8:
        raise ValueError("Require group_size 128, K divisible by 128, N divisible by 8")
    if tuple(qzeros.shape) != (K // 128, N // 8) or tuple(scales.shape) != (K // 128, N):
        raise ValueError("Require qzeros [K/128, N/8] and scales [K/128, N]")
    if any(not t.is_cuda or not t.is_contiguous() or t.device != qweight.device for t in (qweight, qzeros, scales)):
        raise ValueError("All tensors must be contiguous on one CUDA device")
    w = torch.empty((K, N), dtype=dtype, device=qweight.device)
    lib = _lib.load()
    stream = torch.cuda.current_stream(qweight.device).cuda_stream
    with torch.cuda.device(qweight.device):
        rc = lib.nv4_w4a16_dequant(ctypes.c_void_p(qweight.data_ptr()), ctypes.c_void_p(qzeros.data_ptr()),
                                   ctypes.c_void_p(scales.data_ptr()), ctypes.c_void_p(w.data_ptr()), _DT[dtype],
                                   N, K, group_size, ctypes.c_void_p(stream))
    _lib.check(rc, "dequant_w4a16")
    return w


_CUS = {}


def one_launch(M, N, K, device=None):
    """Whether ``nv4_w4a16_gemm`` runs these sizes in its one-launch kernel
    (the rule it applies itself): the packed weight (K * N / 2 bytes) under
    2 GiB and M <= 16, or M <= 32 with K <= 4096 and ceil(N / 32) workgroups
    at most one per CU."""
    if M > ONE_LAUNCH_MAX_M or K * N // 2 >= (1 << 31):
        return False
    if M <= 16:
        return True
    idx = (torch.device(device).index or 0) if device is not None else torch.cuda.current_device()
    if idx not in _CUS:
        _CUS[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return K <= 4096 and (N + 31) // 32 <= _CUS[idx]


def dequant_matmul_w4a16(x, qweight, qzeros, scales, group_size=128, out=None):
    """x [M,K] bf16/fp16 -> out [M,N] in x's dtype."""
    if x.ndim != 2 or x.dtype not in _DT:
        raise ValueError("Expected BF16 or FP16 activations [M,K]")
    M, K = x.shape
    if qweight.dtype != torch.int32 or qzeros.dtype != torch.int32 or scales.dtype != torch.float16:
        raise TypeError("Expected int32 qweight/qzeros and fp16 scales")
    if qweight.ndim != 2 or qweight.shape[0] * 8 != K:
        raise ValueError("qweight must be [K/8, N]")
    N = qweight.shape[1]
    if group_size != 128 or K % 128 or N % 8 or M < 1:
        raise ValueError("Require group_size 128, K divisible by 128, N divisible by 8, M > 0")
    if tuple(qzeros.shape) != (K // 128, N // 8) or tuple(scales.shape) != (K // 128, N):
        raise ValueError("Require qzeros [K/128, N/8] and scales [K/128, N]")
    if out is None:
        out = torch.empty((M, N), device=x.device, dtype=x.dtype)
    if tuple(out.shape) != (M, N) or out.dtype not in _DT:
        raise ValueError("Output must be BF16 or FP16 [M,N]")
    tensors = (x, qweight, qzeros, scales, out)
    if any(not t.is_cuda or not t.is_contiguous() or t.device != x.device for t in tensors):
        raise ValueError("All tensors must be contiguous on one CUDA device")
    lib = _lib.load()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    with torch.cuda.device(x.device):
        if one_launch(M, N, K, x.device):
            rc = lib.nv4_w4a16_gemm(ctypes.c_void_p(x.data_ptr()), _DT[x.dtype],
                                    ctypes.c_void_p(qweight.data_ptr()), ctypes.c_void_p(qzeros.data_ptr()),
                                    ctypes.c_void_p(scales.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                                    _DT[out.dtype], M, N, K, group_size, ctypes.c_void_p(stream))
        elif M <= 64:
            S = (K + SLICE_K - 1) // SLICE_K
            ws = torch.empty((S * M * N,), dtype=torch.float32, device=x.device)
            rc = lib.nv4_w4a16_gemm_ws(ctypes.c_void_p(x.data_ptr()), _DT[x.dtype],
                                       ctypes.c_void_p(qweight.data_ptr()), ctypes.c_void_p(qzeros.data_ptr()),
                                       ctypes.c_void_p(scales.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                                       _DT[out.dtype], ctypes.c_void_p(ws.data_ptr()), ws.numel() * 4, M, N, K,
                                       group_size, ctypes.c_void_p(stream))
        else:
            w = torch.empty((K, N), dtype=x.dtype, device=x.device)
            rc = lib.nv4_w4a16_dequant(ctypes.c_void_p(qweight.data_ptr()), ctypes.c_void_p(qzeros.data_ptr()),
                                       ctypes.c_void_p(scales.data_ptr()), ctypes.c_void_p(w.data_ptr()),
                                       _DT[x.dtype], N, K, group_size, ctypes.c_void_p(stream))
            _lib.check(rc, "dequant_matmul_w4a16")
            if out.dtype == x.dtype:
                torch.mm(x, w, out=out)
            else:
                out.copy_(torch.mm(x, w))
            return out
    _lib.check(rc, "dequant_matmul_w4a16")
    return out
