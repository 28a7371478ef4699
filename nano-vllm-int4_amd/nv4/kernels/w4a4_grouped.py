"""Grouped W4A4 INT4 GEMM (MI355X): G=128 activations, G=128 or per-channel weights.

Drop-in for ``nanovllm.kernels.w4a4_grouped_kernel`` (reference file
nanovllm/kernels/w4a4_grouped_kernel.py): ``w4a4_grouped_gemm`` keeps the
signature, validation order and exceptions of :104-129, ``compile_grouped_gemm``
keeps :32 (including the fp32-output diagnostic and the 1-D weight-scale
form), ``GroupedConfig``/``best_grouped_config`` keep :21-28/:94-101.

Each output element is, for g in order, ``total = fmaf(float(dot_g),
sa[m,g]*sw[n,g], total)`` with exact int32 group dots, rounded to bf16 at the
end (or ``total = fmaf(float(dot_g), sa[m,g], total)``; ``bf16(total*sw[n])``
for 1-D weight scales).  The HIP kernels (``nv4_w4a4_gemm``; for prefill-sized
M ``nv4_w4a4_gemm_f6``, the same bits on the fp6 matrix cores, or on request
``nv4_w4a4_gemm_f8`` on the fp8 ones) take M at run time: nothing is compiled
per shape, and there is no split-K and no atomics.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from functools import lru_cache

import torch

from .. import _lib

GROUP_SIZE = 128


@dataclass(frozen=True)
class GroupedConfig:
    """Launch hint kept for API compatibility (w4a4_grouped_kernel.py:21-28).
    The HIP kernels choose their own tiles from M; any valid config gives the
    same bits."""
    bm: int = 32
    bn: int = 64
    stages: int = 2
    threads: int = 128
    cache_scales: bool = False
    cache_weight_scales: bool = False


def _validate_config(cfg: GroupedConfig) -> None:
    if min(cfg.bm, cfg.bn, cfg.threads) < 1 or cfg.stages < 0 or cfg.threads % 32:
        raise ValueError("Require positive dimensions, K divisible by 128, N divisible by 8, and whole warps")


PATHS = ("int8", "fp8", "fp6")


def use_prefill_path(M, N, K):
    """Prefill-sized GEMMs run on the fp6 matrix cores (``nv4_w4a4_gemm_f6``).
    The operand conversion costs about 1.25 (M + N) K bytes of traffic and one
    launch; measured on the decoder's projections (with the fp8 form, whose
    conversion moves more bytes) it pays from M = 384 on weights of
    4096 x 12288 or more, from M = 768 above 4096 x 4096, and from M = 1024 on
    all of them."""
    nk = N * K
    return M >= 1024 or (M >= 768 and nk > 4096 * 4096) or (M >= 384 and nk >= 4096 * 12288)


def _resolve_path(path, M, N, K):
    if path is None:
        return "fp6" if use_prefill_path(M, N, K) else "int8"
    if path not in PATHS:
        raise ValueError(f"path must be None or one of {PATHS}")
    return path


def weights_f6_bytes(N, K):
    """Size of the fp6 tile form of [N, K] weights (``weights_to_f6``)."""
    n = _lib.load().nv4_w4a4_weights_f6_bytes(N, K)
    if n < 0:
        raise ValueError("Require N >= 1 and K a positive multiple of 128")
    return n


# Largest fp6 weight form a layer keeps (``keep_weights_f6``).
KEEP_F6_MAX_BYTES = 48 << 20


def keep_weights_f6(N, K):
    """Whether a layer keeps the fp6 form of its [N, K] weights.  Measured on
    the decoder's projections at M = 4096 (same box, interleaved), calls on
    kept weights beat converting them per call for qkv, o and down (12.6 to
    37.7 MB of fp6 tiles: 111.6 / 78.6 / 207.1 against 114.5 / 81.4 / 212.7
    us) but not for gate_up (75.5 MB: 474 against 439 us): the GEMM fetches
    each operand byte about nine times from beyond the L2, and the per-call
    conversion leaves fresh weight tiles in the 256 MB Infinity Cache, which
    weights read from HBM lack."""
    return weights_f6_bytes(N, K) <= KEEP_F6_MAX_BYTES


def weights_to_f6(w_packed, weights_tiled=False):
    """Packed [N,K/2] weights (or their ``tile_weights`` form) -> the fp6 tile
    blocks that the prefill GEMM reads, as a uint8 tensor.  Made once per
    layer, it lets prefill-sized calls convert only the activations; results
    are bit-identical."""
    if w_packed.ndim != 2 or w_packed.dtype != torch.int8 or not w_packed.is_cuda or not w_packed.is_contiguous():
        raise ValueError("Packed weights must be a contiguous int8 CUDA tensor [N,K/2]")
    N, K = w_packed.shape[0], w_packed.shape[1] * 2
    if N % 8 or K % GROUP_SIZE or (weights_tiled and N % 16):
        raise ValueError("Require N divisible by 8 (16 when tiled) and K divisible by 128")
    w6 = torch.empty(weights_f6_bytes(N, K), dtype=torch.uint8, device=w_packed.device)
    lib = _lib.load()
    stream = torch.cuda.current_stream(w_packed.device).cuda_stream
    with torch.cuda.device(w_packed.device):
        rc = lib.nv4_w4a4_weights_to_f6(ctypes.c_void_p(w_packed.data_ptr()), 1 if weights_tiled else 0,
                                        ctypes.c_void_p(w6.data_ptr()), N, K, w6.numel(), ctypes.c_void_p(stream))
    _lib.check(rc, "weights_to_f6")
    return w6


def _check_weights_f6(weights_f6, N, K, device):
    if weights_f6 is None:
        return
    if (weights_f6.dtype != torch.uint8 or weights_f6.ndim != 1 or not weights_f6.is_contiguous()
            or weights_f6.device != device or weights_f6.numel() != weights_f6_bytes(N, K)):
        raise ValueError("weights_f6 must be the weights_to_f6 tensor of these weights, on the input device")


def _launch(a_packed, w_packed, a_scale, w_scale, out, output_fp32, weight_grouped, weights_tiled=False, path=None,
            weights_f6=None):
    M, N, K = a_packed.shape[0], w_packed.shape[0], a_packed.shape[1] * 2
    path = _resolve_path(path, M, N, K)
    lib = _lib.load()
    stream = torch.cuda.current_stream(a_packed.device).cuda_stream
    with torch.cuda.device(a_packed.device):
        if path != "int8":
            # Matrix-core operands for this call (caching allocator: no
            # hipMalloc once warm); the kernels only read it on this stream.
            # Weights already in fp6 tiles (``weights_f6``) leave only the
            # activations to convert.
            w_form, w_ptr = (1 if weights_tiled else 0), w_packed.data_ptr()
            if path == "fp6":
                fn, nbytes = lib.nv4_w4a4_gemm_f6, lib.nv4_w4a4_gemm_f6_workspace(M, N, K)
                if weights_f6 is not None:
                    w_form, w_ptr = 2, weights_f6.data_ptr()
                    nbytes -= weights_f6.numel()
            else:
                fn, nbytes = lib.nv4_w4a4_gemm_f8, (M + N) * K
            ws = torch.empty(nbytes, dtype=torch.uint8, device=a_packed.device)
            rc = fn(ctypes.c_void_p(a_packed.data_ptr()), ctypes.c_void_p(w_ptr), w_form,
                    ctypes.c_void_p(a_scale.data_ptr()), ctypes.c_void_p(w_scale.data_ptr()),
                    1 if weight_grouped else 0, ctypes.c_void_p(out.data_ptr()),
                    1 if output_fp32 else 0, M, N, K, ctypes.c_void_p(ws.data_ptr()),
                    ws.numel(), ctypes.c_void_p(stream))
        else:
            fn = lib.nv4_w4a4_gemm_tiled if weights_tiled else lib.nv4_w4a4_gemm
            rc = fn(ctypes.c_void_p(a_packed.data_ptr()), ctypes.c_void_p(w_packed.data_ptr()),
                    ctypes.c_void_p(a_scale.data_ptr()), ctypes.c_void_p(w_scale.data_ptr()),
                    1 if weight_grouped else 0, ctypes.c_void_p(out.data_ptr()),
                    1 if output_fp32 else 0, M, N, K, ctypes.c_void_p(stream))
    _lib.check(rc, "w4a4_grouped_gemm")


def _tile(src, to_tiled):
    if src.ndim != 2 or src.dtype != torch.int8 or not src.is_cuda or not src.is_contiguous():
        raise ValueError("Packed weights must be a contiguous int8 CUDA tensor [N,K/2]")
    N, K = src.shape[0], src.shape[1] * 2
    if N % 16 or K % GROUP_SIZE or min(N, K) < 1:
        raise ValueError("The tiled weight layout needs N divisible by 16 and K divisible by 128")
    dst = torch.empty_like(src)
    lib = _lib.load()
    fn = lib.nv4_w4a4_tile_weights if to_tiled else lib.nv4_w4a4_untile_weights
    stream = torch.cuda.current_stream(src.device).cuda_stream
    with torch.cuda.device(src.device):
        rc = fn(ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), N, K, ctypes.c_void_p(stream))
    _lib.check(rc, "tile_weights" if to_tiled else "untile_weights")
    return dst


def tile_weights(w_packed):
    """[N,K/2] packed weights -> the same bytes in the MFMA-tiled order read
    by the decode kernels (1 KiB per 16 columns x 128 k, lane-major)."""
    return _tile(w_packed, True)


def untile_weights(w_tiled):
    """Inverse of ``tile_weights``."""
    return _tile(w_tiled, False)


@lru_cache(None)
def compile_grouped_gemm(M, N, K, cfg=GroupedConfig(), output_fp32=False, weight_grouped=False, path=None):
    """Return ``kernel(A, W, Sa, Sw, C)`` for exact (M, N, K), as the reference does
    (its kernel is JIT-specialised on M; this one only checks the shapes).
    ``path``: "int8", "fp8" or "fp6" forces a kernel family (same bits); None
    chooses by size (``use_prefill_path``)."""
    if path is not None and path not in PATHS:
        raise ValueError(f"path must be None or one of {PATHS}")
    if min(M, N, K) < 1 or K % GROUP_SIZE or N % 8:
        raise ValueError("Require positive dimensions, K divisible by 128, N divisible by 8, and whole warps")
    _validate_config(cfg)
    out_dtype = torch.float32 if output_fp32 else torch.bfloat16
    sw_shape = (N, K // GROUP_SIZE) if weight_grouped else (N,)

    def kernel(a_packed, w_packed, a_scale, w_scale, out):
        if (tuple(a_packed.shape) != (M, K // 2) or tuple(w_packed.shape) != (N, K // 2)
                or tuple(a_scale.shape) != (M, K // GROUP_SIZE) or tuple(w_scale.shape) != sw_shape
                or tuple(out.shape) != (M, N) or out.dtype != out_dtype):
            raise ValueError("Arguments do not match the compiled (M, N, K) kernel")
        tensors = (a_packed, w_packed, a_scale, w_scale, out)
        if any(not t.is_cuda or not t.is_contiguous() or t.device != a_packed.device for t in tensors):
            raise ValueError("All inputs must be contiguous CUDA tensors on one device")
        _launch(a_packed, w_packed, a_scale, w_scale, out, output_fp32, weight_grouped, path=path)
    return kernel


@lru_cache(None)
def best_grouped_config(M, N, K, weight_grouped=False):
    """Reference dispatch-table lookup (w4a4_grouped_kernel.py:94-101); the HIP
    kernels do not use it, so it returns the reference defaults."""
    return GroupedConfig() if M <= 32 else GroupedConfig(64, 128, 2, 128)


def w4a4_grouped_gemm(a_packed, w_packed, a_scale, w_scale, out=None, config=None, *, weights_tiled=False, path=None,
                      weights_f6=None):
    """Packed INT4; BF16 Sa[M,K/128], Sw[N] or Sw[N,K/128], output[M,N].
    ``weights_tiled``: ``w_packed`` holds ``tile_weights`` output (N % 16 == 0);
    the result is bit-identical.  ``path``: "int8", "fp8" or "fp6" forces a
    kernel family (same bits); None chooses by size.  ``weights_f6``: the
    ``weights_to_f6`` form of these weights, used by the fp6 path instead of
    converting them again."""
    if a_packed.ndim != 2 or w_packed.ndim != 2 or a_packed.shape[1] != w_packed.shape[1]:
        raise ValueError("Packed inputs must have compatible [M,K/2] and [N,K/2] shapes")
    M, K = a_packed.shape[0], a_packed.shape[1] * 2
    N = w_packed.shape[0]
    if a_packed.dtype != torch.int8 or w_packed.dtype != torch.int8:
        raise TypeError("Packed inputs must use int8 storage")
    if K % GROUP_SIZE or N % 8 or min(M, N, K) < 1:
        raise ValueError("Require positive dimensions, K divisible by 128, N divisible by 8")
    weight_grouped = w_scale.ndim == 2
    expected_w_scale = (N, K // GROUP_SIZE) if weight_grouped else (N,)
    if tuple(a_scale.shape) != (M, K // GROUP_SIZE) or tuple(w_scale.shape) != expected_w_scale:
        raise ValueError("Require Sa[M,K/128] and Sw[N] or Sw[N,K/128]")
    if a_scale.dtype != torch.bfloat16 or w_scale.dtype != torch.bfloat16:
        raise TypeError("Both scale tensors must be BF16")
    tensors = (a_packed, w_packed, a_scale, w_scale)
    if any(not value.is_cuda or not value.is_contiguous() or value.device != a_packed.device
           for value in tensors):
        raise ValueError("All inputs must be contiguous CUDA tensors on one device")
    if out is None:
        out = torch.empty((M, N), device=a_packed.device, dtype=torch.bfloat16)
    if (tuple(out.shape) != (M, N) or out.dtype != torch.bfloat16 or out.device != a_packed.device
            or not out.is_contiguous()):
        raise ValueError("Output must be contiguous BF16 [M,N] on the input device")
    if config is not None:
        _validate_config(config)
    if weights_tiled and N % 16:
        raise ValueError("The tiled weight layout needs N divisible by 16")
    _check_weights_f6(weights_f6, N, K, a_packed.device)
    _launch(a_packed, w_packed, a_scale, w_scale, out, False, weight_grouped, weights_tiled, path=path,
            weights_f6=weights_f6)
    return out


# Largest M of the row-tiled decode GEMM (nv4_w4a4_gemm_rowtiled).
ROWTILED_MAX_M = 32


def w4a4_gemm_rowtiled(a_rt, w_tiled, a_scale, w_scale, out=None, *, output_fp32=False):
    """``w4a4_grouped_gemm`` for decode-sized M (1..32) on row-tiled packed
    activations (``rht_quant_pack_rowtiled``: int8 [ceil(M/16)*16, K/2]) and
    tiled weights (``tile_weights``); M is taken from ``a_scale`` [M, K/128].
    Bit-identical to the reference-layout call."""
    if a_scale.ndim != 2 or w_tiled.ndim != 2 or a_rt.ndim != 2:
        raise ValueError("Expected Sa[M,K/128], tiled weights [N,K/2] and row-tiled activations")
    M, N, K = a_scale.shape[0], w_tiled.shape[0], w_tiled.shape[1] * 2
    if a_rt.dtype != torch.int8 or w_tiled.dtype != torch.int8:
        raise TypeError("Packed inputs must use int8 storage")
    if a_scale.dtype != torch.bfloat16 or w_scale.dtype != torch.bfloat16:
        raise TypeError("Both scale tensors must be BF16")
    if not 1 <= M <= ROWTILED_MAX_M or K % GROUP_SIZE or N % 16 or K < GROUP_SIZE:
        raise ValueError("Require 1 <= M <= 32, K divisible by 128 and N divisible by 16")
    if tuple(a_rt.shape) != ((M + 15) // 16 * 16, K // 2) or tuple(a_scale.shape) != (M, K // GROUP_SIZE):
        raise ValueError("Require row-tiled activations [ceil(M/16)*16,K/2] and Sa[M,K/128]")
    weight_grouped = w_scale.ndim == 2
    if tuple(w_scale.shape) != ((N, K // GROUP_SIZE) if weight_grouped else (N,)):
        raise ValueError("Require Sw[N] or Sw[N,K/128]")
    dtype = torch.float32 if output_fp32 else torch.bfloat16
    if out is None:
        out = torch.empty((M, N), device=a_rt.device, dtype=dtype)
    if tuple(out.shape) != (M, N) or out.dtype != dtype:
        raise ValueError("Output must be [M,N] of the requested dtype")
    if any(not t.is_cuda or not t.is_contiguous() or t.device != a_rt.device
           for t in (a_rt, w_tiled, a_scale, w_scale, out)):
        raise ValueError("All tensors must be contiguous CUDA tensors on one device")
    lib = _lib.load()
    stream = torch.cuda.current_stream(a_rt.device).cuda_stream
    with torch.cuda.device(a_rt.device):
        rc = lib.nv4_w4a4_gemm_rowtiled(ctypes.c_void_p(a_rt.data_ptr()), ctypes.c_void_p(w_tiled.data_ptr()),
                                        ctypes.c_void_p(a_scale.data_ptr()), ctypes.c_void_p(w_scale.data_ptr()),
                                        1 if weight_grouped else 0, ctypes.c_void_p(out.data_ptr()),
                                        1 if output_fp32 else 0, M, N, K, ctypes.c_void_p(stream))
    _lib.check(rc, "w4a4_gemm_rowtiled")
    return out


# Limits of the wide decode kernel (its LDS holds the widened activation block
# and the scales): the same rule the library applies.
_WIDE_A_BYTES, _WIDE_SCALES, _WIDE_WSCALES = 128 * 1024, 1024, 3072
_CUS = {}


def rowtiled_silu_fits(M, N, K, device=None):
    """Whether ``w4a4_gemm_rowtiled_silu`` serves a fused gate/up weight of N
    rows (gate rows, then up rows) at these sizes: the wide decode kernel's
    limits (4 to 8 column blocks of 16 per CU, activations and scales in LDS)
    and N a multiple of 32."""
    if not 1 <= M <= ROWTILED_MAX_M or N % 32 or K % 256:
        return False
    idx = (torch.device(device).index or 0) if device is not None else torch.cuda.current_device()
    if idx not in _CUS:
        _CUS[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    mb = (M + 15) // 16
    per_cu = (N // 16 + _CUS[idx] - 1) // _CUS[idx]
    cbw = 4 if per_cu <= 4 else 6 if per_cu <= 6 else 8
    return (mb * 16 * K <= _WIDE_A_BYTES and (K // 128) * mb * 16 <= _WIDE_SCALES and 4 <= per_cu <= 8
            and (K // 128) * 16 * cbw <= _WIDE_WSCALES)


def w4a4_gemm_rowtiled_silu(a_rt, w_tiled, a_scale, w_scale, out=None):
    """SiLU-and-mul of a fused gate/up projection in one launch: with the
    tiled weight's first N/2 rows the gate and the last N/2 the up projection,
    out bf16 [M, N/2] = bf16(bf16(silu(g)) * u) for g, u the bf16 results
    ``w4a4_gemm_rowtiled`` would store -- the same bits as that GEMM followed
    by ``silu_mul``.  Sizes as ``rowtiled_silu_fits``."""
    if a_scale.ndim != 2 or w_tiled.ndim != 2 or a_rt.ndim != 2:
        raise ValueError("Expected Sa[M,K/128], tiled weights [N,K/2] and row-tiled activations")
    M, N, K = a_scale.shape[0], w_tiled.shape[0], w_tiled.shape[1] * 2
    if a_rt.dtype != torch.int8 or w_tiled.dtype != torch.int8:
        raise TypeError("Packed inputs must use int8 storage")
    if a_scale.dtype != torch.bfloat16 or w_scale.dtype != torch.bfloat16:
        raise TypeError("Both scale tensors must be BF16")
    if not rowtiled_silu_fits(M, N, K, a_rt.device):
        raise ValueError("Sizes outside the paired gate/up kernel (see rowtiled_silu_fits)")
    if tuple(a_rt.shape) != ((M + 15) // 16 * 16, K // 2) or tuple(a_scale.shape) != (M, K // GROUP_SIZE):
        raise ValueError("Require row-tiled activations [ceil(M/16)*16,K/2] and Sa[M,K/128]")
    weight_grouped = w_scale.ndim == 2
    if tuple(w_scale.shape) != ((N, K // GROUP_SIZE) if weight_grouped else (N,)):
        raise ValueError("Require Sw[N] or Sw[N,K/128]")
    if out is None:
        out = torch.empty((M, N // 2), device=a_rt.device, dtype=torch.bfloat16)
    if tuple(out.shape) != (M, N // 2) or out.dtype != torch.bfloat16:
        raise ValueError("Output must be bf16 [M,N/2]")
    if any(not t.is_cuda or not t.is_contiguous() or t.device != a_rt.device
           for t in (a_rt, w_tiled, a_scale, w_scale, out)):
        raise ValueError("All tensors must be contiguous CUDA tensors on one device")
    lib = _lib.load()
    stream = torch.cuda.current_stream(a_rt.device).cuda_stream
    with torch.cuda.device(a_rt.device):
        rc = lib.nv4_w4a4_gemm_rowtiled_silu(ctypes.c_void_p(a_rt.data_ptr()), ctypes.c_void_p(w_tiled.data_ptr()),
                                             ctypes.c_void_p(a_scale.data_ptr()), ctypes.c_void_p(w_scale.data_ptr()),
                                             1 if weight_grouped else 0, ctypes.c_void_p(out.data_ptr()), M, N, K,
                                             ctypes.c_void_p(stream))
    _lib.check(rc, "w4a4_gemm_rowtiled_silu")
    return out
