"""The W4A4 linear forward as one operator call (MI355X).

``W4A4Linear.forward`` of the reference (nanovllm/layers/linear_w4a4.py:27-35)
is ``rht_quant_pack`` followed by ``w4a4_grouped_gemm``.  ``w4a4_linear`` runs
the same two HIP kernels back to back through one C ABI call
(``nv4_w4a4_linear``) on torch's current stream, so it can be captured in a
HIP graph; the quantized activations are returned through ``out_packed`` /
``out_scale`` (allocated when not given).  With tiled weights, M <= 32 and
no ``out_packed`` given, K1 writes the codes in the row-tiled order and the
decode GEMM reads them from there (``nv4_w4a4_linear_rowtiled``, same bits).
Prefill-sized M
(``use_prefill_path``) runs K1 and then the fp6 matrix-core GEMM
(``nv4_w4a4_gemm_f6``, same bits).
"""
from __future__ import annotations

import ctypes

import torch

from .. import _lib
from .rht_a4 import rht_quant_pack, rowtiled_rows
from .w4a4_grouped import ROWTILED_MAX_M, _check_weights_f6, _launch, use_prefill_path


def w4a4_linear(x, signs, w_packed, w_scale, *, out=None, out_packed=None, out_scale=None, weights_tiled=False,
                weights_f6=None, packed_rowtiled=None):
    """x bf16 [M,K] (K = 4096 or 12288) -> bf16 [M,N].  ``weights_tiled``:
    ``w_packed`` is in the MFMA-tiled order (``tile_weights``).
    ``weights_f6``: the ``weights_to_f6`` form of the weights, used by
    prefill-sized calls instead of converting them again.
    ``packed_rowtiled``: whether ``out_packed`` receives the codes in the
    row-tiled order ([ceil(M/16)*16, K/2]; tiled weights, M <= 32); None
    chooses it exactly when ``out_packed`` is not given."""
    if x.ndim != 2 or x.dtype != torch.bfloat16 or x.shape[1] not in (4096, 12288) or x.shape[0] < 1:
        raise ValueError("Expected BF16 X[M,K], M>0, K=4096/12288")
    M, K = x.shape
    if w_packed.dtype != torch.int8 or signs.dtype != torch.int8:
        raise TypeError("Packed weights and signs must use int8 storage")
    if w_scale.dtype != torch.bfloat16:
        raise TypeError("Weight scales must be BF16")
    N = w_packed.shape[0] if w_packed.ndim == 2 else -1
    if tuple(signs.shape) != (K,) or tuple(w_packed.shape) != (N, K // 2) or N % 8 or N < 8:
        raise ValueError("Expected signs[K] and packed weights [N,K/2] with N divisible by 8")
    if weights_tiled and N % 16:
        raise ValueError("The tiled weight layout needs N divisible by 16")
    if tuple(w_scale.shape) != (N, K // 128):
        raise ValueError("Expected weight scales [N,K/128]")
    dev = x.device
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    # Decode-sized M whose codes only the GEMM needs: K1 writes them in the
    # row-tiled order that the decode GEMM loads straight into registers
    # (same bits).
    rowtiled = (weights_tiled and M <= ROWTILED_MAX_M and out_packed is None) if packed_rowtiled is None \
        else bool(packed_rowtiled)
    if rowtiled and (not weights_tiled or M > ROWTILED_MAX_M):
        raise ValueError("Row-tiled activation codes need tiled weights and M <= 32")
    if out_packed is None:
        out_packed = torch.empty((rowtiled_rows(M) if rowtiled else M, K // 2), dtype=torch.int8, device=dev)
    if out_scale is None:
        out_scale = torch.empty((M, K // 128), dtype=torch.bfloat16, device=dev)
    if (tuple(out.shape) != (M, N) or out.dtype != torch.bfloat16
            or tuple(out_packed.shape) != ((rowtiled_rows(M) if rowtiled else M), K // 2)
            or out_packed.dtype != torch.int8 or tuple(out_scale.shape) != (M, K // 128)
            or out_scale.dtype != torch.bfloat16):
        raise ValueError("Outputs must be BF16 [M,N], INT8 [M,K/2] and BF16 [M,K/128]")
    tensors = (x, signs, w_packed, w_scale, out, out_packed, out_scale)
    if any(not t.is_cuda or not t.is_contiguous() or t.device != dev for t in tensors):
        raise ValueError("All tensors must be contiguous on one CUDA device")
    _check_weights_f6(weights_f6, N, K, dev)
    if use_prefill_path(M, N, K):
        # Prefill-sized M: K1, then the grouped GEMM on the fp6 matrix cores.
        rht_quant_pack(x, signs, out_packed=out_packed, out_scale=out_scale)
        _launch(out_packed, w_packed, out_scale, w_scale, out, False, True, weights_tiled, path="fp6",
                weights_f6=weights_f6)
        return out
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    fn = lib.nv4_w4a4_linear_tiled if weights_tiled else lib.nv4_w4a4_linear
    if rowtiled:
        fn = lib.nv4_w4a4_linear_rowtiled
    with torch.cuda.device(dev):
        rc = fn(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(signs.data_ptr()),
                ctypes.c_void_p(w_packed.data_ptr()), ctypes.c_void_p(w_scale.data_ptr()),
                ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(out_packed.data_ptr()),
                ctypes.c_void_p(out_scale.data_ptr()), M, N, K, ctypes.c_void_p(stream))
    _lib.check(rc, "w4a4_linear")
    return out
