"""Fused RHT + group-128 INT4 activation quantization + packing (MI355X).

Drop-in for ``nanovllm.kernels.rht_a4_tilelang`` (reference file
nanovllm/kernels/rht_a4_tilelang.py): same ``rht_quant_pack`` signature,
argument meaning, return value and ValueError conditions (:150-163), same
``Config``/``best_config``/``compile_kernel`` names (:13-16, :19-34,
:139-147).  The work runs in the hand-written HIP kernel
``nv4_rht_quant_pack`` of libnv4.so on torch's current stream; nothing
synchronises, so the call can be captured in a HIP graph and replays read the
current contents of ``x`` and ``signs``.

Contract (benchmarks/rht_a4_bench_common.py:19-36): layout
``row_DH_paley12_kron_sylvester_v1``, group 128, clip 0.9, BF16 scales rounded
before the codes, ties-to-even codes in [-7, 7], two signed nibbles per byte
with even k in the low nibble.  ``layout="block128"`` selects the per-128-block
Hadamard variant instead (not a reference layout).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from functools import lru_cache

import torch

from .. import _lib

LAYOUT_VERSION = "row_DH_paley12_kron_sylvester_v1"
_LAYOUTS = {"reference": _lib.LAYOUT_REFERENCE, LAYOUT_VERSION: _lib.LAYOUT_REFERENCE,
            "block128": _lib.LAYOUT_BLOCK128}


@dataclass(frozen=True)
class Config:
    """Launch hint kept for API compatibility with the reference
    (rht_a4_tilelang.py:13-16).  The HIP kernel picks its own launch shape
    (one 256-thread workgroup per row); a valid Config is accepted and does
    not change results."""
    threads_per_row: int = 128
    rows_per_block: int = 1


def _validate_config(cfg: Config) -> None:
    # Same acceptance rule as the reference's compile step (rht_a4_tilelang.py:22-23).
    tr, br = cfg.threads_per_row, cfg.rows_per_block
    if tr not in (32, 64, 128, 256, 512) or br < 1 or tr * br > 1024:
        raise ValueError("Unsupported RHT configuration")


@lru_cache(None)
def compile_kernel(K, cfg=Config()):
    """Return a callable ``kernel(X, D, Packed, Scale)`` for rows of width K."""
    if K not in (4096, 12288):
        raise ValueError("Unsupported RHT configuration")
    _validate_config(cfg)

    def kernel(x, signs, packed, scale, layout=_lib.LAYOUT_REFERENCE):
        _launch(x, signs, packed, scale, layout)
    return kernel


@lru_cache(None)
def best_config(M, K):
    """The reference's dispatch key is (M<=32 ? 32 : 4096, K); the HIP
    kernel has one launch shape per K, so every key maps to the default."""
    return Config()


def _launch(x, signs, packed, scale, layout):
    m, k = x.shape
    lib = _lib.load()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    with torch.cuda.device(x.device):
        rc = lib.nv4_rht_quant_pack(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(signs.data_ptr()),
                                    ctypes.c_void_p(packed.data_ptr()), ctypes.c_void_p(scale.data_ptr()),
                                    m, k, layout, ctypes.c_void_p(stream))
    _lib.check(rc, "rht_quant_pack")


def rht_quant_pack(x, signs, *, out_packed, out_scale, config=None, layout="reference"):
    """X[M,K] bf16, signs[K] int8 -> (out_packed int8 [M,K/2], out_scale bf16 [M,K/128]).

    Writes into the caller's buffers and returns them (reference :150-163).
    """
    lay = _LAYOUTS.get(layout)
    if lay is None:
        raise ValueError(f"Unknown RHT layout {layout!r}")
    widths_ok = (x.ndim == 2 and x.shape[1] in (4096, 12288)) if lay == _lib.LAYOUT_REFERENCE else (
        x.ndim == 2 and x.shape[1] % 128 == 0 and 0 < x.shape[1] <= 65536)
    if x.ndim != 2 or x.dtype != torch.bfloat16 or not widths_ok or x.shape[0] < 1:
        raise ValueError('Expected BF16 X[M,K], M>0, K=4096/12288')
    m, k = x.shape
    if signs.shape != (k,) or signs.dtype != torch.int8:
        raise ValueError('Expected INT8 signs[K]')
    if out_packed.shape != (m, k // 2) or out_packed.dtype != torch.int8:
        raise ValueError('Expected INT8 output[M,K/2]')
    if out_scale.shape != (m, k // 128) or out_scale.dtype != torch.bfloat16:
        raise ValueError('Expected BF16 scales[M,K/128]')
    if any(not t.is_cuda or not t.is_contiguous() or t.device != x.device
           for t in [x, signs, out_packed, out_scale]):
        raise ValueError('All tensors must be contiguous on one CUDA device')
    if config is not None:
        _validate_config(config)
    _launch(x, signs, out_packed, out_scale, lay)
    return out_packed, out_scale


def rowtiled_rows(m):
    """Rows of a row-tiled packed-activation buffer for M rows (16-row blocks)."""
    return (m + 15) // 16 * 16


def prefetch_args(prefetch):
    """(pointer, bytes) of a buffer for the prefetch tail of the row-tiled K1
    launches: a contiguous CUDA tensor whose size is a multiple of 16 bytes,
    or None."""
    if prefetch is None:
        return None, 0
    n = prefetch.numel() * prefetch.element_size()
    if not prefetch.is_cuda or not prefetch.is_contiguous() or n % 16:
        raise ValueError("prefetch must be a contiguous CUDA tensor of a multiple of 16 bytes")
    return ctypes.c_void_p(prefetch.data_ptr()), n


def rht_quant_pack_rowtiled(x, signs, *, out_packed=None, out_scale=None, prefetch=None):
    """``rht_quant_pack`` with the packed codes in the row-tiled order that the
    decode GEMM reads (``nv4_rht_quant_pack_rowtiled``): out_packed int8
    [ceil(M/16)*16, K/2] holds the same codes as the [M,K/2] form, in 1 KiB
    blocks of 16 rows x 128 k in matrix-core lane order; out_scale bf16
    [M,K/128] as usual.  ``prefetch``: a tensor (the weights of the GEMM that
    consumes the codes) that spare workgroups of the launch read into the
    Infinity Cache meanwhile; no result depends on it.  Returns
    (out_packed, out_scale)."""
    if x.ndim != 2 or x.dtype != torch.bfloat16 or x.shape[1] not in (4096, 12288) or x.shape[0] < 1:
        raise ValueError('Expected BF16 X[M,K], M>0, K=4096/12288')
    m, k = x.shape
    if signs.shape != (k,) or signs.dtype != torch.int8:
        raise ValueError('Expected INT8 signs[K]')
    if out_packed is None:
        out_packed = torch.empty((rowtiled_rows(m), k // 2), dtype=torch.int8, device=x.device)
    if out_scale is None:
        out_scale = torch.empty((m, k // 128), dtype=torch.bfloat16, device=x.device)
    if tuple(out_packed.shape) != (rowtiled_rows(m), k // 2) or out_packed.dtype != torch.int8:
        raise ValueError('Expected INT8 row-tiled output[ceil(M/16)*16,K/2]')
    if tuple(out_scale.shape) != (m, k // 128) or out_scale.dtype != torch.bfloat16:
        raise ValueError('Expected BF16 scales[M,K/128]')
    if any(not t.is_cuda or not t.is_contiguous() or t.device != x.device
           for t in [x, signs, out_packed, out_scale]):
        raise ValueError('All tensors must be contiguous on one CUDA device')
    if prefetch is not None and prefetch.device != x.device:
        raise ValueError('prefetch must be on the input device')
    pf, pf_bytes = prefetch_args(prefetch)
    lib = _lib.load()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    with torch.cuda.device(x.device):
        rc = lib.nv4_rht_quant_pack_rowtiled(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(signs.data_ptr()),
                                             ctypes.c_void_p(out_packed.data_ptr()),
                                             ctypes.c_void_p(out_scale.data_ptr()), m, k, pf, pf_bytes,
                                             ctypes.c_void_p(stream))
    _lib.check(rc, "rht_quant_pack_rowtiled")
    return out_packed, out_scale
