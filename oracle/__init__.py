"""CPU oracle for the quantized-linear path -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg may
import this package, and only to check results against; the product (the ``nv4``
package and its HIP library) never imports it and has no CPU fallback.

The numerics live in ``oracle.c`` (a C restatement of the reference's RHT,
group-128 quantizer, INT4 packing, grouped INT4 GEMM and W4A16 dequant GEMM,
each citing the reference file:line it follows).  This module is a thin
ctypes/numpy layer over it, plus bf16/fp16 bit helpers.

Arrays of bf16 or fp16 values are carried as ``uint16`` bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "liboracle.so"
_lib = None

LAYOUT_REFERENCE = 0   # row_DH_paley12_kron_sylvester_v1
LAYOUT_BLOCK128 = 1    # per-128-block Hadamard (not a reference layout)


def build(force: bool = False) -> Path:
    """Compile liboracle.so with oracle/Makefile."""
    cmd = ["make", "-C", str(_DIR)] + (["-B"] if force else [])
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        sigs = {
            "orc_rht_rows": [P, P, P, I64, I64, I, I],
            "orc_quantize_rows": [P, P, P, I64, I64, I64, I],
            "orc_weight_quantize": [P, P, P, I64, I64, I64, ctypes.c_float, I, I],
            "orc_weight_dequantize": [P, P, P, I64, I64, I64],
            "orc_pack_int4": [P, P, I64],
            "orc_unpack_int4": [P, P, I64],
            "orc_rht_quant_pack": [P, P, P, P, I64, I64, I, I],
            "orc_w4a4_gemm": [P, P, P, P, I, P, I, I64, I64, I64, I],
            "orc_w4a4_group_dots": [P, P, P, I64, I64, I64],
            "orc_w4a16_dequant": [P, P, P, P, I64, I64, I64, I],
            "orc_w4a16_gemm": [P, I, P, P, P, P, I64, I64, I64, I64, I],
            "orc_set_mutation": [I],
            "orc_paley_sign": [I, I],
            "orc_constant_bits": [I],
            "orc_max_threads": [],
        }
        for name, args in sigs.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        L.orc_constant_bits.restype = ctypes.c_uint32
        for name in ("orc_f32_to_bf16", "orc_bf16_to_f32", "orc_f32_to_f16", "orc_f16_to_f32"):
            fn = getattr(L, name)
            fn.argtypes = [P, P, I64]
            fn.restype = None
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _check(rc: int, what: str):
    if rc != 0:
        raise ValueError(f"oracle {what} rejected its arguments (code {rc})")


def threads_default() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


# --------------------------------------------------------------- bit helpers
def f32_to_bf16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16(_ptr(x), _ptr(out), x.size)
    return out


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_bf16_to_f32(_ptr(h), _ptr(out), h.size)
    return out


def f32_to_f16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16(_ptr(x), _ptr(out), x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32(_ptr(h), _ptr(out), h.size)
    return out


def constant_bits(which: int) -> int:
    """0: fp32(0.9), 1: RN(1/7), 2: RN(1/sqrt 12), 3: RN(1/sqrt 128)."""
    return int(lib().orc_constant_bits(which))


def paley_sign(s: int, d: int) -> int:
    return int(lib().orc_paley_sign(s, d))


def set_mutation(m: int) -> int:
    """Plant a known mistake in the oracle (tests only); returns the previous one."""
    return int(lib().orc_set_mutation(m))


# ------------------------------------------------------------------- K1 path
def rht_rows(x_bf16: np.ndarray, signs: np.ndarray, layout: int = LAYOUT_REFERENCE,
             threads: int = 0) -> np.ndarray:
    """fp32 X D H for bf16 rows ``x_bf16`` [M,K] (uint16 bits) and int8 signs [K]."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    s = np.ascontiguousarray(signs, dtype=np.int8)
    M, K = x.shape
    out = np.empty((M, K), dtype=np.float32)
    _check(lib().orc_rht_rows(_ptr(x), _ptr(s), _ptr(out), M, K, layout, threads), "rht_rows")
    return out


def quantize_rows(rotated: np.ndarray, group: int = 128, threads: int = 0):
    """fp32 rows -> (int8 codes [M,K] in [-7,7], bf16 scale bits [M,K/group])."""
    r = np.ascontiguousarray(rotated, dtype=np.float32)
    M, K = r.shape
    codes = np.empty((M, K), dtype=np.int8)
    scales = np.empty((M, K // group), dtype=np.uint16)
    _check(lib().orc_quantize_rows(_ptr(r), _ptr(codes), _ptr(scales), M, K, group, threads), "quantize_rows")
    return codes, scales


def pack_int4(codes: np.ndarray) -> np.ndarray:
    c = np.ascontiguousarray(codes, dtype=np.int8)
    out = np.empty(c.shape[:-1] + (c.shape[-1] // 2,), dtype=np.int8)
    _check(lib().orc_pack_int4(_ptr(c), _ptr(out), c.size), "pack_int4")
    return out


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    p = np.ascontiguousarray(packed, dtype=np.int8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.int8)
    _check(lib().orc_unpack_int4(_ptr(p), _ptr(out), out.size), "unpack_int4")
    return out


def rht_quant_pack(x_bf16: np.ndarray, signs: np.ndarray, layout: int = LAYOUT_REFERENCE,
                   threads: int = 0):
    """The K1 contract: (packed int8 [M,K/2], bf16 scale bits [M,K/128])."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    s = np.ascontiguousarray(signs, dtype=np.int8)
    M, K = x.shape
    packed = np.empty((M, K // 2), dtype=np.int8)
    scales = np.empty((M, K // 128), dtype=np.uint16)
    _check(lib().orc_rht_quant_pack(_ptr(x), _ptr(s), _ptr(packed), _ptr(scales), M, K, layout, threads),
           "rht_quant_pack")
    return packed, scales


# ------------------------------------------------------- weight quantization
DIVISION_CPU, DIVISION_CUDA = 0, 1


def weight_quantize(w, group: int = 128, clip: float = 1.0, division: int = DIVISION_CUDA,
                    threads: int = 0):
    """Round-to-nearest grouped quantizer of fp32 rows ``w`` [N,K].

    ``grouped_quantize(w, group, clip)`` (benchmarks/kernel_bench_common.py:
    36-42) and, at clip 1, ``quantize_groups`` (benchmarks/rht_gptq_grouped.py:
    27-34; K need not be a multiple of ``group``) and ``quantize_rows``
    (benchmarks/rht_reference.py:70-77, group = K).  ``division`` names the
    device the reference ran the expression on: DIVISION_CUDA multiplies by
    RN(1/7), DIVISION_CPU divides by 7.  Returns (int8 codes [N,K], bf16 scale
    bits [N, ceil(K/group)]).
    """
    x = np.ascontiguousarray(w, dtype=np.float32)
    N, K = x.shape
    G = -(-K // group)
    codes = np.empty((N, K), dtype=np.int8)
    scales = np.empty((N, G), dtype=np.uint16)
    _check(lib().orc_weight_quantize(_ptr(x), _ptr(codes), _ptr(scales), N, K, group, ctypes.c_float(clip),
                                     division, threads), "weight_quantize")
    return codes, scales


def weight_dequantize(codes, scales_bf16, group: int = 128) -> np.ndarray:
    """codes [N,K] x bf16 scale bits [N,ceil(K/group)] -> exact fp32 [N,K]
    (benchmarks/rht_gptq_grouped.py:37-39)."""
    c = np.ascontiguousarray(codes, dtype=np.int8)
    s = np.ascontiguousarray(scales_bf16, dtype=np.uint16)
    N, K = c.shape
    if s.shape != (N, -(-K // group)):
        raise ValueError("scale shape does not match codes and group")
    out = np.empty((N, K), dtype=np.float32)
    _check(lib().orc_weight_dequantize(_ptr(c), _ptr(s), _ptr(out), N, K, group), "weight_dequantize")
    return out


def error_stats(actual, reference) -> dict:
    """Error summary of ``actual`` against ``reference``
    (benchmarks/rht_reference.py:99-108).  As there, both are taken to fp32,
    the difference and the squares are fp32 operations, and the squares are
    summed in float64; the cosine's dot product is float64.  Returns relative
    RMSE sqrt(sse/energy), max |d|, cosine, sse, reference energy and element
    count, with denominators floored at 1e-30.  The float64 sums run in numpy's
    pairwise order, so their last bits may differ from torch's reduction."""
    a = np.ascontiguousarray(actual, dtype=np.float32).ravel()
    r = np.ascontiguousarray(reference, dtype=np.float32).ravel()
    d = a - r
    sse = float(np.sum((d * d).astype(np.float64)))
    energy = float(np.sum((r * r).astype(np.float64)))
    own = float(np.sum((a * a).astype(np.float64)))
    cosine = float(a.astype(np.float64) @ r.astype(np.float64)) / max(np.sqrt(own * energy), 1e-30)
    return {"relative_rmse": float(np.sqrt(sse / max(energy, 1e-30))),
            "max_abs": float(np.max(np.abs(d))) if d.size else 0.0,
            "cosine": cosine, "sse": sse, "reference_energy": energy, "elements": int(d.size)}


# ------------------------------------------------------------------- K2 path
def w4a4_gemm(a_packed, w_packed, sa_bf16, sw_bf16, out_fp32: bool = False, threads: int = 0):
    """Grouped INT4 GEMM; ``sw_bf16`` [N,K/128] (grouped) or [N] (per channel).

    Returns bf16 bits [M,N] (uint16) or fp32 [M,N] when ``out_fp32``.
    """
    a = np.ascontiguousarray(a_packed, dtype=np.int8)
    w = np.ascontiguousarray(w_packed, dtype=np.int8)
    sa = np.ascontiguousarray(sa_bf16, dtype=np.uint16)
    sw = np.ascontiguousarray(sw_bf16, dtype=np.uint16)
    M, N, K = a.shape[0], w.shape[0], a.shape[1] * 2
    grouped = 1 if sw.ndim == 2 else 0
    out = np.empty((M, N), dtype=np.float32 if out_fp32 else np.uint16)
    _check(lib().orc_w4a4_gemm(_ptr(a), _ptr(w), _ptr(sa), _ptr(sw), grouped, _ptr(out),
                               1 if out_fp32 else 0, M, N, K, threads), "w4a4_gemm")
    return out


def w4a4_group_dots(a_packed, w_packed) -> np.ndarray:
    """Exact int32 per-group dots d[m, n, g]."""
    a = np.ascontiguousarray(a_packed, dtype=np.int8)
    w = np.ascontiguousarray(w_packed, dtype=np.int8)
    M, N, K = a.shape[0], w.shape[0], a.shape[1] * 2
    out = np.empty((M, N, K // 128), dtype=np.int32)
    _check(lib().orc_w4a4_group_dots(_ptr(a), _ptr(w), _ptr(out), M, N, K), "w4a4_group_dots")
    return out


# ------------------------------------------------------------------- K3 path
X_BF16, X_FP16 = 0, 1


def w4a16_dequant(qweight, qzeros, scales_f16, group: int = 128, x_dtype: int = X_BF16) -> np.ndarray:
    """fp32 [K,N] of the rounded dequantized GPTQ weights."""
    qw = np.ascontiguousarray(qweight, dtype=np.int32)
    qz = np.ascontiguousarray(qzeros, dtype=np.int32)
    sc = np.ascontiguousarray(scales_f16, dtype=np.uint16)
    K, N = qw.shape[0] * 8, qw.shape[1]
    out = np.empty((K, N), dtype=np.float32)
    _check(lib().orc_w4a16_dequant(_ptr(qw), _ptr(qz), _ptr(sc), _ptr(out), N, K, group, x_dtype),
           "w4a16_dequant")
    return out


def w4a16_gemm(x_bits, qweight, qzeros, scales_f16, group: int = 128, x_dtype: int = X_BF16,
               threads: int = 0) -> np.ndarray:
    """float64 [M,N] exact-sum product of the activations and the dequantized weights."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    qw = np.ascontiguousarray(qweight, dtype=np.int32)
    qz = np.ascontiguousarray(qzeros, dtype=np.int32)
    sc = np.ascontiguousarray(scales_f16, dtype=np.uint16)
    M, K = x.shape
    N = qw.shape[1]
    out = np.empty((M, N), dtype=np.float64)
    _check(lib().orc_w4a16_gemm(_ptr(x), x_dtype, _ptr(qw), _ptr(qz), _ptr(sc), _ptr(out),
                                M, N, K, group, threads), "w4a16_gemm")
    return out


def max_threads() -> int:
    return int(lib().orc_max_threads())
