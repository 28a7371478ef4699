"""ctypes binding of libnv4.so, the gfx950 HIP library behind every nv4 operator.

There is no fallback: if the library is missing or fails to load, every
operator raises.  Build it with ``make -C nano-vllm-int4_amd`` (or
``__graft_entry__.build()``).
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

_HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("NV4_LIB", _HERE / "libnv4.so"))

NV4_OK = 0
NV4_E_NULL = -1
NV4_E_SHAPE = -2
NV4_E_ALIGN = -3
NV4_E_LAYOUT = -4
NV4_E_DTYPE = -5
NV4_E_GROUP = -6
NV4_E_SCRATCH = -7
PA_SCRATCH_BYTES = 16 << 20  # device scratch of nv4_paged_decode_attention_noalloc

LAYOUT_REFERENCE = 0
LAYOUT_BLOCK128 = 1
BF16, FP16, FP32 = 0, 1, 2

# Every symbol declared in include/nv4.h, with its ctypes signature.
_P, _I, _I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
SIGNATURES = {
    "nv4_rht_quant_pack": ([_P, _P, _P, _P, _I64, _I64, _I, _P], _I),
    "nv4_w4a4_gemm": ([_P, _P, _P, _P, _I, _P, _I, _I64, _I64, _I64, _P], _I),
    "nv4_w4a4_linear": ([_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P], _I),
    "nv4_w4a4_gemm_tiled": ([_P, _P, _P, _P, _I, _P, _I, _I64, _I64, _I64, _P], _I),
    "nv4_w4a4_gemm_f8": ([_P, _P, _I, _P, _P, _I, _P, _I, _I64, _I64, _I64, _P, _I64, _P], _I),
    "nv4_w4a4_gemm_f6": ([_P, _P, _I, _P, _P, _I, _P, _I, _I64, _I64, _I64, _P, _I64, _P], _I),
    "nv4_w4a4_gemm_f6_workspace": ([_I64, _I64, _I64], _I64),
    "nv4_w4a4_weights_to_f6": ([_P, _I, _P, _I64, _I64, _I64, _P], _I),
    "nv4_w4a4_weights_f6_bytes": ([_I64, _I64], _I64),
    "nv4_prefill_attention": ([_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, ctypes.c_float, _P], _I),
    "nv4_w4a4_linear_tiled": ([_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P], _I),
    "nv4_rht_quant_pack_rowtiled": ([_P, _P, _P, _P, _I64, _I64, _P, _I64, _P], _I),
    "nv4_w4a4_gemm_rowtiled": ([_P, _P, _P, _P, _I, _P, _I, _I64, _I64, _I64, _P], _I),
    "nv4_w4a4_gemm_rowtiled_silu": ([_P, _P, _P, _P, _I, _P, _I64, _I64, _I64, _P], _I),
    "nv4_w4a4_linear_rowtiled": ([_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P], _I),
    "nv4_w4a4_prefetch_bytes": ([_I64, _I64], _I64),
    "nv4_rmsnorm_rht_quant_pack_rowtiled": ([_P, _P, _P, _P, ctypes.c_float, _P, _P, _P, _I64, _I64, _P, _I64, _P],
                                            _I),
    "nv4_silu_mul_rht_quant_pack_rowtiled": ([_P, _P, _P, _P, _I64, _I64, _P, _I64, _P], _I),
    "nv4_w4a4_tile_weights": ([_P, _P, _I64, _I64, _P], _I),
    "nv4_w4a4_untile_weights": ([_P, _P, _I64, _I64, _P], _I),
    "nv4_w4a16_gemm": ([_P, _I, _P, _P, _P, _P, _I, _I64, _I64, _I64, _I, _P], _I),
    "nv4_w4a16_gemm_ws": ([_P, _I, _P, _P, _P, _P, _I, _P, _I64, _I64, _I64, _I64, _I, _P], _I),
    "nv4_w4a16_dequant": ([_P, _P, _P, _P, _I, _I64, _I64, _I, _P], _I),
    "nv4_paged_decode_attention": ([_P, _I64, _P, _P, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                                    _I64, ctypes.c_float, _P], _I),
    "nv4_paged_decode_attention_qkv": ([_P, _I64, _P, _P, _P, _I64, _P, _P, _I64, _P, _P, _P, _I64, _P, _P, _P,
                                        _I64, _I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_float, ctypes.c_float,
                                        _P], _I),
    "nv4_paged_decode_attention_noalloc": ([_P, _I64, _P, _P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64,
                                            _I64, ctypes.c_float, _P], _I),
    "nv4_rmsnorm": ([_P, _P, _P, _P, _P, _I64, _I64, ctypes.c_float, _P], _I),
    "nv4_qk_norm_rope_store": ([_P, _I64, _I64, _I64, _I64, _P, _P, _P, _I64, _P, _P, _I64, _P, _P, _P, _P, _P,
                                ctypes.c_float, _P], _I),
    "nv4_silu_mul": ([_P, _P, _I64, _I64, _P], _I),
    "nv4_rmsnorm_rht_quant_pack": ([_P, _P, _P, _P, ctypes.c_float, _P, _P, _P, _I64, _I64, _P], _I),
    "nv4_silu_mul_rht_quant_pack": ([_P, _P, _P, _P, _I64, _I64, _P], _I),
    "nv4_gumbel_sample": ([_P, _I64, _I, _P, _I64, _I64, ctypes.c_uint64, ctypes.c_uint64, _P, _P], _I),
    "nv4_gumbel_sample_chunks": ([_I64, _I64], _I64),
    "nv4_gumbel_sample_ws": ([_P, _I64, _I, _P, _I64, _I64, ctypes.c_uint64, ctypes.c_uint64, _P, _I64, _P, _P], _I),
    "nv4_philox4x32_10": ([_P, _P, _P], None),
    "nv4_probe_mfma": ([_I, _I64, _I64, _P, _P], _I),
    "nv4_probe_read": ([_P, _I64, _P, _P], _I),
    "nv4_probe_bf16_rne": ([_P, _P], _I),
    "nv4_lm_head": ([_P, _I64, _P, _P, _I64, _I64, _I64, _I64, _P], _I),
    "nv4_version": ([], ctypes.c_char_p),
    "nv4_strerror": ([_I], ctypes.c_char_p),
}

_lib = None
_lock = threading.Lock()


class NV4LibraryError(RuntimeError):
    """libnv4.so is missing or does not load."""


def load():
    """Load libnv4.so once; raise NV4LibraryError when it is not there."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise NV4LibraryError(
                    f"{LIB_PATH} is missing: build the HIP library first "
                    "(make -C nano-vllm-int4_amd, or __graft_entry__.build())")
            try:
                lib = ctypes.CDLL(str(LIB_PATH))
            except OSError as exc:  # pragma: no cover - depends on the host
                raise NV4LibraryError(f"cannot load {LIB_PATH}: {exc}") from exc
            for name, (args, res) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = res
            _lib = lib
    return _lib


def strerror(code: int) -> str:
    return load().nv4_strerror(int(code)).decode()


def check(code: int, op: str) -> None:
    """Map an ABI return code to the exception the reference raises for it."""
    if code == NV4_OK:
        return
    if code < 0:
        raise ValueError(f"{op}: {strerror(code)} (nv4 code {code})")
    raise RuntimeError(f"{op}: HIP launch failed with hipError_t {code}")


def version() -> str:
    return load().nv4_version().decode()
