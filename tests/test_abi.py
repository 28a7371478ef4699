"""The C ABI of libnv4.so and the host-side argument checks (CPU only).

Every entry point declared in include/nv4.h is exported by the library and
bound by nv4._lib; invalid arguments are rejected with the documented
negative codes before anything is launched (so these calls need no GPU);
the Python wrappers raise the reference's exceptions (ValueError/TypeError,
nanovllm/kernels/*.py and nanovllm/layers/linear_w4a4.py) for the same
conditions.
"""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from nv4 import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "nv4.h"
P = ctypes.c_void_p
A16 = 0x10000  # a fake, 16-byte aligned device address: never dereferenced below


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|int64_t|void|const char\*)\s+(nv4_\w+)\(", text, re.M)))


def test_every_declared_symbol_is_exported_and_bound():
    names = declared()
    assert names, "no entry points parsed from nv4.h"
    lib = _lib.load()
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, n
    assert set(_lib.SIGNATURES) == set(names)
    assert _lib.version().startswith("nv4 ")


def test_error_text():
    assert _lib.strerror(_lib.NV4_OK) == "ok"
    for code in (_lib.NV4_E_NULL, _lib.NV4_E_SHAPE, _lib.NV4_E_ALIGN, _lib.NV4_E_LAYOUT, _lib.NV4_E_DTYPE,
                 _lib.NV4_E_GROUP):
        assert _lib.strerror(code) not in ("ok", "unknown error")
    assert _lib.strerror(7) == "hip error"


def test_rht_quant_pack_rejections():
    f = _lib.load().nv4_rht_quant_pack
    assert f(None, P(A16), P(A16), P(A16), 4, 4096, 0, None) == _lib.NV4_E_NULL
    assert f(P(A16), P(A16), P(A16), P(A16), 0, 4096, 0, None) == _lib.NV4_E_SHAPE
    assert f(P(A16 + 8), P(A16), P(A16), P(A16), 4, 4096, 0, None) == _lib.NV4_E_ALIGN
    assert f(P(A16), P(A16), P(A16), P(A16), 4, 2048, 0, None) == _lib.NV4_E_SHAPE
    assert f(P(A16), P(A16), P(A16), P(A16), 4, 100, 1, None) == _lib.NV4_E_SHAPE
    assert f(P(A16), P(A16), P(A16), P(A16), 4, 4096, 9, None) == _lib.NV4_E_LAYOUT


def test_w4a4_gemm_rejections():
    f = _lib.load().nv4_w4a4_gemm
    ok = [P(A16)] * 4
    assert f(None, *ok[1:], 1, P(A16), 0, 4, 64, 4096, None) == _lib.NV4_E_NULL
    assert f(*ok, 1, P(A16), 0, 4, 60, 4096, None) == _lib.NV4_E_SHAPE        # N % 8
    assert f(*ok, 1, P(A16), 0, 4, 64, 4000, None) == _lib.NV4_E_SHAPE       # K % 128
    assert f(*ok, 1, P(A16), 0, 0, 64, 4096, None) == _lib.NV4_E_SHAPE       # M = 0
    assert f(P(A16 + 4), *ok[1:], 1, P(A16), 0, 4, 64, 4096, None) == _lib.NV4_E_ALIGN
    assert f(*ok, 1, P(A16 + 2), 1, 4, 64, 4096, None) == _lib.NV4_E_ALIGN   # fp32 output


def test_w4a4_gemm_f8_rejections():
    f = _lib.load().nv4_w4a4_gemm_f8
    a = w = sa = sw = out = P(A16)
    M, N, K = 256, 64, 4096
    need = (M + N) * K

    def call(a=a, w=w, tiled=0, sa=sa, sw=sw, out=out, fp32=0, M=M, N=N, K=K, ws=P(A16), nbytes=need):
        return f(a, w, tiled, sa, sw, 1, out, fp32, M, N, K, ws, nbytes, None)

    assert call(ws=None) == _lib.NV4_E_NULL
    assert call(a=None) == _lib.NV4_E_NULL
    assert call(nbytes=need - 1) == _lib.NV4_E_SHAPE                     # workspace too small
    assert call(N=60) == _lib.NV4_E_SHAPE                                # N % 8
    assert call(N=40, tiled=1, nbytes=(M + 40) * K) == _lib.NV4_E_SHAPE  # tiled needs N % 16
    assert call(K=4000) == _lib.NV4_E_SHAPE                              # K % 128
    assert call(M=0) == _lib.NV4_E_SHAPE
    assert call(ws=P(A16 + 8)) == _lib.NV4_E_ALIGN
    assert call(a=P(A16 + 4)) == _lib.NV4_E_ALIGN
    assert call(out=P(A16 + 2), fp32=1) == _lib.NV4_E_ALIGN
    big = 1 << 27                                                        # M*K/32 beyond a 32-bit grid
    assert call(M=big, nbytes=(big + N) * K) == _lib.NV4_E_SHAPE


def test_w4a4_gemm_f6_rejections():
    lib = _lib.load()
    f, size = lib.nv4_w4a4_gemm_f6, lib.nv4_w4a4_gemm_f6_workspace
    a = w = sa = sw = out = P(A16)
    M, N, K = 256, 64, 4096
    need = size(M, N, K)
    assert need == (2 + 1) * 32 * 12288                                  # 128-row tiles x groups x 12 KiB
    assert size(300, 136, 1152) == (3 + 2) * 9 * 12288
    assert size(0, N, K) == -1 and size(M, N, 4000) == -1 and size(M, 0, K) == -1

    def call(a=a, w=w, tiled=0, sa=sa, sw=sw, out=out, fp32=0, M=M, N=N, K=K, ws=P(A16), nbytes=need):
        return f(a, w, tiled, sa, sw, 1, out, fp32, M, N, K, ws, nbytes, None)

    assert call(ws=None) == _lib.NV4_E_NULL
    assert call(sw=None) == _lib.NV4_E_NULL
    assert call(nbytes=need - 1) == _lib.NV4_E_SHAPE                     # workspace too small
    assert call(N=60) == _lib.NV4_E_SHAPE                                # N % 8
    assert call(N=40, tiled=1) == _lib.NV4_E_SHAPE                       # tiled needs N % 16
    assert call(K=4000) == _lib.NV4_E_SHAPE                              # K % 128
    assert call(M=0) == _lib.NV4_E_SHAPE
    assert call(K=1 << 21) == _lib.NV4_E_SHAPE                           # K beyond 2^20
    assert call(ws=P(A16 + 8)) == _lib.NV4_E_ALIGN
    assert call(w=P(A16 + 4)) == _lib.NV4_E_ALIGN
    assert call(out=P(A16 + 2), fp32=1) == _lib.NV4_E_ALIGN
    big = 1 << 26                                                        # conversion grid beyond 32 bits
    assert call(M=big, nbytes=size(big, N, K)) == _lib.NV4_E_SHAPE
    assert call(tiled=3) == _lib.NV4_E_SHAPE                             # weight forms are 0, 1 and 2
    assert call(tiled=-1) == _lib.NV4_E_SHAPE
    a_part = 2 * 32 * 12288                                              # fp6 weights: workspace for A only
    assert call(tiled=2, nbytes=a_part - 1) == _lib.NV4_E_SHAPE
    assert call(tiled=2, nbytes=a_part, w=P(A16 + 8)) == _lib.NV4_E_ALIGN


def test_w4a4_weights_to_f6_rejections():
    lib = _lib.load()
    f, size = lib.nv4_w4a4_weights_to_f6, lib.nv4_w4a4_weights_f6_bytes
    N, K = 200, 1024
    need = size(N, K)
    assert need == 2 * 8 * 12288                                         # 128-row tiles x groups x 12 KiB
    assert size(0, K) == -1 and size(N, 1000) == -1 and size(N, 0) == -1

    def call(w=P(A16), tiled=0, w6=P(A16), N=N, K=K, nbytes=need):
        return f(w, tiled, w6, N, K, nbytes, None)

    assert call(w=None) == _lib.NV4_E_NULL
    assert call(w6=None) == _lib.NV4_E_NULL
    assert call(nbytes=need - 1) == _lib.NV4_E_SHAPE
    assert call(N=204) == _lib.NV4_E_SHAPE                               # N % 8
    assert call(N=200, tiled=1) == _lib.NV4_E_SHAPE                      # tiled needs N % 16
    assert call(tiled=2) == _lib.NV4_E_SHAPE                             # source forms are 0 and 1
    assert call(K=1000) == _lib.NV4_E_SHAPE
    assert call(K=1 << 21) == _lib.NV4_E_SHAPE
    assert call(w=P(A16 + 8)) == _lib.NV4_E_ALIGN
    assert call(w6=P(A16 + 4)) == _lib.NV4_E_ALIGN


def test_prefill_attention_rejections():
    f = _lib.load().nv4_prefill_attention
    Hq, Hkv, D = 32, 8, 128

    def call(q=P(A16), qr=Hq * D, k=P(A16), kr=Hkv * D, v=P(A16), vr=Hkv * D, o=P(A16), orow=Hq * D, cu=P(A16),
             B=2, maxlen=100, hq=Hq, hkv=Hkv, d=D, scale=0.088):
        return f(q, qr, k, kr, v, vr, o, orow, cu, B, maxlen, hq, hkv, d, ctypes.c_float(scale), None)

    assert call(q=None) == _lib.NV4_E_NULL
    assert call(cu=None) == _lib.NV4_E_NULL
    assert call(d=64) == _lib.NV4_E_SHAPE                                # head dim 128 only
    assert call(hq=12, hkv=8) == _lib.NV4_E_SHAPE                        # Hq % Hkv
    assert call(hq=48, hkv=3) == _lib.NV4_E_SHAPE                        # group of 16
    assert call(B=0) == _lib.NV4_E_SHAPE
    assert call(maxlen=0) == _lib.NV4_E_SHAPE
    assert call(qr=Hq * D - 8) == _lib.NV4_E_SHAPE                       # row shorter than the heads
    assert call(scale=0.0) == _lib.NV4_E_SHAPE
    assert call(scale=-1.0) == _lib.NV4_E_SHAPE
    assert call(scale=float("nan")) == _lib.NV4_E_SHAPE
    assert call(kr=Hkv * D + 4) == _lib.NV4_E_ALIGN                     # row stride % 8
    assert call(v=P(A16 + 8)) == _lib.NV4_E_ALIGN
    assert call(cu=P(A16 + 2)) == _lib.NV4_E_ALIGN


def test_w4a16_and_linear_rejections():
    f = _lib.load().nv4_w4a16_gemm
    ok = [P(A16)] * 4
    assert f(P(A16), 7, P(A16), P(A16), P(A16), P(A16), 0, 4, 64, 4096, 128, None) == _lib.NV4_E_DTYPE
    assert f(P(A16), 0, P(A16), P(A16), P(A16), P(A16), 0, 4, 64, 4096, 64, None) == _lib.NV4_E_GROUP
    assert f(P(A16), 0, P(A16), P(A16), P(A16), P(A16), 0, 4, 60, 4096, 128, None) == _lib.NV4_E_SHAPE
    assert f(None, 0, *ok[:3], P(A16), 0, 4, 64, 4096, 128, None) == _lib.NV4_E_NULL
    d = _lib.load().nv4_w4a16_dequant
    # qweight, qzeros, scales, w, w_dtype, N, K, group
    assert d(None, P(A16), P(A16), P(A16), 0, 64, 4096, 128, None) == _lib.NV4_E_NULL
    assert d(P(A16), P(A16), P(A16), P(A16), 2, 64, 4096, 128, None) == _lib.NV4_E_DTYPE   # fp32 target
    assert d(P(A16), P(A16), P(A16), P(A16), 0, 64, 4096, 64, None) == _lib.NV4_E_GROUP
    assert d(P(A16), P(A16), P(A16), P(A16), 0, 60, 4096, 128, None) == _lib.NV4_E_SHAPE   # N % 8
    assert d(P(A16), P(A16), P(A16), P(A16), 0, 64, 4000, 128, None) == _lib.NV4_E_SHAPE   # K % 128
    assert d(P(A16), P(A16), P(A16 + 8), P(A16), 0, 64, 4096, 128, None) == _lib.NV4_E_ALIGN
    g = _lib.load().nv4_w4a4_linear
    assert g(*([P(A16)] * 7), 4, 64, 2048, None) == _lib.NV4_E_SHAPE
    assert g(None, *([P(A16)] * 6), 4, 64, 4096, None) == _lib.NV4_E_NULL
    assert g(*([P(A16)] * 7), 0, 64, 4096, None) == _lib.NV4_E_SHAPE


def test_paged_decode_attention_rejections():
    f = _lib.load().nv4_paged_decode_attention
    # q, q_row, k, v, block_tables, max_blocks, context_lens, out, ws, ws_bytes, B, Hq, Hkv, D, bs, max_ctx
    def call(q_row=4096, max_blocks=17, ws_bytes=1 << 30, B=32, Hq=32, Hkv=8, D=128, bs=256, max_ctx=4352,
             q=P(A16), ws=P(A16)):
        return f(q, q_row, P(A16), P(A16), P(A16), max_blocks, P(A16), P(A16), ws, ws_bytes, B, Hq, Hkv, D, bs,
                 max_ctx, 0.1, None)
    assert call(q=None) == _lib.NV4_E_NULL
    assert call(ws=None) == _lib.NV4_E_NULL
    assert call(D=64) == _lib.NV4_E_SHAPE
    assert call(Hkv=5) == _lib.NV4_E_SHAPE                    # Hq % Hkv
    assert call(Hq=64, q_row=8192) == _lib.NV4_E_SHAPE       # GQA group 8
    assert call(max_blocks=16) == _lib.NV4_E_SHAPE           # 16 blocks of 256 < 4352
    assert call(ws_bytes=1000) == _lib.NV4_E_SHAPE
    assert call(q_row=100) == _lib.NV4_E_SHAPE
    assert call(q=P(A16 + 4)) == _lib.NV4_E_ALIGN


def test_lm_head_rejections():
    f = _lib.load().nv4_lm_head
    def call(h=P(A16), w=P(A16), out=P(A16), h_row=4096, out_row=151936, M=32, N=151936, K=4096):
        return f(h, h_row, w, out, out_row, M, N, K, None)
    assert call(h=None) == _lib.NV4_E_NULL
    assert call(w=None) == _lib.NV4_E_NULL
    assert call(out=None) == _lib.NV4_E_NULL
    assert call(M=0) == _lib.NV4_E_SHAPE
    assert call(M=33) == _lib.NV4_E_SHAPE
    assert call(K=3072, h_row=3072) == _lib.NV4_E_SHAPE     # unsupported hidden size
    assert call(h_row=4000) == _lib.NV4_E_SHAPE             # rows narrower than K
    assert call(out_row=100) == _lib.NV4_E_SHAPE
    assert call(N=0) == _lib.NV4_E_SHAPE
    assert call(h=P(A16 + 8)) == _lib.NV4_E_ALIGN
    assert call(w=P(A16 + 2)) == _lib.NV4_E_ALIGN
    assert call(h_row=4100) == _lib.NV4_E_ALIGN


def test_paged_decode_attention_qkv_rejections():
    f = _lib.load().nv4_paged_decode_attention_qkv
    # qkv, row, qw, kw, cos_sin, max_pos, positions, slots, num_slots, k, v, block_tables, max_blocks,
    # context_lens, out, ws, ws_bytes, B, Hq, Hkv, D, bs, max_ctx, eps, scale, stream
    def call(row=6144, qw=P(A16), cs=P(A16), pos=P(A16), slots=P(A16), ws=P(A16), max_pos=4096, num_slots=1 << 20,
             ws_bytes=1 << 30, Hq=32, Hkv=8, max_ctx=4352, max_blocks=17):
        return f(P(A16), row, qw, P(A16), cs, max_pos, pos, slots, num_slots, P(A16), P(A16), P(A16), max_blocks,
                 P(A16), P(A16), ws, ws_bytes, 32, Hq, Hkv, 128, 256, max_ctx, 1e-6, 0.1, None)
    assert call(qw=None) == _lib.NV4_E_NULL
    assert call(cs=None) == _lib.NV4_E_NULL
    assert call(pos=None) == _lib.NV4_E_NULL
    assert call(slots=None) == _lib.NV4_E_NULL
    assert call(ws=None) == _lib.NV4_E_NULL
    assert call(row=4096 + 2048 - 8) == _lib.NV4_E_SHAPE      # row narrower than Hq + 2 Hkv heads
    assert call(max_pos=0) == _lib.NV4_E_SHAPE
    assert call(num_slots=-1) == _lib.NV4_E_SHAPE
    assert call(ws_bytes=1000) == _lib.NV4_E_SHAPE
    assert call(max_blocks=16) == _lib.NV4_E_SHAPE
    assert call(Hq=64, row=(64 + 16) * 128) == _lib.NV4_E_SHAPE  # GQA group 8
    assert call(cs=P(A16 + 2)) == _lib.NV4_E_ALIGN
    assert call(pos=P(A16 + 4)) == _lib.NV4_E_ALIGN
    assert call(qw=P(A16 + 1)) == _lib.NV4_E_ALIGN


def test_paged_decode_attention_size_checks_do_not_wrap():
    """Sizes at the accepted maxima whose workspace size does not fit in int64
    (B * Hq * splits * 130 * 4 ~ 2^65) are rejected -- NV4_E_SHAPE for the
    workspace form whatever workspace size is claimed, NV4_E_SCRATCH for the
    allocation-free form -- and block counts whose product with the block
    size would wrap are rejected as shapes."""
    lib = _lib.load()
    f, g = lib.nv4_paged_decode_attention, lib.nv4_paged_decode_attention_noalloc
    B, Hkv, Hq, D, bs, max_blocks, max_ctx = 65535, 65535, 4 * 65535, 128, 1 << 14, 1 << 16, 1 << 30
    args = (P(A16), Hq * D, P(A16), P(A16), P(A16), max_blocks, P(A16), P(A16))
    assert f(*args, P(A16), (1 << 62), B, Hq, Hkv, D, bs, max_ctx, 0.1, None) == _lib.NV4_E_SHAPE
    assert g(*args, B, Hq, Hkv, D, bs, max_ctx, 0.1, None) == _lib.NV4_E_SCRATCH
    # max_blocks * block_size = 2^33 * (2^31 + 1) wraps to 2^33 in int64 arithmetic
    wrap = (P(A16), 4096, P(A16), P(A16), P(A16), 1 << 33, P(A16), P(A16))
    assert f(*wrap, P(A16), 1 << 30, 32, 32, 8, 128, (1 << 31) + 1, 4352, 0.1, None) == _lib.NV4_E_SHAPE
    assert g(*wrap, 32, 32, 8, 128, (1 << 31) + 1, 4352, 0.1, None) == _lib.NV4_E_SHAPE


def test_prefetch_size_rule():
    f = _lib.load().nv4_w4a4_prefetch_bytes
    assert f(4096, 12288) == 4096 * 6144           # down: all of its weights
    assert f(4096, 4096) == 4096 * 2048             # o (8 MiB): all of it
    assert f(6144, 4096) == 6 << 20                 # qkv (12 MiB): the first 6 MiB
    assert f(24576, 4096) == 9 << 20                # gate_up (48 MiB): the first 9 MiB
    assert f(16, 256) == 16 * 128
    assert f(0, 4096) == 0 and f(64, 100) == 0


def test_rowtiled_entry_point_rejections():
    lib = _lib.load()
    ok = [P(A16)] * 4
    g = lib.nv4_w4a4_gemm_rowtiled
    assert g(None, *ok[1:], 1, P(A16), 0, 4, 64, 4096, None) == _lib.NV4_E_NULL
    assert g(*ok, 1, P(A16), 0, 33, 64, 4096, None) == _lib.NV4_E_SHAPE    # M > 32
    assert g(*ok, 1, P(A16), 0, 0, 64, 4096, None) == _lib.NV4_E_SHAPE     # M = 0
    assert g(*ok, 1, P(A16), 0, 4, 72, 4096, None) == _lib.NV4_E_SHAPE     # N % 16
    assert g(*ok, 1, P(A16), 0, 4, 64, 4000, None) == _lib.NV4_E_SHAPE     # K % 128
    assert g(P(A16 + 8), *ok[1:], 1, P(A16), 0, 4, 64, 4096, None) == _lib.NV4_E_ALIGN
    k = lib.nv4_rht_quant_pack_rowtiled
    assert k(None, P(A16), P(A16), P(A16), 4, 4096, None, 0, None) == _lib.NV4_E_NULL
    assert k(P(A16), P(A16), P(A16), P(A16), 4, 2048, None, 0, None) == _lib.NV4_E_SHAPE
    assert k(P(A16), P(A16), P(A16), P(A16), 0, 4096, None, 0, None) == _lib.NV4_E_SHAPE
    # prefetch arguments: a buffer with a positive multiple of 16 bytes, 16-byte aligned
    assert k(P(A16), P(A16), P(A16), P(A16), 4, 4096, None, 4096, None) == _lib.NV4_E_NULL
    assert k(P(A16), P(A16), P(A16), P(A16), 4, 4096, P(A16), 100, None) == _lib.NV4_E_SHAPE
    assert k(P(A16), P(A16), P(A16), P(A16), 4, 4096, P(A16), -16, None) == _lib.NV4_E_SHAPE
    assert k(P(A16), P(A16), P(A16), P(A16), 4, 4096, P(A16 + 8), 4096, None) == _lib.NV4_E_ALIGN
    lin = lib.nv4_w4a4_linear_rowtiled
    assert lin(*([P(A16)] * 7), 33, 64, 4096, None) == _lib.NV4_E_SHAPE
    assert lin(*([P(A16)] * 7), 4, 72, 4096, None) == _lib.NV4_E_SHAPE
    assert lin(*([P(A16)] * 7), 4, 64, 2048, None) == _lib.NV4_E_SHAPE
    r = lib.nv4_rmsnorm_rht_quant_pack_rowtiled
    assert r(P(A16), None, None, P(A16), 1e-6, P(A16), P(A16), P(A16), 4, 12288, None, 0, None) == _lib.NV4_E_SHAPE
    assert r(P(A16), None, None, P(A16), 1e-6, P(A16), P(A16), P(A16), 4, 4096, P(A16), 24, None) == _lib.NV4_E_SHAPE
    sm = lib.nv4_silu_mul_rht_quant_pack_rowtiled
    assert sm(P(A16), P(A16), P(A16), P(A16), 4, 2048, None, 0, None) == _lib.NV4_E_SHAPE
    assert sm(P(A16), P(A16), P(A16), P(A16), 4, 4096, None, 32, None) == _lib.NV4_E_NULL
    gs = lib.nv4_w4a4_gemm_rowtiled_silu
    assert gs(None, *ok[1:], 1, P(A16), 4, 24576, 4096, None) == _lib.NV4_E_NULL
    assert gs(*ok, 1, P(A16), 33, 24576, 4096, None) == _lib.NV4_E_SHAPE      # M > 32
    assert gs(*ok, 1, P(A16), 4, 24592, 4096, None) == _lib.NV4_E_SHAPE      # N % 32
    assert gs(*ok, 1, P(A16), 4, 24576, 4224, None) == _lib.NV4_E_SHAPE      # K % 256
    assert gs(*ok, 1, P(A16), 4, 4096, 4096, None) == _lib.NV4_E_SHAPE       # fewer than 4 blocks per CU


def test_gumbel_split_rejections():
    lib = _lib.load()
    assert lib.nv4_gumbel_sample_chunks(32, 151936) == 64     # 2048 workgroups over 32 rows
    assert lib.nv4_gumbel_sample_chunks(1, 37) == 1
    f = lib.nv4_gumbel_sample_ws
    def call(ws=P(A16), ws_bytes=1 << 20, B=32, V=151936, dtype=0, logits=P(A16)):
        return f(logits, V, dtype, P(A16), B, V, 1, 0, ws, ws_bytes, P(A16), None)
    assert call(ws=None) == _lib.NV4_E_NULL
    assert call(ws_bytes=8 * 32 * 64 - 1) == _lib.NV4_E_SHAPE
    assert call(B=70000) == _lib.NV4_E_SHAPE
    assert call(dtype=1) == _lib.NV4_E_DTYPE
    assert call(ws=P(A16 + 2)) == _lib.NV4_E_ALIGN


def test_decoder_ops_rejections():
    lib = _lib.load()
    rms = lib.nv4_rmsnorm
    assert rms(None, None, None, P(A16), P(A16), 4, 4096, 1e-6, None) == _lib.NV4_E_NULL
    assert rms(P(A16), P(A16), None, P(A16), P(A16), 4, 4096, 1e-6, None) == _lib.NV4_E_NULL  # residual pair
    assert rms(P(A16), None, None, P(A16), P(A16), 4, 4104, 1e-6, None) == _lib.NV4_E_SHAPE   # H % 16
    assert rms(P(A16), None, None, P(A16), P(A16), 4, 16384, 1e-6, None) == _lib.NV4_E_SHAPE  # H > 8192
    assert rms(P(A16), None, None, P(A16), P(A16), 0, 4096, 1e-6, None) == _lib.NV4_E_SHAPE
    assert rms(P(A16 + 2), None, None, P(A16), P(A16), 4, 4096, 1e-6, None) == _lib.NV4_E_ALIGN
    qk = lib.nv4_qk_norm_rope_store
    def call(qkv=P(A16), row=6144, T=4, Hq=32, Hkv=8, max_pos=4096, num_slots=1024):
        return qk(qkv, row, T, Hq, Hkv, P(A16), P(A16), P(A16), max_pos, P(A16), P(A16), num_slots, P(A16),
                  P(A16), P(A16), None, None, 1e-6, None)
    assert call(qkv=None) == _lib.NV4_E_NULL
    assert call(row=6000) == _lib.NV4_E_SHAPE
    assert call(T=0) == _lib.NV4_E_SHAPE
    assert call(max_pos=0) == _lib.NV4_E_SHAPE
    assert call(row=6146) == _lib.NV4_E_ALIGN                            # 8-byte row accesses
    assert call(qkv=P(A16 + 4)) == _lib.NV4_E_ALIGN
    silu = lib.nv4_silu_mul
    assert silu(None, P(A16), 4, 12288, None) == _lib.NV4_E_NULL
    assert silu(P(A16), P(A16), 4, 12, None) == _lib.NV4_E_SHAPE
    assert silu(P(A16 + 8), P(A16), 4, 12288, None) == _lib.NV4_E_ALIGN
    rq = lib.nv4_rmsnorm_rht_quant_pack
    def rcall(x=P(A16), ri=None, ro=None, K=4096, M=4, sgn=P(A16)):
        return rq(x, ri, ro, P(A16), 1e-6, sgn, P(A16), P(A16), M, K, None)
    assert rcall(x=None) == _lib.NV4_E_NULL
    assert rcall(ri=P(A16)) == _lib.NV4_E_NULL                   # residual pair
    assert rcall(K=12288) == _lib.NV4_E_SHAPE
    assert rcall(M=0) == _lib.NV4_E_SHAPE
    assert rcall(sgn=P(A16 + 1)) == _lib.NV4_E_ALIGN
    sq = lib.nv4_silu_mul_rht_quant_pack
    assert sq(None, P(A16), P(A16), P(A16), 4, 12288, None) == _lib.NV4_E_NULL
    assert sq(P(A16), P(A16), P(A16), P(A16), 4, 8192, None) == _lib.NV4_E_SHAPE
    assert sq(P(A16 + 2), P(A16), P(A16), P(A16), 4, 12288, None) == _lib.NV4_E_ALIGN


def test_probe_rejections():
    lib = _lib.load()
    sink = P(A16)
    assert lib.nv4_probe_mfma(0, 10, 8, None, None) == _lib.NV4_E_NULL
    assert lib.nv4_probe_bf16_rne(None, None) == _lib.NV4_E_NULL
    assert lib.nv4_probe_mfma(3, 10, 8, sink, None) == _lib.NV4_E_SHAPE        # unknown kind
    assert lib.nv4_probe_mfma(-1, 10, 8, sink, None) == _lib.NV4_E_SHAPE
    assert lib.nv4_probe_mfma(1, 0, 8, sink, None) == _lib.NV4_E_SHAPE         # no rounds
    assert lib.nv4_probe_mfma(0, 10, 0, sink, None) == _lib.NV4_E_SHAPE        # no workgroups
    assert lib.nv4_probe_mfma(0, 10, (1 << 20) + 1, sink, None) == _lib.NV4_E_SHAPE
    assert lib.nv4_probe_read(None, 65536, sink, None) == _lib.NV4_E_NULL
    assert lib.nv4_probe_read(P(A16), 65536 + 16, sink, None) == _lib.NV4_E_SHAPE  # not whole 64 KiB chunks
    assert lib.nv4_probe_read(P(A16), 0, sink, None) == _lib.NV4_E_SHAPE
    assert lib.nv4_probe_read(P(A16 + 8), 65536, sink, None) == _lib.NV4_E_ALIGN


def test_python_wrappers_validate_like_the_reference():
    from nv4 import W4A4Linear, rht_quant_pack, w4a4_grouped_gemm
    x = torch.zeros(2, 4096, dtype=torch.bfloat16)
    signs = torch.ones(4096, dtype=torch.int8)
    with pytest.raises(ValueError):
        rht_quant_pack(x.float(), signs, out_packed=torch.empty(2, 2048, dtype=torch.int8),
                       out_scale=torch.empty(2, 32, dtype=torch.bfloat16))
    with pytest.raises(ValueError):  # CPU tensors: the reference requires CUDA tensors
        rht_quant_pack(x, signs, out_packed=torch.empty(2, 2048, dtype=torch.int8),
                       out_scale=torch.empty(2, 32, dtype=torch.bfloat16))
    a = torch.zeros(2, 2048, dtype=torch.int8)
    w = torch.zeros(64, 2048, dtype=torch.int8)
    sa = torch.zeros(2, 32, dtype=torch.bfloat16)
    sw = torch.zeros(64, 32, dtype=torch.bfloat16)
    with pytest.raises(TypeError):
        w4a4_grouped_gemm(a.to(torch.int16), w, sa, sw)
    with pytest.raises(TypeError):
        w4a4_grouped_gemm(a, w, sa.float(), sw)
    with pytest.raises(ValueError):
        w4a4_grouped_gemm(a, torch.zeros(60, 2048, dtype=torch.int8), sa, sw[:60])
    with pytest.raises(ValueError):
        w4a4_grouped_gemm(a, w, sa, sw)  # CPU tensors
    for kwargs in ({"bias": True}, {}):
        with pytest.raises(ValueError):
            W4A4Linear(1000 if not kwargs else 4096, 64, **kwargs)
    with pytest.raises(ValueError):
        W4A4Linear(4096, 60)
    m = W4A4Linear(4096, 64)
    assert {k: (tuple(v.shape), v.dtype) for k, v in m.state_dict().items()} == {
        "packed_weight": ((64, 2048), torch.int8), "weight_scale": ((64, 32), torch.bfloat16),
        "signs": ((4096,), torch.int8)}
