"""GPU parity of the matrix-core forms of K2 for prefill-sized M:
``nv4_w4a4_gemm_f6`` (INT4 codes as fp6 e3m2 values, the size-chosen kernel)
and ``nv4_w4a4_gemm_f8`` (codes as fp8 e4m3 values).

The grouped W4A4 GEMM of nanovllm/kernels/w4a4_grouped_kernel.py:64-90 for
prefill-sized M: results must equal the oracle
(benchmarks/verify_w4a4_aw_grouped.py:13-29) bit for bit, like every other K2
path.  Covers the reference shapes, tails in M and N (partial 128-row tiles),
K from one group (no scale windows) to 12288, scale pointers that rule the
windows out, both weight layouts, both weight-scale forms, bf16 and fp32
outputs, the extreme scales of the int8 prefill test (bf16 subnormals, tiny
normals, 2^70, zeros: the scale product is formed on the matrix cores and
must still be the exact fp32 product), repeated calls on one workspace,
full-matrix equality with the int8 path at Qwen3-8B projection shapes, and
weights converted to fp6 once (``weights_to_f6``) instead of per call.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from conftest import bf16_bits
from nv4 import _lib, compile_grouped_gemm, tile_weights, w4a4_grouped_gemm, weights_to_f6
from test_gpu_w4a4 import assert_bits_equal, extreme_scales, gemm_inputs, to_dev

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
PATHS = ["fp6", "fp8"]


def check_against_oracle(ap, wp, sa, sw, M, N, K, what, path):
    grouped = sw.ndim == 2
    a, w, s_a, s_w = to_dev(ap, wp, sa, sw)
    exp16 = oracle.w4a4_gemm(ap, wp, sa, sw)
    exp32 = oracle.w4a4_gemm(ap, wp, sa, sw, out_fp32=True)
    storage = torch.full((M * N + 128,), -1234, device=DEV, dtype=torch.bfloat16)
    sentinel = storage[:64].clone()
    out = storage[64:-64].view(M, N)
    for rep in range(2):
        out.fill_(float("nan"))
        w4a4_grouped_gemm(a, w, s_a, s_w, out=out, path=path)
        torch.cuda.synchronize()
        assert_bits_equal(bf16_bits(out), exp16, f"{what}: bf16 output (call {rep})")
        assert torch.equal(storage[:64], sentinel) and torch.equal(storage[-64:], sentinel)
    out32 = torch.full((M, N), float("nan"), device=DEV, dtype=torch.float32)
    compile_grouped_gemm(M, N, K, output_fp32=True, weight_grouped=grouped, path=path)(a, w, s_a, s_w, out32)
    torch.cuda.synchronize()
    assert_bits_equal(out32.cpu().numpy().view(np.uint32), exp32.view(np.uint32), f"{what}: fp32 output")
    if N % 16 == 0:
        out.fill_(float("nan"))
        w4a4_grouped_gemm(a, tile_weights(w), s_a, s_w, out=out, weights_tiled=True, path=path)
        torch.cuda.synchronize()
        assert_bits_equal(bf16_bits(out), exp16, f"{what}: bf16 output, tiled weights")


@pytest.mark.parametrize("M,N,K", [(17, 96, 512), (33, 136, 4096), (32, 128, 12288), (1, 8, 128), (129, 24, 384),
                                   (200, 264, 1024), (257, 392, 2048), (300, 16, 1152), (128, 128, 8192),
                                   (600, 264, 1024), (513, 136, 2048), (1030, 24, 3072)])
@pytest.mark.parametrize("grouped", [True, False])
@pytest.mark.parametrize("path", PATHS)
def test_matches_oracle(M, N, K, grouped, path):
    print(f"[{path}] M={M} N={N} K={K} grouped={grouped}", flush=True)
    ap, wp, sa, sw = gemm_inputs(M, N, K, M * 3 + N + K)
    if not grouped:
        sw = sw[:, 0].copy()
    check_against_oracle(ap, wp, sa, sw, M, N, K, f"{path} M={M} N={N} K={K}", path)


@pytest.mark.parametrize("path", PATHS)
def test_scales_without_windows(path):
    """Scale tensors 2 bytes off a 16-byte boundary: the kernel reads each
    group's scales on its own instead of 8-group windows."""
    M, N, K = 160, 144, 2048
    print(f"[{path}-unaligned-scales] M={M} N={N} K={K}", flush=True)
    ap, wp, sa, sw = gemm_inputs(M, N, K, 99)
    exp = oracle.w4a4_gemm(ap, wp, sa, sw)
    a, w, s_a, s_w = to_dev(ap, wp, sa, sw)
    sa_buf = torch.empty(M * (K // 128) + 1, dtype=torch.bfloat16, device=DEV)
    sw_buf = torch.empty(N * (K // 128) + 1, dtype=torch.bfloat16, device=DEV)
    s_a2 = sa_buf[1:].view(M, K // 128)
    s_w2 = sw_buf[1:].view(N, K // 128)
    s_a2.copy_(s_a)
    s_w2.copy_(s_w)
    out = w4a4_grouped_gemm(a, w, s_a2, s_w2, path=path)
    torch.cuda.synchronize()
    assert_bits_equal(bf16_bits(out), exp, "bf16 output, unaligned scales")


@pytest.mark.parametrize("M,N,K,rows_special", [(200, 264, 1024, True), (257, 392, 2048, False),
                                                 (150, 136, 12288, True), (130, 400, 1024, False),
                                                 (700, 264, 1024, True), (520, 400, 2048, False)])
@pytest.mark.parametrize("path", PATHS)
def test_extreme_scales(M, N, K, rows_special, path):
    print(f"[{path}-extreme] M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M * 7 + K)
    ap, wp, _, _ = gemm_inputs(M, N, K, M + N + K)
    G = K // 128
    sa = oracle.f32_to_bf16((rng.random((M, G)) * 2 + 0.01).astype(np.float32))
    sw = oracle.f32_to_bf16((rng.random((N, G)) * 0.03 + 0.001).astype(np.float32))
    if rows_special:
        sa[130:] = extreme_scales(rng, M - 130, G)
    else:
        sw[:128] = extreme_scales(rng, 128, G)
    check_against_oracle(ap, wp, sa, sw, M, N, K, f"{path} extreme M={M} N={N} K={K}", path)


@pytest.mark.parametrize("M,N,K", [(1024, 6144, 4096), (2048, 4096, 4096), (4097, 24576, 4096),
                                   (1100, 4096, 12288)])
def test_equals_int8_path(M, N, K):
    """Full-matrix equality of both matrix-core forms with the int8 prefill
    kernel (itself pinned to the oracle) at projection shapes, random packed
    bytes, tiled and reference weight layouts."""
    print(f"[mc-vs-int8] M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=DEV)
    g.manual_seed(M + N + K)
    a = torch.randint(-128, 128, (M, K // 2), generator=g, device=DEV, dtype=torch.int16).to(torch.int8)
    w = torch.randint(-128, 128, (N, K // 2), generator=g, device=DEV, dtype=torch.int16).to(torch.int8)
    sa = (0.01 + torch.rand(M, K // 128, generator=g, device=DEV)).to(torch.bfloat16)
    sw = (0.005 + 0.015 * torch.rand(N, K // 128, generator=g, device=DEV)).to(torch.bfloat16)
    wt = tile_weights(w)
    o8 = w4a4_grouped_gemm(a, wt, sa, sw, weights_tiled=True, path="int8")
    for path in PATHS:
        of = w4a4_grouped_gemm(a, wt, sa, sw, weights_tiled=True, path=path)
        torch.cuda.synchronize()
        assert torch.equal(o8.view(torch.int16), of.view(torch.int16)), f"{path}, tiled weights"
    of = w4a4_grouped_gemm(a, w, sa, sw, path="fp6")
    torch.cuda.synchronize()
    assert torch.equal(o8.view(torch.int16), of.view(torch.int16)), "fp6, reference weight layout"


@pytest.mark.parametrize("path", PATHS)
def test_workspace_reused_smaller_call(path):
    """Two calls in a row on one workspace, the second smaller: each result
    equals the oracle (the workspace holds nothing that carries over)."""
    lib = _lib.load()
    fn = lib.nv4_w4a4_gemm_f6 if path == "fp6" else lib.nv4_w4a4_gemm_f8
    size = (lambda M, N, K: lib.nv4_w4a4_gemm_f6_workspace(M, N, K)) if path == "fp6" else (lambda M, N, K: (M + N) * K)
    ws = torch.empty(size(300, 264, 2048), dtype=torch.uint8, device=DEV)
    for (M, N, K) in [(300, 264, 2048), (70, 136, 1024)]:
        print(f"[{path}-ws] M={M} N={N} K={K}", flush=True)
        ap, wp, sa, sw = gemm_inputs(M, N, K, M + K)
        exp = oracle.w4a4_gemm(ap, wp, sa, sw)
        a, w, s_a, s_w = to_dev(ap, wp, sa, sw)
        out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
        P = lambda t: ctypes.c_void_p(t.data_ptr())
        rc = fn(P(a), P(w), 0, P(s_a), P(s_w), 1, P(out), 0, M, N, K, P(ws), ws.numel(),
                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        _lib.check(rc, f"w4a4 gemm {path}")
        torch.cuda.synchronize()
        assert_bits_equal(bf16_bits(out), exp, f"{path} workspace call M={M}")


@pytest.mark.parametrize("M,N,K", [(17, 96, 512), (300, 264, 2048), (129, 24, 384), (1030, 136, 3072),
                                   (257, 392, 12288)])
@pytest.mark.parametrize("grouped", [True, False])
def test_prepared_fp6_weights(M, N, K, grouped):
    """Weights converted once by ``weights_to_f6``: the blocks equal the W half
    of the per-call conversion (from either weight layout), the fp6 GEMM on
    them gives the oracle's bits (bf16 and fp32 outputs, a workspace for A
    only), and the calls leave them unchanged."""
    print(f"[fp6-prepared] M={M} N={N} K={K} grouped={grouped}", flush=True)
    lib = _lib.load()
    ap, wp, sa, sw = gemm_inputs(M, N, K, 5 * M + N + K)
    if not grouped:
        sw = sw[:, 0].copy()
    exp16 = oracle.w4a4_gemm(ap, wp, sa, sw)
    exp32 = oracle.w4a4_gemm(ap, wp, sa, sw, out_fp32=True)
    a, w, s_a, s_w = to_dev(ap, wp, sa, sw)
    w6 = weights_to_f6(w)
    if N % 16 == 0:
        assert torch.equal(weights_to_f6(tile_weights(w), True), w6), "tiled source"
    a_part = (M + 127) // 128 * (K // 128) * 12288
    ws = torch.full((lib.nv4_w4a4_gemm_f6_workspace(M, N, K),), 7, dtype=torch.uint8, device=DEV)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    sg = 1 if grouped else 0
    out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    _lib.check(lib.nv4_w4a4_gemm_f6(P(a), P(w), 0, P(s_a), P(s_w), sg, P(out), 0, M, N, K, P(ws), ws.numel(), st),
               "fp6 gemm, per-call conversion")
    torch.cuda.synchronize()
    assert torch.equal(ws[a_part:], w6), "W half of the per-call conversion"
    keep = w6.clone()
    ws_a = torch.empty(a_part, dtype=torch.uint8, device=DEV)
    for fp32 in (0, 1):
        o = torch.full((M, N), float("nan"), dtype=torch.float32 if fp32 else torch.bfloat16, device=DEV)
        _lib.check(lib.nv4_w4a4_gemm_f6(P(a), P(w6), 2, P(s_a), P(s_w), sg, P(o), fp32, M, N, K, P(ws_a), a_part,
                                        st), "fp6 gemm, prepared weights")
        torch.cuda.synchronize()
        if fp32:
            assert_bits_equal(o.cpu().numpy().view(np.uint32), exp32.view(np.uint32), "fp32 output")
        else:
            assert_bits_equal(bf16_bits(o), exp16, "bf16 output")
    o = w4a4_grouped_gemm(a, w, s_a, s_w, path="fp6", weights_f6=w6)
    torch.cuda.synchronize()
    assert_bits_equal(bf16_bits(o), exp16, "w4a4_grouped_gemm(weights_f6=...)")
    assert torch.equal(w6, keep), "prepared weights unchanged"
    with pytest.raises(ValueError):
        w4a4_grouped_gemm(a, w, s_a, s_w, path="fp6", weights_f6=w6[:-16])
