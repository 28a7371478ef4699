"""Writes the golden fixtures of tests/golden/ from the CPU oracle.

The fixtures are small seeded cases of every kernel contract, so that the
oracle (CPU tests) and the HIP kernels (GPU tests) can both be checked
against committed data: K1 on the reference's special rows for K = 4096 and
12288 (reference and block128 layouts), the grouped GEMM at the reference's
own test shape (benchmarks/verify_w4a4_aw_grouped.py: M=17, N=96, K=512, with
a zero row, zeroed scale stripes, bf16 and fp32 outputs, grouped and
per-channel weight scales), the W4A4 linear chain at K = 4096, and the W4A16
GEMM (fp16 and bf16 activations).  Run from the repository root:

    python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "nano-vllm-int4_amd")]

import oracle  # noqa: E402
from nv4 import workloads as W  # noqa: E402

OUT = Path(__file__).resolve().parent


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def k1_fixture(K, m=8):
    x = bits(W.special_rows(m, K))
    s = W.signs(K, W.BASE_SEED + 100 + K).numpy()
    p, sc = oracle.rht_quant_pack(x, s)
    p128, sc128 = oracle.rht_quant_pack(x, s, layout=oracle.LAYOUT_BLOCK128)
    np.savez_compressed(OUT / f"k1_k{K}.npz", x=x, signs=s, packed=p, scale=sc, packed128=p128, scale128=sc128)


def gemm_fixture(M=17, N=96, K=512, seed=20261110):
    rng = np.random.default_rng(seed)
    qa = rng.integers(-8, 8, (M, K)).astype(np.int8)
    qw = rng.integers(-8, 8, (N, K)).astype(np.int8)
    qa[0] = 0
    qw[0] = 0
    sa = oracle.f32_to_bf16((rng.random((M, K // 128)) * 2).astype(np.float32))
    sw = oracle.f32_to_bf16((rng.random((N, K // 128)) * .03).astype(np.float32))
    sa[1, ::2] = 0
    sw[1, 1::2] = 0
    a, w = oracle.pack_int4(qa), oracle.pack_int4(qw)
    sw1 = sw[:, 0].copy()
    np.savez_compressed(OUT / "k2_m17_n96_k512.npz", a=a, w=w, sa=sa, sw=sw, sw1=sw1,
                        out=oracle.w4a4_gemm(a, w, sa, sw), out_f32=oracle.w4a4_gemm(a, w, sa, sw, out_fp32=True),
                        out1=oracle.w4a4_gemm(a, w, sa, sw1),
                        out1_f32=oracle.w4a4_gemm(a, w, sa, sw1, out_fp32=True))


def chain_fixture(M=5, N=64, K=4096):
    x = bits(W.activations(M, K, W.BASE_SEED + 200))
    s = W.signs(K, W.BASE_SEED + 201).numpy()
    wp, sw = W.w4a4_weights(N, K, W.BASE_SEED + 203, W.BASE_SEED + 204)
    p, sc = oracle.rht_quant_pack(x, s)
    np.savez_compressed(OUT / "chain_m5_n64_k4096.npz", x=x, signs=s, w=wp.numpy(), sw=bits(sw),
                        packed=p, scale=sc, out=oracle.w4a4_gemm(p, wp.numpy(), sc, bits(sw)))


def w4a16_fixture(M=3, N=64, K=256):
    case = W.w4a16_case(M, N=N, K=K, seed=W.BASE_SEED + 300)
    xb = case.x.to(torch.bfloat16)
    arrays = dict(qweight=case.qweight.numpy(), qzeros=case.qzeros.numpy(),
                  scales=case.scales.numpy().view(np.uint16), x_f16=bits(case.x), x_bf16=bits(xb))
    arrays["out_f16"] = oracle.w4a16_gemm(arrays["x_f16"], arrays["qweight"], arrays["qzeros"], arrays["scales"],
                                          x_dtype=oracle.X_FP16)
    arrays["out_bf16"] = oracle.w4a16_gemm(arrays["x_bf16"], arrays["qweight"], arrays["qzeros"], arrays["scales"],
                                           x_dtype=oracle.X_BF16)
    np.savez_compressed(OUT / "w4a16_m3_n64_k256.npz", **arrays)


if __name__ == "__main__":
    k1_fixture(4096)
    k1_fixture(12288)
    gemm_fixture()
    chain_fixture()
    w4a16_fixture()
    for f in sorted(OUT.glob("*.npz")):
        print(f.name, f.stat().st_size)
