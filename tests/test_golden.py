"""The committed golden fixtures (tests/golden/, written by make_golden.py).

CPU: the oracle reproduces every fixture bit for bit, so a change to the
oracle cannot go unnoticed.  GPU: the HIP kernels reproduce them -- K1 codes
and scales (reference and block128 layouts, the reference's special rows),
the grouped GEMM in bf16 and fp32 with grouped and per-channel weight scales,
the W4A4 linear chain, and the W4A16 GEMM within 1e-2 relative.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from conftest import bits_to_bf16, bf16_bits

G = Path(__file__).resolve().parent / "golden"
DEV = "cuda:0"


def load(name):
    with np.load(G / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ------------------------------------------------------------------ oracle
@pytest.mark.parametrize("K", [4096, 12288])
def test_oracle_k1_fixture(K):
    f = load(f"k1_k{K}.npz")
    p, s = oracle.rht_quant_pack(f["x"], f["signs"])
    assert np.array_equal(p, f["packed"]) and np.array_equal(s, f["scale"])
    p, s = oracle.rht_quant_pack(f["x"], f["signs"], layout=oracle.LAYOUT_BLOCK128)
    assert np.array_equal(p, f["packed128"]) and np.array_equal(s, f["scale128"])


def test_oracle_gemm_fixture():
    f = load("k2_m17_n96_k512.npz")
    assert np.array_equal(oracle.w4a4_gemm(f["a"], f["w"], f["sa"], f["sw"]), f["out"])
    assert np.array_equal(oracle.w4a4_gemm(f["a"], f["w"], f["sa"], f["sw"], out_fp32=True).view(np.uint32),
                          f["out_f32"].view(np.uint32))
    assert np.array_equal(oracle.w4a4_gemm(f["a"], f["w"], f["sa"], f["sw1"]), f["out1"])


def test_oracle_chain_and_w4a16_fixtures():
    f = load("chain_m5_n64_k4096.npz")
    p, s = oracle.rht_quant_pack(f["x"], f["signs"])
    assert np.array_equal(p, f["packed"]) and np.array_equal(s, f["scale"])
    assert np.array_equal(oracle.w4a4_gemm(p, f["w"], s, f["sw"]), f["out"])
    f = load("w4a16_m3_n64_k256.npz")
    for xd, key in ((oracle.X_FP16, "f16"), (oracle.X_BF16, "bf16")):
        got = oracle.w4a16_gemm(f[f"x_{key}"], f["qweight"], f["qzeros"], f["scales"], x_dtype=xd)
        assert np.array_equal(got, f[f"out_{key}"])


# ------------------------------------------------------------------ kernels
@pytest.mark.gpu
@pytest.mark.parametrize("K", [4096, 12288])
def test_gpu_k1_fixture(K):
    from nv4 import rht_quant_pack
    f = load(f"k1_k{K}.npz")
    m = f["x"].shape[0]
    x = bits_to_bf16(f["x"]).to(DEV)
    s = torch.from_numpy(f["signs"]).to(DEV)
    for layout, pk, sk in (("reference", "packed", "scale"), ("block128", "packed128", "scale128")):
        packed = torch.empty((m, K // 2), dtype=torch.int8, device=DEV)
        scale = torch.empty((m, K // 128), dtype=torch.bfloat16, device=DEV)
        rht_quant_pack(x, s, out_packed=packed, out_scale=scale, layout=layout)
        torch.cuda.synchronize()
        assert np.array_equal(packed.cpu().numpy(), f[pk]), layout
        assert np.array_equal(bf16_bits(scale), f[sk]), layout


@pytest.mark.gpu
def test_gpu_gemm_fixture():
    from nv4 import compile_grouped_gemm, w4a4_grouped_gemm
    f = load("k2_m17_n96_k512.npz")
    a, w = torch.from_numpy(f["a"]).to(DEV), torch.from_numpy(f["w"]).to(DEV)
    sa, sw, sw1 = (bits_to_bf16(f[k]).to(DEV) for k in ("sa", "sw", "sw1"))
    assert np.array_equal(bf16_bits(w4a4_grouped_gemm(a, w, sa, sw)), f["out"])
    assert np.array_equal(bf16_bits(w4a4_grouped_gemm(a, w, sa, sw1)), f["out1"])
    M, N, K = a.shape[0], w.shape[0], a.shape[1] * 2
    for sws, key, grouped in ((sw, "out_f32", True), (sw1, "out1_f32", False)):
        out = torch.empty((M, N), dtype=torch.float32, device=DEV)
        compile_grouped_gemm(M, N, K, output_fp32=True, weight_grouped=grouped)(a, w, sa, sws, out)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), f[key].view(np.uint32)), key


@pytest.mark.gpu
def test_gpu_chain_fixture():
    from nv4 import w4a4_linear
    f = load("chain_m5_n64_k4096.npz")
    x = bits_to_bf16(f["x"]).to(DEV)
    packed = torch.empty(f["packed"].shape, dtype=torch.int8, device=DEV)
    scale = torch.empty(f["scale"].shape, dtype=torch.bfloat16, device=DEV)
    out = w4a4_linear(x, torch.from_numpy(f["signs"]).to(DEV), torch.from_numpy(f["w"]).to(DEV),
                      bits_to_bf16(f["sw"]).to(DEV), out_packed=packed, out_scale=scale)
    torch.cuda.synchronize()
    assert np.array_equal(packed.cpu().numpy(), f["packed"])
    assert np.array_equal(bf16_bits(scale), f["scale"])
    assert np.array_equal(bf16_bits(out), f["out"])


@pytest.mark.gpu
def test_gpu_w4a16_fixture():
    from nv4 import dequant_matmul_w4a16
    f = load("w4a16_m3_n64_k256.npz")
    qw, qz = torch.from_numpy(f["qweight"]).to(DEV), torch.from_numpy(f["qzeros"]).to(DEV)
    sc = torch.from_numpy(f["scales"].view(np.int16)).view(torch.float16).to(DEV)
    for key, dt in (("f16", torch.float16), ("bf16", torch.bfloat16)):
        x = torch.from_numpy(f[f"x_{key}"].view(np.int16)).view(dt).to(DEV)
        y = dequant_matmul_w4a16(x, qw, qz, sc).float().cpu().numpy()
        ref = f[f"out_{key}"]
        err = np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30)
        assert err < 1e-2, f"{key}: relative error {err}"
