"""Known-answer tests of the CPU oracle, restated from the reference's own checks.

Sources: benchmarks/bench_rht_a4.py:17-52 (oracle_checks: impulse responses,
ties-to-even, BF16 scale before codes, zero and tiny groups, packed bytes) and
benchmarks/rht_reference.py:111-146 (self_test: H12 orthogonality, dense
Kronecker equality, norm/linearity preservation, pack round trip, zero row).
The reference ran these in float64 PyTorch; the oracle is the fp32 contract,
so closed forms that are exact in fp32 are compared exactly and the rest with
an fp32-sized tolerance.
"""
import math

import numpy as np
import pytest

import oracle


def bf16(x):
    return oracle.f32_to_bf16(np.asarray(x, dtype=np.float32))


def test_quantizer_constants_bit_patterns():
    # fp32(0.9), RN(1/7), RN(1/sqrt 12), RN(1/sqrt 128)
    assert oracle.constant_bits(0) == 0x3F666666
    assert oracle.constant_bits(1) == 0x3E124925
    assert oracle.constant_bits(2) == 0x3E93CD3A
    assert oracle.constant_bits(3) == 0x3DB504F3
    # The same values as a multiply by the fp32 reciprocal of the fp32 divisor
    # (how CUDA PyTorch evaluates tensor / python-scalar).
    assert np.float32(1.0) / np.float32(7.0) == np.float32(1 / 7)
    assert np.float32(1.0) / np.float32(math.sqrt(12)) == np.float32(1 / math.sqrt(12))


def test_impulse_k4096_closed_form():
    # bench_rht_a4.py:22-29: impulse at 5 -> (-1)^popcount(j & 5) / sqrt(4096); exact in fp32.
    K = 4096
    x = np.zeros((1, K), np.float32)
    x[0, 5] = 1
    r = oracle.rht_rows(bf16(x), np.ones(K, np.int8))
    expected = np.array([(-1.0 if bin(j & 5).count("1") % 2 else 1.0) / 64 for j in range(K)], np.float32)
    assert np.array_equal(r[0], expected)


def test_impulse_k12288_paley_row1():
    # bench_rht_a4.py:30-34: impulse at 1024 -> Paley row 1 repeat-interleaved x1024 / sqrt(12288).
    K = 12288
    x = np.zeros((1, K), np.float32)
    x[0, 1024] = 1
    r = oracle.rht_rows(bf16(x), np.ones(K, np.int8))
    residues = {i * i % 11 for i in range(1, 11)}
    row = [1] + [(-1 if j == 0 else 1 if j in residues else -1) for j in range(11)]
    expected = np.repeat(np.array(row, np.float64), 1024) / math.sqrt(K)
    np.testing.assert_allclose(r[0], expected, rtol=2e-7, atol=0)
    # In fp32 the value is exactly +-2^-5 * RN(1/sqrt 12).
    inv12 = np.float32(1 / math.sqrt(12))
    assert np.array_equal(np.abs(r[0]), np.full(K, inv12 * np.float32(2.0**-5), np.float32))


def test_ties_to_even_and_clip():
    # bench_rht_a4.py:36-41
    values = np.zeros((1, 128), np.float32)
    values[0, :10] = [-7.5, -6.5, -4.5, -2.5, -.5, .5, 2.5, 4.5, 6.5, 7.5]
    values[0, -1] = 7 / .9
    codes, scales = oracle.quantize_rows(values)
    assert oracle.bf16_to_f32(scales)[0, 0] == 1.0
    assert codes[0, :10].tolist() == [-7, -6, -4, -2, 0, 0, 2, 4, 6, 7]


def test_bf16_scale_rounded_before_codes():
    # bench_rht_a4.py:42-45
    raw = np.float32(.9 / 7)
    rounded = oracle.bf16_to_f32(bf16(raw)).item()
    values = np.zeros((1, 128), np.float32)
    values[0, 0] = 1
    values[0, 1] = np.float32(np.float32(2.5) * np.float32(raw + np.float32(rounded))) / np.float32(2)
    codes, _ = oracle.quantize_rows(values)
    assert codes[0, 1] == 2
    assert np.round(values[0, 1] / raw) == 3


@pytest.mark.parametrize("magnitude,expected", [(0.0, 1.0), (1e-40, 2.0**-126)])
def test_zero_and_tiny_groups(magnitude, expected):
    # bench_rht_a4.py:46-48
    codes, scales = oracle.quantize_rows(np.full((1, 128), magnitude, np.float32))
    assert oracle.bf16_to_f32(scales)[0, 0] == np.float32(expected)
    assert np.count_nonzero(codes) == 0


def test_known_packed_bytes():
    # bench_rht_a4.py:49-50
    codes = np.arange(-8, 8, dtype=np.int8).reshape(1, 16)
    packed = oracle.pack_int4(codes)
    assert (packed.view(np.uint8)).ravel().tolist() == [0x98, 0xBA, 0xDC, 0xFE, 0x10, 0x32, 0x54, 0x76]
    assert np.array_equal(oracle.unpack_int4(packed), codes)


def test_h12_orthogonal():
    # rht_reference.py:113-114
    h = np.array([[oracle.paley_sign(s, d) for d in range(12)] for s in range(12)], np.float64)
    assert np.array_equal(h @ h.T, 12 * np.eye(12))
    # Paley construction over F_11 (rht_reference.py:15-23), built independently.
    residues = {i * i % 11 for i in range(1, 11)}
    ref = np.ones((12, 12))
    for i in range(11):
        for j in range(11):
            delta = (j - i) % 11
            ref[i + 1, j + 1] = -1 if delta == 0 else (1 if delta in residues else -1)
    assert np.array_equal(h, ref)
    assert not np.array_equal(h, h.T)  # orientation matters


def _sylvester(n):
    h = np.ones((1, 1))
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


@pytest.mark.parametrize("K", [16, 24, 48])
def test_dense_kronecker_small_k(K):
    # rht_reference.py:115-125: rht(x, signs) == (x * signs) @ H, H = H(K) or H12 (x) H(K/12), normalised.
    rng = np.random.default_rng(100 + K)
    n = K if K == 16 else K // 12
    hs = _sylvester(n)
    h12 = np.array([[oracle.paley_sign(s, d) for d in range(12)] for s in range(12)], np.float64)
    H = (hs if K == 16 else np.kron(h12, hs)) / math.sqrt(K)
    xb = bf16(rng.standard_normal((3, K)))
    x = oracle.bf16_to_f32(xb).astype(np.float64)
    signs = (rng.integers(0, 2, K) * 2 - 1).astype(np.int8)
    r = oracle.rht_rows(xb, signs)
    np.testing.assert_allclose(r, (x * signs) @ H, rtol=0, atol=2e-6 * np.abs(x).max())


@pytest.mark.parametrize("K", [4096, 12288])
def test_norm_and_linearity_preserved(K):
    # rht_reference.py:126-141 (norm, X W^T preservation, zero row -> scale 1 and no codes)
    rng = np.random.default_rng(K + 2026)
    signs = (rng.integers(0, 2, K) * 2 - 1).astype(np.int8)
    x = rng.standard_normal((17, K)).astype(np.float32)
    x[0] = 0
    x[1] = 0
    x[1, 7] = 1000
    w = (rng.standard_normal((32, K)) / math.sqrt(K)).astype(np.float32)
    xb, wb = bf16(x), bf16(w)
    xf, wf = oracle.bf16_to_f32(xb).astype(np.float64), oracle.bf16_to_f32(wb).astype(np.float64)
    xr, wr = oracle.rht_rows(xb, signs).astype(np.float64), oracle.rht_rows(wb, signs).astype(np.float64)
    nx = np.linalg.norm(xf, axis=1)
    assert (np.abs(np.linalg.norm(xr, axis=1) - nx) / np.maximum(nx, 1)).max() < 5e-6
    ref = xf @ wf.T
    rrmse = math.sqrt(((xr @ wr.T - ref) ** 2).sum() / (ref ** 2).sum())
    assert rrmse < 5e-6
    codes, scales = oracle.quantize_rows(xr.astype(np.float32))
    assert np.array_equal(oracle.unpack_int4(oracle.pack_int4(codes)), codes)
    assert oracle.bf16_to_f32(scales)[0].tolist() == [1.0] * (K // 128)
    assert np.count_nonzero(codes[0]) == 0
