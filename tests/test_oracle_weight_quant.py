"""Pins of the oracle's weight RTN quantizer, dequantizer and error summary.

``oracle.weight_quantize`` restates quantize_rows / quantize_groups
(benchmarks/rht_reference.py:70-77, benchmarks/rht_gptq_grouped.py:27-39) and
grouped_quantize (benchmarks/kernel_bench_common.py:36-42);
``oracle.error_stats`` restates benchmarks/rht_reference.py:99-108.  The
checks do not retype those formulas:

* at clip 0.9 with the CUDA division the weight quantizer must equal the
  activation quantizer ``oracle.quantize_rows``, which the reference's own
  known answers pin (the reference feeds grouped_quantize(x, 128, .9) codes to
  its activation-side kernels, benchmarks/tune_w4a4_aw_grouped.py:46);
* the reference self-test's zero row (rht_reference.py:140-141) and the
  2^-126 floor;
* exact dyadic groups whose codes and scale are known in closed form;
* brute force: every code is a nearest grid point of its scale, the bf16
  scale lies within half a bf16 ulp of max*clip/7;
* torch's CPU kernels evaluating the reference's expression (a library
  routine with the CPU division);
* closed forms of the error summary;
* two planted mistakes (the other device's division, truncation) rejected.
"""
import math

import numpy as np
import pytest

import oracle

F32 = np.float32


def bf16(x):
    return oracle.f32_to_bf16(np.asarray(x, dtype=F32))


def rows(N, K, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) / math.sqrt(K)).astype(F32)
    w[0] = 0
    if N > 2:
        w[2, 5] = 1000.0
    if N > 3:
        w[3] *= F32(1e-30)
    return w


# ------------------------------------------------------------ cross-pinning
@pytest.mark.parametrize("K", [128, 4096])
def test_clip09_cuda_division_equals_activation_quantizer(K):
    rng = np.random.default_rng(K)
    r = rng.standard_normal((40, K)).astype(F32)
    r[0] = 0
    r[1, ::2], r[1, 1::2] = 1, -1
    r[2] *= F32(1e-38)
    r[3] *= F32(1e4)
    r[4, :] = rng.integers(-7, 8, K).astype(F32) * F32(0.5)  # tie-rich rows
    codes, scales = oracle.weight_quantize(r, 128, 0.9, oracle.DIVISION_CUDA)
    c2, s2 = oracle.quantize_rows(r)
    assert np.array_equal(scales, s2)
    assert np.array_equal(codes, c2)


def test_zero_row_and_tiny_floor():
    w = np.zeros((3, 256), F32)
    w[1, 7] = F32(1e-40)        # max/7 below 2^-126: the scale floors to 2^-126
    w[2, 130] = F32(-3e-39)
    for division in (oracle.DIVISION_CPU, oracle.DIVISION_CUDA):
        codes, scales = oracle.weight_quantize(w, 128, 1.0, division)
        assert (scales[0] == 0x3F80).all() and not codes[0].any()   # zero group: scale 1, codes 0
        assert scales[1, 0] == 0x0080 and scales[1, 1] == 0x3F80    # 2^-126; untouched group 1
        assert not codes[1].any()                                    # 1e-40 / 2^-126 rounds to 0
        assert scales[2, 1] == 0x0080 and codes[2, 130] == 0         # 3e-39 / 1.18e-38 = 0.25 -> 0


@pytest.mark.parametrize("division", [0, 1])
def test_dyadic_groups_are_recovered_exactly(division):
    rng = np.random.default_rng(5)
    N, K = 16, 512
    c = rng.integers(-7, 8, (N, K)).astype(np.int8)
    c[:, ::128] = np.where(rng.random((N, K // 128)) < .5, 7, -7)    # every group reaches |7|
    e = rng.integers(-30, 20, (N, K // 128))
    w = (c.astype(np.float64) * np.ldexp(1.0, np.repeat(e, 128, axis=1))).astype(F32)
    codes, scales = oracle.weight_quantize(w, 128, 1.0, division)
    assert np.array_equal(codes, c)
    assert np.array_equal(oracle.bf16_to_f32(scales), np.ldexp(1.0, e).astype(F32))
    deq = oracle.weight_dequantize(codes, scales)
    assert np.array_equal(deq, w)
    st = oracle.error_stats(deq, w)
    assert st["relative_rmse"] == 0 and st["max_abs"] == 0 and st["cosine"] == pytest.approx(1, abs=1e-15)


def check_grid_and_scale(division, clip, K, group):
    w = rows(24, K, 17 + K)
    codes, scales = oracle.weight_quantize(w, group, clip, division)
    G = -(-K // group)
    assert scales.shape == (24, G)
    s = oracle.bf16_to_f32(scales).astype(np.float64)
    grid = np.arange(-7, 8, dtype=np.float64)
    for n in range(24):
        for g in range(G):
            seg = w[n, g * group:(g + 1) * group].astype(np.float64)
            q = codes[n, g * group:(g + 1) * group].astype(np.float64)
            mx = np.abs(seg).max()
            if mx == 0:
                assert s[n, g] == 1.0 and not q.any()
                continue
            exact = max(mx * float(F32(clip)) / 7.0, 2.0 ** -126)
            # one bf16 rounding (8 significant bits) after at most two fp32 roundings
            assert abs(s[n, g] - exact) <= exact * (2.0 ** -8 + 2.0 ** -22), (n, g, s[n, g], exact)
            best = np.abs(seg[:, None] - grid[None, :] * s[n, g]).min(1)
            mine = np.abs(seg - q * s[n, g])
            assert np.all(mine <= best * (1 + 2.0 ** -18) + 1e-300), (n, g)
            assert np.all(np.abs(q) <= 7)


def test_codes_are_nearest_points_and_scale_is_rounded_max():
    for division in (0, 1):
        for clip in (1.0, 0.9, 0.45):
            for K, group in ((512, 128), (300, 128), (96, 7)):
                check_grid_and_scale(division, clip, K, group)


def torch_cpu_quantize(w, group, clip):
    """The reference expression evaluated by torch on CPU tensors (IEEE division)."""
    import torch
    x = torch.from_numpy(w)
    n, k = x.shape
    codes, scales = [], []
    for start in range(0, k, group):
        part = x[:, start:start + group].float()
        maximum = part.abs().amax(-1)
        scale = torch.where(maximum == 0, 1., (maximum * clip / 7).clamp_min(torch.finfo(torch.bfloat16).tiny))
        scale = scale.bfloat16()
        codes.append((part / scale.float()[:, None]).round().clamp(-7, 7).to(torch.int8))
        scales.append(scale)
    return (torch.cat(codes, 1).numpy(), torch.stack(scales, 1).view(torch.int16).numpy().view(np.uint16))


def division_sensitive_rows(clip):
    """Groups whose bf16 scale differs between mx*clip/7 and mx*clip*RN(1/7)."""
    rng = np.random.default_rng(23)
    mx = rng.uniform(0.5, 8.0, 400000).astype(F32)
    t = mx * F32(clip)
    hit = np.nonzero(bf16(t / F32(7)) != bf16(t * (F32(1) / F32(7))))[0][:8]
    assert hit.size, "no division-sensitive maximum found"
    w = rng.uniform(-0.4, 0.4, (hit.size, 128)).astype(F32)
    w[:, 9] = mx[hit]
    return w


@pytest.mark.parametrize("clip", [1.0, 0.9])
def test_cpu_division_equals_torch_cpu(clip):
    sens = division_sensitive_rows(clip)
    w = np.ascontiguousarray(np.concatenate([rows(12, 256, 3), np.concatenate([sens, sens[:, ::-1]], 1)], 0))
    for group in (128, 100):
        c_ref, s_ref = torch_cpu_quantize(w, group, clip)
        codes, scales = oracle.weight_quantize(w, group, clip, oracle.DIVISION_CPU)
        assert np.array_equal(scales, s_ref)
        assert np.array_equal(codes, c_ref)
    # and the two device semantics really differ on these rows
    assert not np.array_equal(oracle.weight_quantize(sens, 128, clip, oracle.DIVISION_CPU)[1],
                              oracle.weight_quantize(sens, 128, clip, oracle.DIVISION_CUDA)[1])


def test_ragged_last_group_equals_per_slice_rows():
    """quantize_groups(w) = concatenation of quantize_rows over K-slices
    (rht_gptq_grouped.py:27-34), the last slice shorter."""
    w = rows(9, 300, 41)
    codes, scales = oracle.weight_quantize(w, 128, 1.0, oracle.DIVISION_CPU)
    for g, (a, b) in enumerate(((0, 128), (128, 256), (256, 300))):
        c1, s1 = oracle.weight_quantize(np.ascontiguousarray(w[:, a:b]), b - a, 1.0, oracle.DIVISION_CPU)
        assert np.array_equal(codes[:, a:b], c1) and np.array_equal(scales[:, g], s1[:, 0])


def test_dequantize_is_exact():
    rng = np.random.default_rng(8)
    codes = rng.integers(-8, 8, (7, 300)).astype(np.int8)
    scales = bf16(rng.standard_normal((7, 3)).astype(F32) * F32(1e3))
    out = oracle.weight_dequantize(codes, scales)
    expect = codes.astype(np.float64) * np.repeat(oracle.bf16_to_f32(scales).astype(np.float64), 128, 1)[:, :300]
    assert np.array_equal(out.astype(np.float64), expect)
    with pytest.raises(ValueError):
        oracle.weight_dequantize(codes, scales[:, :2])


# ------------------------------------------------------------- error_stats
def test_error_stats_closed_forms():
    rng = np.random.default_rng(2)
    r = rng.standard_normal(1000).astype(F32)
    same = oracle.error_stats(r, r)
    assert same["relative_rmse"] == 0 and same["max_abs"] == 0 and same["sse"] == 0
    # squares are fp32 products (rounded), the dot is float64: cosine is 1 within 2^-24
    assert same["cosine"] == pytest.approx(1, abs=2 ** -23) and same["elements"] == 1000
    double = oracle.error_stats(2 * r, r)               # exact in fp32
    assert double["relative_rmse"] == pytest.approx(1, rel=1e-14)
    assert double["cosine"] == pytest.approx(1, abs=2 ** -23)
    assert double["max_abs"] == float(np.abs(r).max())
    neg = oracle.error_stats(-r, r)
    assert neg["relative_rmse"] == pytest.approx(2, rel=1e-14) and neg["cosine"] == pytest.approx(-1, abs=2 ** -23)
    ortho = oracle.error_stats(np.array([3, 0], F32), np.array([0, 4], F32))
    assert ortho["cosine"] == 0 and ortho["sse"] == 25 and ortho["reference_energy"] == 16
    assert ortho["relative_rmse"] == pytest.approx(5 / 4, rel=1e-15) and ortho["max_abs"] == 4
    zero = oracle.error_stats(np.array([1e-10], F32), np.zeros(1, F32))
    assert zero["relative_rmse"] == pytest.approx(math.sqrt(float(F32(1e-10)) ** 2 / 1e-30), rel=1e-6)
    assert zero["cosine"] == 0


def test_error_stats_difference_is_fp32():
    """1 - 2^-25 is a tie between 1 - 2^-24 and 1 in fp32 and rounds to 1 (even):
    the reference subtracts fp32 tensors, so sse is exactly 1."""
    st = oracle.error_stats(np.array([1.0], F32), np.array([2.0 ** -25], F32))
    assert st["sse"] == 1.0 and st["max_abs"] == 1.0


# ---------------------------------------------------------------- mutations
@pytest.fixture
def mutation():
    def plant(m):
        oracle.set_mutation(m)
    yield plant
    oracle.set_mutation(0)


@pytest.mark.parametrize("m,check", [
    (6, lambda: test_cpu_division_equals_torch_cpu(1.0)),        # the other device's division
    (6, lambda: test_clip09_cuda_division_equals_activation_quantizer(4096)),
    (7, test_codes_are_nearest_points_and_scale_is_rounded_max),  # truncation toward zero
])
def test_planted_mistake_is_rejected(mutation, m, check):
    check()
    mutation(m)
    with pytest.raises(AssertionError):
        check()
