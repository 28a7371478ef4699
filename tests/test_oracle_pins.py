"""Pinning the CPU oracle beyond the reference's known answers.

The C oracle restates the reference's TileLang kernels (op order of
nanovllm/kernels/rht_a4_tilelang.py and w4a4_grouped_kernel.py).  The checks
here are independent formulations taken from *other* reference sources:

* the vectorised float32 restatement of the reference's PyTorch oracle
  (benchmarks/rht_reference.py:26-39 fwht, benchmarks/a4_group_quant.py:47-70
  rotate/quantize_rotated, evaluated with CUDA's reciprocal-multiply scalar
  division), which must agree bit for bit -- the reference asserts exactly
  this equality between its kernel and its PyTorch path
  (benchmarks/bench_rht_a4.py:55-61, 80-88);
* an exact-rational replay of the GEMM epilogue with a correctly rounded
  fp32 FMA (benchmarks/verify_w4a4_aw_grouped.py:13-29 emulates the same
  thing in float64);
* mathematical invariants: constant dyadic scales reduce to ungrouped
  integer dots (benchmarks/verify_w4a4_grouped.py:75-79,
  verify_w4a4_aw_grouped.py:84-90), float64 relative RMSE < 2e-6;
* closed forms of the W4A16 dequantisation.

Each plausible mistake is then planted in the oracle (a mutation switch in
oracle.c) to show one of these checks rejects it.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

import oracle
from nv4 import workloads as W

F32 = np.float32


def bf16(x):
    return oracle.f32_to_bf16(np.asarray(x, dtype=np.float32))


# ---------------------------------------------------------------- restatements
def fwht_vectorized(x):
    """rht_reference.py:26-39 in float32; / sqrt(n) is a multiply by RN(1/RN(sqrt n))."""
    shape, n = x.shape, x.shape[-1]
    y, step = x.astype(F32), 1
    while step < n:
        z = y.reshape(*shape[:-1], n // (2 * step), 2, step)
        a, b = z[..., 0, :], z[..., 1, :]
        y = np.stack((a + b, a - b), axis=-2).reshape(shape)
        step *= 2
    return y * (F32(1.0) / F32(math.sqrt(n)))


def h12_matrix():
    residues = {i * i % 11 for i in range(1, 11)}
    h = np.ones((12, 12), F32)
    for i in range(11):
        for j in range(11):
            delta = (j - i) % 11
            h[i + 1, j + 1] = -1 if delta == 0 else (1 if delta in residues else -1)
    return h


def rotate_vectorized(x_f32, signs):
    """a4_group_quant.py:47-56: x*signs, fwht, and for K=12288 H12^T @ z / sqrt(12)
    with the 12-term sums accumulated in source order."""
    x = x_f32.astype(F32) * signs.astype(F32)
    K = x.shape[-1]
    if K == 4096:
        return fwht_vectorized(x)
    z = fwht_vectorized(x.reshape(-1, 12, 1024))
    h = h12_matrix()
    out = np.zeros_like(z)
    for d in range(12):
        acc = np.zeros(z.shape[::2], F32)
        for s in range(12):
            acc = acc + h[s, d] * z[:, s, :]
        out[:, d, :] = acc
    return (out * (F32(1.0) / F32(math.sqrt(12)))).reshape(x.shape)


def quantize_vectorized(r, group=128, clip=0.9):
    """a4_group_quant.py:60-70 under CUDA semantics (tensor * python float in fp32,
    tensor / python float as a multiply by the fp32 reciprocal)."""
    m, k = r.shape
    g = r.reshape(m, k // group, group).astype(F32)
    mx = np.abs(g).max(-1)
    t = (mx * F32(clip)) * (F32(1.0) / F32(7.0))
    t = np.maximum(t, F32(2.0 ** -126))
    scale = oracle.bf16_to_f32(bf16(np.where(mx == 0, F32(1.0), t)))
    codes = np.clip(np.round(g / scale[..., None]), -7, 7).astype(np.int8).reshape(m, k)
    return codes, bf16(scale)


def make_rows(M, K, seed):
    """The reference's special rows (rht_a4_bench_common.py:104-120) on seeded randn."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(F32)
    x[0] = 0
    if M > 1:
        x[1] = 0
        x[1, K // 12 if K == 12288 else 5] = 1000
    if M > 2:
        x[2] = 1
    if M > 3:
        x[3, ::2], x[3, 1::2] = 1, -1
    if M > 4:
        x[4] *= 1e-9
    if M > 5:
        x[5] *= 1e4
    return bf16(x)


def check_rotation_matches_vectorized(K, M=9, seed=7):
    xb = make_rows(M, K, seed)
    signs = (np.random.default_rng(seed + 1).integers(0, 2, K) * 2 - 1).astype(np.int8)
    r = oracle.rht_rows(xb, signs)
    ref = rotate_vectorized(oracle.bf16_to_f32(xb), signs)
    assert np.array_equal(r.view(np.uint32), ref.view(np.uint32)), "rotation differs from the vectorised restatement"


def check_quantize_matches_vectorized(K, M=9, seed=11):
    xb = make_rows(M, K, seed)
    signs = (np.random.default_rng(seed + 1).integers(0, 2, K) * 2 - 1).astype(np.int8)
    r = oracle.rht_rows(xb, signs)
    codes, scales = oracle.quantize_rows(r)
    c2, s2 = quantize_vectorized(r)
    assert np.array_equal(scales, s2), "scales differ"
    assert np.array_equal(codes, c2), "codes differ"
    packed, sc = oracle.rht_quant_pack(xb, signs)
    assert np.array_equal(packed, oracle.pack_int4(c2)) and np.array_equal(sc, s2)


@pytest.mark.parametrize("K", [4096, 12288])
def test_rotation_bit_exact_vs_pytorch_restatement(K):
    check_rotation_matches_vectorized(K)


@pytest.mark.parametrize("K", [4096, 12288])
def test_quantizer_bit_exact_vs_pytorch_restatement(K):
    check_quantize_matches_vectorized(K)


def find_reciprocal_sensitive_max():
    """A group maximum whose BF16 scale differs between RN(RN(mx*0.9)*RN(1/7)) (the
    reference kernel, rht_a4_tilelang.py:123-126) and RN(RN(mx*0.9)/7) (true division)."""
    rng = np.random.default_rng(3)
    for _ in range(200):
        mx = rng.uniform(0.5, 8.0, 100000).astype(F32)
        t1 = (mx * F32(0.9)) * (F32(1.0) / F32(7.0))
        t2 = (mx * F32(0.9)) / F32(7.0)
        d = np.nonzero(bf16(t1) != bf16(t2))[0]
        if d.size:
            return mx[d[0]], bf16(t1[d[0]])
    raise AssertionError("no reciprocal-sensitive value found")


def check_reciprocal_scale():
    mx, expected = find_reciprocal_sensitive_max()
    v = np.zeros((1, 128), F32)
    v[0, 3] = mx
    _, s = oracle.quantize_rows(v)
    assert s[0, 0] == expected, "scale is not the reciprocal-multiply value"


def test_scale_uses_fp32_reciprocal_of_7():
    check_reciprocal_scale()


def test_block128_layout_is_per_block_hadamard():
    K = 512
    xb = make_rows(4, K, 5)
    signs = (np.random.default_rng(9).integers(0, 2, K) * 2 - 1).astype(np.int8)
    r = oracle.rht_rows(xb, signs, layout=oracle.LAYOUT_BLOCK128)
    x = oracle.bf16_to_f32(xb) * signs.astype(F32)
    blocks = x.reshape(4, K // 128, 128)
    # 128-point vectorised butterflies, then one multiply by RN(1/sqrt 128).
    shape, y, step = blocks.shape, blocks, 1
    while step < 128:
        z = y.reshape(*shape[:-1], 128 // (2 * step), 2, step)
        y = np.stack((z[..., 0, :] + z[..., 1, :], z[..., 0, :] - z[..., 1, :]), axis=-2).reshape(shape)
        step *= 2
    ref = (y * F32(1 / math.sqrt(128))).reshape(4, K)
    assert np.array_equal(r, ref)
    # Dense check of the orthogonal transform it represents.
    hs = np.ones((1, 1))
    while hs.shape[0] < 128:
        hs = np.block([[hs, hs], [hs, -hs]])
    dense = (x.reshape(4, K // 128, 128).astype(np.float64) @ hs / math.sqrt(128)).reshape(4, K)
    np.testing.assert_allclose(r, dense, rtol=0, atol=1e-5 * max(1.0, np.abs(x).max()))


# ------------------------------------------------------------------------ GEMM
def rn32(q: Fraction) -> float:
    """Round an exact rational to the nearest fp32 (ties to even), subnormals kept."""
    if q == 0:
        return 0.0
    sign = -1.0 if q < 0 else 1.0
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    unit = Fraction(2) ** max(e - 23, -149)
    m = a / unit
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * float(n * unit)


def gemm_exact_replay(qa, qw, sa, sw):
    """for g: total = RN(d * RN(sa*sw) + total), exact rationals in between."""
    M, K = qa.shape
    N = qw.shape[0]
    G = K // 128
    saf, swf = oracle.bf16_to_f32(sa), oracle.bf16_to_f32(sw)
    out = np.zeros((M, N), F32)
    dots = np.einsum("mgk,ngk->mng", qa.reshape(M, G, 128).astype(np.int64), qw.reshape(N, G, 128).astype(np.int64))
    for m in range(M):
        for n in range(N):
            total = 0.0
            for g in range(G):
                p = rn32(Fraction(float(saf[m, g])) * Fraction(float(swf[n, g])))
                total = rn32(Fraction(int(dots[m, n, g])) * Fraction(p) + Fraction(total))
            out[m, n] = total
    return out


def gemm_inputs(M, N, K, seed):
    """The reference's GEMM test recipe (verify_w4a4_aw_grouped.py:47-56)."""
    rng = np.random.default_rng(seed)
    qa = rng.integers(-8, 8, (M, K)).astype(np.int8)
    qw = rng.integers(-8, 8, (N, K)).astype(np.int8)
    qa[0] = 0
    qw[0] = 0
    sa = bf16(rng.random((M, K // 128)) * 2)
    sw = bf16(rng.random((N, K // 128)) * .03)
    sa[1, ::2] = 0
    sw[1, 1::2] = 0
    return qa, qw, sa, sw


def check_gemm_exact_replay(M=17, N=96, K=512, seed=20261110):
    qa, qw, sa, sw = gemm_inputs(M, N, K, seed)
    got = oracle.w4a4_gemm(oracle.pack_int4(qa), oracle.pack_int4(qw), sa, sw, out_fp32=True)
    ref = gemm_exact_replay(qa, qw, sa, sw)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "GEMM epilogue differs from exact fma replay"
    assert np.array_equal(oracle.w4a4_gemm(oracle.pack_int4(qa), oracle.pack_int4(qw), sa, sw), bf16(ref))


def test_gemm_matches_exact_rational_fma_replay():
    check_gemm_exact_replay()


def test_gemm_group_dots_are_integer_products():
    qa, qw, sa, sw = gemm_inputs(9, 40, 1024, 4)
    d = oracle.w4a4_group_dots(oracle.pack_int4(qa), oracle.pack_int4(qw))
    ref = np.einsum("mgk,ngk->mng", qa.reshape(9, 8, 128).astype(np.int64), qw.reshape(40, 8, 128).astype(np.int64))
    assert np.array_equal(d, ref)


@pytest.mark.parametrize("M,N,K", [(17, 96, 512), (33, 136, 4096), (32, 128, 12288)])
def test_gemm_precise_and_constant_scale_reductions(M, N, K):
    qa, qw, sa, sw = gemm_inputs(M, N, K, 20261110 + K)
    ap, wp = oracle.pack_int4(qa), oracle.pack_int4(qw)
    out32 = oracle.w4a4_gemm(ap, wp, sa, sw, out_fp32=True)
    # float64 relative RMSE (verify_w4a4_aw_grouped.py:74-75)
    G = K // 128
    dots = np.einsum("mgk,ngk->mng", qa.reshape(M, G, 128).astype(np.float64), qw.reshape(N, G, 128).astype(np.float64))
    precise = (dots * oracle.bf16_to_f32(sa)[:, None, :] * oracle.bf16_to_f32(sw)[None, :, :]).sum(-1)
    rrmse = math.sqrt(((out32 - precise) ** 2).mean()) / max(math.sqrt((precise ** 2).mean()), 1e-20)
    assert rrmse < 2e-6
    # Constant dyadic weight scale: 2-D == 1-D == activation-only grouped reference.
    channel = bf16(np.full(N, 0.125, F32))
    repeated = np.repeat(channel[:, None], G, axis=1)
    a_only = np.zeros((M, N), F32)
    saf = oracle.bf16_to_f32(sa)
    for g in range(G):
        a_only = a_only + (dots[:, :, g].astype(F32) * saf[:, g][:, None])
    a_only_ref = bf16(a_only * F32(0.125))
    assert np.array_equal(oracle.w4a4_gemm(ap, wp, sa, channel), a_only_ref)
    assert np.array_equal(oracle.w4a4_gemm(ap, wp, sa, repeated), a_only_ref)
    # Constant dyadic activation scale reduces to one ungrouped integer dot.
    sa_c = bf16(np.full((M, G), 0.125, F32))
    swc = bf16(np.random.default_rng(K).random(N) * .03)
    full = (qa.astype(np.int64) @ qw.astype(np.int64).T).astype(F32)
    assert np.array_equal(oracle.w4a4_gemm(ap, wp, sa_c, swc),
                          bf16((full * F32(0.125)) * oracle.bf16_to_f32(swc)[None, :]))


def test_gemm_grouped_order_is_not_dense_dequant():
    # benchmarks/README.md:135-138: a dense dequantised GEMM is a different function.
    qa, qw, sa, sw = gemm_inputs(33, 136, 4096, 77)
    ap, wp = oracle.pack_int4(qa), oracle.pack_int4(qw)
    grouped = oracle.w4a4_gemm(ap, wp, sa, sw, out_fp32=True)
    G = 32
    dq_a = (qa.reshape(33, G, 128) * oracle.bf16_to_f32(sa)[:, :, None]).reshape(33, 4096).astype(F32)
    dq_w = (qw.reshape(136, G, 128) * oracle.bf16_to_f32(sw)[:, :, None]).reshape(136, 4096).astype(F32)
    dense = dq_a @ dq_w.T
    assert not np.array_equal(grouped, dense)
    np.testing.assert_allclose(grouped, dense, rtol=1e-4, atol=1e-4)


# ---------------------------------------------------------------------- W4A16
def test_w4a16_dequant_closed_form():
    K, N = 256, 16
    q = np.zeros((K, N), np.int64)
    z = np.zeros((K // 128, N), np.int64)
    s = np.zeros((K // 128, N), np.float16)
    # q - z - 1 takes every value in [-16, 14]; scales are exact fp16/bf16 values.
    rng = np.random.default_rng(0)
    q[:] = rng.integers(0, 16, (K, N))
    z[:] = rng.integers(0, 16, (K // 128, N))
    s[:] = np.float16(0.0078125) * (1 + (np.arange(N) % 4))  # 2^-7 * {1,2,3,4}: exact in bf16
    import torch
    qweight = W.pack_qweight(torch.from_numpy(q)).numpy()
    qzeros = W.pack_qzeros(torch.from_numpy(z)).numpy()
    deq = oracle.w4a16_dequant(qweight, qzeros, s.view(np.uint16))
    zz = np.repeat(z, 128, axis=0)
    ss = np.repeat(s.astype(np.float64), 128, axis=0)
    assert np.array_equal(deq.astype(np.float64), (q - zz - 1) * ss)
    deq16 = oracle.w4a16_dequant(qweight, qzeros, s.view(np.uint16), x_dtype=oracle.X_FP16)
    assert np.array_equal(deq16.astype(np.float64), (q - zz - 1) * ss)
    # q == z + 1 dequantises to exactly zero.
    q2 = np.repeat(z + 1, 128, axis=0) % 16
    ok = np.repeat(z + 1, 128, axis=0) < 16
    qweight2 = W.pack_qweight(torch.from_numpy(q2)).numpy()
    d2 = oracle.w4a16_dequant(qweight2, qzeros, s.view(np.uint16))
    assert np.all(d2[ok] == 0)


def test_w4a16_bf16_rounding_of_dequantised_weight():
    # A scale with more fp16 mantissa bits than bf16 keeps: the reference converts
    # the fp16 scale to bf16 first (linear_w4a16.py:28,42) and rounds the product to bf16.
    import torch
    s = np.full((1, 8), np.float16(0.0123), np.float16)
    q = np.full((128, 8), 15, np.int64)
    z = np.zeros((1, 8), np.int64)
    deq = oracle.w4a16_dequant(W.pack_qweight(torch.from_numpy(q)).numpy(),
                               W.pack_qzeros(torch.from_numpy(z)).numpy(), s.view(np.uint16))
    sb = oracle.bf16_to_f32(bf16(np.float32(s[0, 0])))
    assert deq[0, 0] == oracle.bf16_to_f32(bf16(F32(14) * sb))


def test_w4a16_gemm_float64():
    import torch
    case = W.w4a16_case(5, N=64, K=256)
    x = case.x.numpy().view(np.uint16)
    out = oracle.w4a16_gemm(x, case.qweight.numpy(), case.qzeros.numpy(), case.scales.numpy().view(np.uint16),
                            x_dtype=oracle.X_FP16)
    deq = oracle.w4a16_dequant(case.qweight.numpy(), case.qzeros.numpy(), case.scales.numpy().view(np.uint16),
                               x_dtype=oracle.X_FP16).astype(np.float64)
    ref = case.x.numpy().astype(np.float64) @ deq
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------ mutations
@pytest.fixture
def mutation():
    def plant(m):
        oracle.set_mutation(m)
    yield plant
    oracle.set_mutation(0)


@pytest.mark.parametrize("m,check", [
    (1, lambda: check_rotation_matches_vectorized(4096)),       # butterfly strides descending
    (2, lambda: check_rotation_matches_vectorized(12288)),      # H12 transposed
    (3, check_reciprocal_scale),                                # true division by 7
    (4, lambda: check_quantize_matches_vectorized(4096)),       # codes from the unrounded scale
    (5, check_gemm_exact_replay),                               # unfused multiply-add in the epilogue
])
def test_planted_mistake_is_rejected(mutation, m, check):
    check()                 # faithful oracle passes
    mutation(m)
    with pytest.raises(AssertionError):
        check()
