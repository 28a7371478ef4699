"""GPU parity of K2 (grouped W4A4 INT4 GEMM) against the oracle.

Restates benchmarks/verify_w4a4_aw_grouped.py and verify_w4a4_grouped.py:
the reference shapes (17,96,512), (33,136,4096), (32,128,12288) with codes
in [-8,7], a zero row in each operand, zeroed scale stripes, BF16 and fp32
outputs bit-exact against the per-group FMA reference, 64-element canaries,
three repeated calls, and the constant-scale reductions to the per-channel
API.  Adds an M sweep across the kernel boundaries (skinny M <= 64, tiled
above; tails in M and N) and the four Qwen3-8B projections at M = 32 (every
element) and M = 4096 (a row sample, like the reference's pipeline audit,
benchmarks/bench_rht_a4.py:184-190).  Every case with N % 16 == 0 runs again
on the same weights in the MFMA-tiled layout (``tile_weights``), whose
results must equal the reference-layout results bit for bit, and the tiled
layout itself is pinned against its definition.  Bar: bit-exact.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import bf16_bits, bits_to_bf16
from nv4 import compile_grouped_gemm, rht_quant_pack, tile_weights, untile_weights, w4a4_grouped_gemm
from nv4 import workloads as W

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def gemm_inputs(M, N, K, seed):
    rng = np.random.default_rng(seed)
    qa = rng.integers(-8, 8, (M, K)).astype(np.int8)
    qw = rng.integers(-8, 8, (N, K)).astype(np.int8)
    qa[0] = 0
    qw[0] = 0
    sa = oracle.f32_to_bf16((rng.random((M, K // 128)) * 2).astype(np.float32))
    sw = oracle.f32_to_bf16((rng.random((N, K // 128)) * .03).astype(np.float32))
    if M > 1:
        sa[1, ::2] = 0
    if N > 1:
        sw[1, 1::2] = 0
    return oracle.pack_int4(qa), oracle.pack_int4(qw), sa, sw


def to_dev(ap, wp, sa, sw):
    return (torch.from_numpy(ap).to(DEV), torch.from_numpy(wp).to(DEV),
            bits_to_bf16(sa).to(DEV), bits_to_bf16(sw).to(DEV))


def describe_mismatch(got, ref):
    bad = np.argwhere(got != ref)
    rows = np.unique(bad[:, 0])[:10].tolist()
    cols = np.unique(bad[:, 1])[:10].tolist()
    return f"{len(bad)} of {got.size} differ; rows {rows}; cols {cols}"


def assert_bits_equal(got, ref, what):
    if not np.array_equal(got, ref):
        raise AssertionError(f"{what}: " + describe_mismatch(got, ref))


def run_case(M, N, K, seed, grouped=True):
    print(f"[k2] M={M} N={N} K={K} grouped={grouped}", flush=True)
    ap, wp, sa, sw = gemm_inputs(M, N, K, seed)
    if not grouped:
        sw = sw[:, 0].copy()
    exp_bf16 = oracle.w4a4_gemm(ap, wp, sa, sw)
    exp_f32 = oracle.w4a4_gemm(ap, wp, sa, sw, out_fp32=True)
    a, w, s_a, s_w = to_dev(ap, wp, sa, sw)
    storage = torch.full((M * N + 128,), -1234, device=DEV, dtype=torch.bfloat16)
    sentinel = storage[:64].clone()
    out = storage[64:-64].view(M, N)
    for _ in range(3):
        out.fill_(float("nan"))
        got = w4a4_grouped_gemm(a, w, s_a, s_w, out=out)
        torch.cuda.synchronize()
        assert got.data_ptr() == out.data_ptr()
        assert_bits_equal(bf16_bits(out), exp_bf16, "bf16 output")
        assert torch.equal(storage[:64], sentinel) and torch.equal(storage[-64:], sentinel)
    out32 = torch.full((M, N), float("nan"), device=DEV, dtype=torch.float32)
    compile_grouped_gemm(M, N, K, output_fp32=True, weight_grouped=grouped)(a, w, s_a, s_w, out32)
    torch.cuda.synchronize()
    assert_bits_equal(out32.cpu().numpy().view(np.uint32), exp_f32.view(np.uint32), "fp32 output")
    if N % 16 == 0:
        wt = tile_weights(w)
        out.fill_(float("nan"))
        w4a4_grouped_gemm(a, wt, s_a, s_w, out=out, weights_tiled=True)
        torch.cuda.synchronize()
        assert_bits_equal(bf16_bits(out), exp_bf16, "bf16 output, tiled weights")
        assert torch.equal(storage[:64], sentinel) and torch.equal(storage[-64:], sentinel)
    return ap, wp, sa, sw, a, w, s_a, s_w


@pytest.mark.parametrize("N,K", [(16, 128), (48, 384), (6144, 4096), (4096, 12288)])
def test_tiled_weight_layout(N, K):
    """The tiled order is the documented permutation: unit (cb*G + g)*64 + l
    holds bytes 64 g + 16 (l/16) .. +15 of column 16 cb + l%16; untiling
    restores the input."""
    rng = np.random.default_rng(N + K)
    w = rng.integers(-128, 128, (N, K // 2), dtype=np.int8)
    ref = w.reshape(N // 16, 16, K // 128, 4, 16).transpose(0, 2, 3, 1, 4).reshape(N, K // 2)
    wt = tile_weights(torch.from_numpy(w).to(DEV))
    torch.cuda.synchronize()
    assert np.array_equal(wt.cpu().numpy(), ref)
    assert np.array_equal(untile_weights(wt).cpu().numpy(), w)
    with pytest.raises(ValueError):
        tile_weights(torch.zeros((24, 64), dtype=torch.int8, device=DEV))


@pytest.mark.parametrize("M,N,K", [(17, 96, 512), (33, 136, 4096), (32, 128, 12288)])
def test_k2_reference_shapes(M, N, K):
    ap, wp, sa, sw, a, w, s_a, _ = run_case(M, N, K, 20261110 + K)
    # Constant dyadic weight scale: grouped == per-channel API (verify_w4a4_aw_grouped.py:84-90).
    channel = torch.full((N,), .125, device=DEV, dtype=torch.bfloat16)
    repeated = channel[:, None].expand(N, K // 128).contiguous()
    one = w4a4_grouped_gemm(a, w, s_a, channel)
    two = w4a4_grouped_gemm(a, w, s_a, repeated)
    exp = oracle.w4a4_gemm(ap, wp, sa, bf16_bits(channel))
    assert_bits_equal(bf16_bits(one), exp, "per-channel API")
    assert_bits_equal(bf16_bits(two), exp, "grouped API with constant scale")
    # Constant dyadic activation scale reduces to one ungrouped integer dot (verify_w4a4_grouped.py:75-79).
    s_a.fill_(.125)
    sw1 = torch.rand(N, generator=torch.Generator("cpu").manual_seed(K)).mul(.03).to(torch.bfloat16).to(DEV)
    got = w4a4_grouped_gemm(a, w, s_a, sw1)
    qa, qw = oracle.unpack_int4(ap).astype(np.int64), oracle.unpack_int4(wp).astype(np.int64)
    full = torch.from_numpy((qa @ qw.T).astype(np.float32))
    exp_ptpc = ((full * .125) * sw1.cpu().float()[None, :]).to(torch.bfloat16)
    assert torch.equal(got.cpu(), exp_ptpc)


@pytest.mark.parametrize("M,N,K", [(17, 96, 512), (33, 136, 4096), (32, 128, 12288)])
def test_k2_per_channel_scale(M, N, K):
    run_case(M, N, K, 20261109 + K, grouped=False)


@pytest.mark.parametrize("M", [1, 2, 15, 16, 17, 31, 33, 47, 48, 49, 63, 64, 65, 100, 127, 128, 129, 257])
def test_k2_m_sweep(M):
    run_case(M, 136, 1024, 1000 + M)
    run_case(M, 264, 256, 2000 + M, grouped=False)
    run_case(M, 272, 512, 2500 + M)  # 17 column blocks: tiled weights, column-block tail in a prefill tile


@pytest.mark.parametrize("M,N,K", [(1, 4104, 4096), (16, 4104, 4096), (17, 4104, 4096), (32, 4104, 4096),
                                   (33, 4104, 4096), (48, 264, 4096), (8, 520, 12288), (16, 264, 8192),
                                   (32, 4112, 4096), (7, 6160, 2048)])
def test_k2_decode_activations_in_lds(M, N, K):
    """Shapes served by the decode kernel (one workgroup per 16 columns, the
    K groups split over its waves, activation slices staged in LDS): every
    M block, a column tail, more 16-column blocks than compute units, K =
    8192 and 12288 (rounds beyond the load ring).  With tiled weights and
    more 16-column blocks than CUs (N = 4112, 6160: 257 and 385 blocks) a
    workgroup takes two column blocks, the last one a single block."""
    run_case(M, N, K, 3000 + M + K)
    if M in (17, 48):
        run_case(M, N, K, 4000 + M + K, grouped=False)


@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (32, 4096, 2176), (16, 4096, 6272), (9, 2048, 3200),
                                   (32, 136, 12160), (20, 4000, 2048), (17, 1024, 12288)])
def test_k2_decode_sixteen_waves(M, N, K):
    """Shapes served by the 16-wave decode kernel (M <= 32, K >= 2048, no
    more 16-column blocks than compute units: 16 K groups per round, a
    two-round load ring): partial last rounds (K/128 = 17, 49, 25, 95), a
    single round (K = 2048), column tails, grouped and per-channel scales."""
    run_case(M, N, K, 7000 + M + K)
    if M in (9, 32):
        run_case(M, N, K, 8000 + M + K, grouped=False)


@pytest.mark.parametrize("M,N,K", [(1, 16392, 4096), (17, 16392, 4096), (32, 16392, 2048), (32, 16384, 4096)])
def test_k2_decode_wide_n(M, N, K):
    """Shapes served by the wide decode kernel (each wave owns 16 columns over
    the whole K, activations resident in LDS): M blocks 1 and 2, row and
    column tails, K = 2048 and 4096, grouped and per-channel scales."""
    run_case(M, N, K, 5000 + M + K)
    if M == 32:
        run_case(M, N, K, 6000 + M + K, grouped=False)


def chain_expected(case, rows=None):
    xb = bf16_bits(case.x)
    if rows is not None:
        xb = xb[rows]
    packed, scale = oracle.rht_quant_pack(xb, case.signs.numpy())
    return packed, scale, oracle.w4a4_gemm(packed, case.w_packed.numpy(), scale, bf16_bits(case.w_scale))


@pytest.mark.parametrize("tiled", [False, True])
@pytest.mark.parametrize("proj", ["o", "qkv", "gate_up", "down"])
def test_k2_chain_qwen3_shapes_m32(proj, tiled):
    case = W.w4a4_case(proj, 32)
    M, N, K = case.shape
    print(f"[chain] {proj} M={M} N={N} K={K} tiled={tiled}", flush=True)
    x, signs = case.x.to(DEV), case.signs.to(DEV)
    wpk, wsc = case.w_packed.to(DEV), case.w_scale.to(DEV)
    if tiled:
        wpk = tile_weights(wpk)
    packed = torch.empty((M, K // 2), dtype=torch.int8, device=DEV)
    scale = torch.empty((M, K // 128), dtype=torch.bfloat16, device=DEV)
    rht_quant_pack(x, signs, out_packed=packed, out_scale=scale)
    out = w4a4_grouped_gemm(packed, wpk, scale, wsc, weights_tiled=tiled)
    torch.cuda.synchronize()
    p_ref, s_ref, o_ref = chain_expected(case)
    assert np.array_equal(packed.cpu().numpy(), p_ref)
    assert np.array_equal(bf16_bits(scale), s_ref)
    assert_bits_equal(bf16_bits(out), o_ref, f"{proj} M=32 chain")


@pytest.mark.parametrize("path", [None, "int8", "fp8"])
@pytest.mark.parametrize("tiled", [False, True])
@pytest.mark.parametrize("proj", ["o", "qkv", "gate_up", "down"])
def test_k2_chain_qwen3_shapes_m4096_sampled(proj, tiled, path):
    """path=None takes the size-chosen kernels (the fp6 matrix cores at
    M = 4096); "int8" the int8 prefill kernel, "fp8" the fp8 one."""
    case = W.w4a4_case(proj, 4096)
    M, N, K = case.shape
    print(f"[chain] {proj} M={M} N={N} K={K} tiled={tiled} path={path} (row sample)", flush=True)
    x, signs = case.x.to(DEV), case.signs.to(DEV)
    wpk, wsc = case.w_packed.to(DEV), case.w_scale.to(DEV)
    if tiled:
        wpk = tile_weights(wpk)
    packed = torch.empty((M, K // 2), dtype=torch.int8, device=DEV)
    scale = torch.empty((M, K // 128), dtype=torch.bfloat16, device=DEV)
    rht_quant_pack(x, signs, out_packed=packed, out_scale=scale)
    out = w4a4_grouped_gemm(packed, wpk, scale, wsc, weights_tiled=tiled, path=path)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([np.arange(0, 3), np.linspace(0, M - 1, 21).round().astype(int),
                                     np.arange(M - 3, M), [127, 128, 129]]))
    p_ref, s_ref, o_ref = chain_expected(case, rows)
    assert np.array_equal(packed.cpu().numpy()[rows], p_ref)
    assert np.array_equal(bf16_bits(scale)[rows], s_ref)
    assert_bits_equal(bf16_bits(out)[rows], o_ref, f"{proj} M=4096 sampled rows")


@pytest.mark.parametrize("proj", ["o", "down", "gate_up"])
def test_k2_chain_m4096_every_row(proj):
    """The prefill-sized chain (K1, then the size-chosen fp6 matrix-core GEMM
    on tiled weights, as W4A4Linear runs it) at M = 4096, every row and
    every element against the oracle's K1 + grouped GEMM."""
    from nv4 import W4A4Linear
    case = W.w4a4_case(proj, 4096)
    M, N, K = case.shape
    print(f"[chain] {proj} M={M} N={N} K={K} every row", flush=True)
    lin = W4A4Linear(K, N).to(DEV)
    lin.assign_quantized_(case.w_packed.to(DEV), case.w_scale.to(DEV), case.signs.to(DEV))
    packed = torch.empty((M, K // 2), dtype=torch.int8, device=DEV)
    scale = torch.empty((M, K // 128), dtype=torch.bfloat16, device=DEV)
    x = case.x.to(DEV)
    rht_quant_pack(x, lin.signs, out_packed=packed, out_scale=scale)
    out = lin.forward_quantized(packed, scale)
    whole = lin(x)
    torch.cuda.synchronize()
    p_ref, s_ref, o_ref = chain_expected(case)
    assert np.array_equal(packed.cpu().numpy(), p_ref)
    assert np.array_equal(bf16_bits(scale), s_ref)
    assert_bits_equal(bf16_bits(out), o_ref, f"{proj} M=4096 every row")
    assert_bits_equal(bf16_bits(whole), o_ref, f"{proj} M=4096 W4A4Linear.forward")


@pytest.mark.parametrize("M", [32, 4096])
def test_k2_chain_config0_block128(M):
    """Config 0 (o_proj, 1 % x20 outlier channels) with the block128 RHT
    layout: K1 on the workload's inputs chained into the grouped GEMM,
    codes, scales and every output element against the oracle."""
    case = W.w4a4_case("o", M)
    _, N, K = case.shape
    print(f"[chain-block128] o M={M}", flush=True)
    x, signs = case.x.to(DEV), case.signs.to(DEV)
    packed = torch.empty((M, K // 2), dtype=torch.int8, device=DEV)
    scale = torch.empty((M, K // 128), dtype=torch.bfloat16, device=DEV)
    rht_quant_pack(x, signs, out_packed=packed, out_scale=scale, layout="block128")
    for tiled in (False, True):
        wpk = case.w_packed.to(DEV)
        out = w4a4_grouped_gemm(packed, tile_weights(wpk) if tiled else wpk, scale, case.w_scale.to(DEV),
                                weights_tiled=tiled)
        torch.cuda.synchronize()
        p_ref, s_ref = oracle.rht_quant_pack(bf16_bits(case.x), case.signs.numpy(), layout=oracle.LAYOUT_BLOCK128)
        assert np.array_equal(packed.cpu().numpy(), p_ref)
        assert np.array_equal(bf16_bits(scale), s_ref)
        o_ref = oracle.w4a4_gemm(p_ref, case.w_packed.numpy(), s_ref, bf16_bits(case.w_scale))
        assert_bits_equal(bf16_bits(out), o_ref, f"block128 chain M={M} tiled={tiled}")


def rtn_inputs(M, N, K, seed):
    """Operands as the reference's kernel benchmarks make them
    (benchmarks/tune_w4a4_aw_grouped.py:41-49): bf16 x ~ N(0,1) and
    w ~ N(0,1)/sqrt(K), a zero row in each (x's kept when M = 1), activations quantized at clip 0.9
    and weights round-to-nearest at clip 1 in groups of 128 (the oracle's
    restatement of grouped_quantize, CUDA division)."""
    rng = np.random.default_rng(seed)
    x = oracle.bf16_to_f32(oracle.f32_to_bf16(rng.standard_normal((M, K)).astype(np.float32)))
    w = oracle.bf16_to_f32(oracle.f32_to_bf16((rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)))
    if M > 1:
        x[0] = 0
    w[0] = 0
    qa, sa = oracle.weight_quantize(x, 128, 0.9, oracle.DIVISION_CUDA)
    qw, sw = oracle.weight_quantize(w, 128, 1.0, oracle.DIVISION_CUDA)
    return x, w, oracle.pack_int4(qa), oracle.pack_int4(qw), sa, sw


@pytest.mark.parametrize("M,N,K", [(1, 6144, 4096), (32, 4096, 12288), (32, 24576, 4096), (600, 528, 4096),
                                   (2048, 1040, 4096)])
def test_k2_rtn_quantized_weights(M, N, K):
    """Realistic per-group weight scales (RTN-G128 of Gaussian weights) through
    the size-chosen kernel, reference and tiled layouts: bit-exact against the
    oracle in bf16; the fp32 output within 2e-6 relative RMSE of the float64
    grouped sum (verify_w4a4_aw_grouped.py:75-76); the W4A4 product within the
    expected INT4 error of the unquantized x @ w.T."""
    print(f"[k2-rtn] M={M} N={N} K={K}", flush=True)
    x, wf, ap, wp, sa, sw = rtn_inputs(M, N, K, M * 3 + N + K)
    exp = oracle.w4a4_gemm(ap, wp, sa, sw)
    a, w, s_a, s_w = to_dev(ap, wp, sa, sw)
    out = w4a4_grouped_gemm(a, w, s_a, s_w)
    out_t = w4a4_grouped_gemm(a, tile_weights(w), s_a, s_w, weights_tiled=True)
    out32 = torch.full((M, N), float("nan"), device=DEV, dtype=torch.float32)
    compile_grouped_gemm(M, N, K, output_fp32=True, weight_grouped=True)(a, w, s_a, s_w, out32)
    torch.cuda.synchronize()
    assert_bits_equal(bf16_bits(out), exp, "bf16 output")
    assert_bits_equal(bf16_bits(out_t), exp, "bf16 output, tiled weights")
    dots = oracle.w4a4_group_dots(ap, wp).astype(np.float64)
    precise = np.einsum("mng,mg,ng->mn", dots, oracle.bf16_to_f32(sa).astype(np.float64),
                        oracle.bf16_to_f32(sw).astype(np.float64))
    got32 = out32.cpu().numpy().astype(np.float64)
    rrmse = np.sqrt(np.mean((got32 - precise) ** 2) / max(np.mean(precise ** 2), 1e-20))
    assert rrmse < 2e-6, rrmse
    st = oracle.error_stats(oracle.bf16_to_f32(bf16_bits(out)), (x.astype(np.float64) @ wf.T.astype(np.float64)))
    assert st["relative_rmse"] < 0.25 and st["cosine"] > 0.97, st


def extreme_scales(rng, rows, G, frac=0.05):
    """bf16 scale bits: ordinary values with a sprinkling of tiny normals
    (2^-126), bf16 subnormals (2^-133), huge values (2^70) and zeros, so the
    scale product can underflow to an fp32 subnormal or exceed 2^63."""
    s = oracle.f32_to_bf16((rng.random((rows, G)) * 0.5 + 0.01).astype(np.float32))
    special = np.array([0x0080, 0x0001, 0x62800000 >> 16, 0x0000, 0x0081], dtype=np.uint16)
    pick = rng.random((rows, G)) < frac
    s[pick] = special[rng.integers(0, len(special), pick.sum())]
    return s


@pytest.mark.parametrize("M,N,K,rows_special", [(200, 264, 1024, True), (257, 392, 2048, False),
                                                 (150, 136, 12288, True), (130, 400, 1024, False)])
def test_k2_prefill_extreme_scales(M, N, K, rows_special):
    """Prefill tiles whose scales leave the range where the kernel folds the
    x256 of the widened nibbles into the activation scale must take the
    literal per-group sequence; tiles next to them keep the short form.
    Only some rows (or some columns) carry the special values, so both forms
    run in one launch.  Bit-exact in bf16 and fp32."""
    print(f"[k2-extreme] M={M} N={N} K={K}", flush=True)
    rng = np.random.default_rng(M * 7 + K)
    ap, wp, _, _ = gemm_inputs(M, N, K, M + N + K)
    G = K // 128
    sa = oracle.f32_to_bf16((rng.random((M, G)) * 2 + 0.01).astype(np.float32))
    sw = oracle.f32_to_bf16((rng.random((N, G)) * 0.03 + 0.001).astype(np.float32))
    if rows_special:
        sa[130:] = extreme_scales(rng, M - 130, G)
    else:
        sw[:128] = extreme_scales(rng, 128, G)
    for out_fp32 in (False, True):
        exp = oracle.w4a4_gemm(ap, wp, sa, sw, out_fp32=out_fp32)
        a, w, s_a, s_w = to_dev(ap, wp, sa, sw)
        if out_fp32:
            out = torch.full((M, N), float("nan"), device=DEV, dtype=torch.float32)
            compile_grouped_gemm(M, N, K, output_fp32=True, weight_grouped=True)(a, w, s_a, s_w, out)
            torch.cuda.synchronize()
            assert_bits_equal(out.cpu().numpy().view(np.uint32), exp.view(np.uint32), "fp32 output")
        else:
            out = w4a4_grouped_gemm(a, w, s_a, s_w)
            torch.cuda.synchronize()
            assert_bits_equal(bf16_bits(out), exp, "bf16 output")
            if N % 16 == 0:
                out = w4a4_grouped_gemm(a, tile_weights(w), s_a, s_w, weights_tiled=True)
                torch.cuda.synchronize()
                assert_bits_equal(bf16_bits(out), exp, "bf16 output, tiled weights")


@pytest.mark.parametrize("M,N,K", [(1000, 1032, 512), (300, 520, 1024), (4096, 264, 2048)])
def test_k2_prefill_tile_orders(M, N, K):
    """Every output of prefill launches whose tile counts are (72, 15, 96) --
    divisible by the 8 XCDs or not -- so every tile of both orderings is
    written exactly once and lands where it belongs."""
    run_case(M, N, K, 7000 + M + N)


@pytest.mark.parametrize("N,K", [(4096, 12288), (6144, 4096), (24576, 4096)])
def test_k2_decode_back_to_back_repeatable(N, K):
    """Decode-sized K2 launched back to back over rotating weight sets (the
    benchmark's pattern, eager and as a replayed graph) gives every call the
    bits of the same call made alone: no state leaks between launches and no
    race inside one."""
    M = 32
    print(f"[k2-repeat] M={M} N={N} K={K}", flush=True)
    g = torch.Generator(device=DEV)
    g.manual_seed(N + K)
    a = torch.randint(-128, 128, (M, K // 2), generator=g, device=DEV, dtype=torch.int16).to(torch.int8)
    sa = (0.01 + torch.rand(M, K // 128, generator=g, device=DEV)).to(torch.bfloat16)
    sets = []
    for _ in range(3):
        w = torch.randint(-128, 128, (N, K // 2), generator=g, device=DEV, dtype=torch.int16).to(torch.int8)
        sw = (0.005 + 0.015 * torch.rand(N, K // 128, generator=g, device=DEV)).to(torch.bfloat16)
        sets.append((tile_weights(w), sw))
    refs = []
    for wt, sw in sets:
        refs.append(w4a4_grouped_gemm(a, wt, sa, sw, weights_tiled=True))
        torch.cuda.synchronize()
    outs = [torch.empty((M, N), dtype=torch.bfloat16, device=DEV) for _ in range(12)]
    for i, o in enumerate(outs):
        wt, sw = sets[i % 3]
        w4a4_grouped_gemm(a, wt, sa, sw, out=o, weights_tiled=True)
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert torch.equal(o.view(torch.int16), refs[i % 3].view(torch.int16)), f"eager call {i}"
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        for i, o in enumerate(outs):
            wt, sw = sets[i % 3]
            w4a4_grouped_gemm(a, wt, sa, sw, out=o, weights_tiled=True)
    for rep in range(3):
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, o in enumerate(outs):
            assert torch.equal(o.view(torch.int16), refs[i % 3].view(torch.int16)), f"replay {rep} call {i}"
