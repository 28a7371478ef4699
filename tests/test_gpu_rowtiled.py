"""GPU parity of the row-tiled decode path (M <= 32).

For decode-sized M the W4A4 linear passes the packed activation codes from
K1 to the GEMM in a row-tiled order (16 rows x 128 k per 1 KiB block, in
matrix-core lane order) instead of [M, K/2]; the decode GEMM then loads them
straight into registers.  The order is this build's own (the reference's
rht_quant_pack returns [M, K/2]), so the tests pin it against its definition
and the results against the oracle:

* K1 (plain, add+RMSNorm, SiLU-mul prologues) writes exactly the reference
  codes, untiled, and never touches the rows past M of the last block;
* the row-tiled GEMM equals the oracle's grouped GEMM bit for bit in bf16
  and fp32, grouped and per-channel weight scales, across M = 1..32, the
  narrow-N kernel (8 and 16 waves), the wide-N kernel, partial last rounds
  and column tails; garbage in the unused rows changes nothing;
* the wide-N kernel's scale fold (the x256 of the widened nibbles carried by
  the activation scale) falls back to the literal sequence for workgroups
  whose scales leave [2^-59, 2^63), with the other workgroups still folding;
* ``W4A4Linear`` at M <= 32 (which takes this path) equals the oracle chain.
Bar: bit-exact.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import bf16_bits, bits_to_bf16
from nv4 import W4A4Linear, rht_quant_pack, tile_weights, w4a4_grouped_gemm
from nv4 import workloads as W
from nv4.kernels.decoder_ops import rmsnorm_rht_quant_pack, silu_mul_rht_quant_pack
from nv4.kernels.rht_a4 import rht_quant_pack_rowtiled, rowtiled_rows
from nv4.kernels.decoder_ops import silu_mul
from nv4.kernels.w4a4_grouped import rowtiled_silu_fits, w4a4_gemm_rowtiled, w4a4_gemm_rowtiled_silu

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
CANARY = 0x5A


def rowtile(ap, fill=None, seed=0):
    """Reference-layout packed codes [M, K/2] (numpy int8) -> the row-tiled
    buffer [ceil(M/16)*16, K/2] by its definition: unit (rb*G + g)*64 + 16*part
    + r holds bytes 64*g + 16*part .. +15 of row 16*rb + r.  Rows past M are
    ``fill`` bytes (random when None)."""
    m, kb = ap.shape
    rows = (m + 15) // 16 * 16
    g = kb // 64
    pad = np.empty((rows, kb), dtype=np.int8)
    pad[:m] = ap
    if rows > m:
        pad[m:] = (np.random.default_rng(seed).integers(-128, 128, (rows - m, kb)) if fill is None else fill)
    return np.ascontiguousarray(pad.reshape(rows // 16, 16, g, 4, 16).transpose(0, 2, 3, 1, 4).reshape(rows, kb))


def untile(rt, m):
    rows, kb = rt.shape
    g = kb // 64
    return np.ascontiguousarray(rt.reshape(rows // 16, g, 4, 16, 16).transpose(0, 3, 1, 2, 4).reshape(rows, kb)[:m])


def test_rowtile_helpers_pin_the_layout():
    """The test's own layout helpers against a hand-placed example: row 17,
    packed byte 64*2 + 16*3 + 5 of a K = 512 buffer (G = 4) sits in unit
    (1*4 + 2)*64 + 16*3 + 1, byte 5."""
    ap = np.zeros((20, 256), dtype=np.int8)
    ap[17, 64 * 2 + 16 * 3 + 5] = 7
    rt = rowtile(ap, fill=0)
    flat = rt.reshape(-1)
    unit = (1 * 4 + 2) * 64 + 16 * 3 + 1
    assert flat[unit * 16 + 5] == 7 and np.count_nonzero(flat) == 1
    assert np.array_equal(untile(rt, 20), ap)


@pytest.mark.parametrize("K", [4096, 12288])
@pytest.mark.parametrize("M", [1, 7, 16, 17, 31, 32, 45])
def test_k1_rowtiled_equals_reference_codes(M, K):
    print(f"[k1-rt] M={M} K={K}", flush=True)
    g = torch.Generator().manual_seed(M * 31 + K)
    x = (torch.randn((M, K), generator=g) * 3).to(torch.bfloat16)
    x[0, ::7] *= 40
    signs = (torch.randint(0, 2, (K,), generator=g) * 2 - 1).to(torch.int8)
    xd, sd = x.to(DEV), signs.to(DEV)
    ref_p = torch.empty((M, K // 2), dtype=torch.int8, device=DEV)
    ref_s = torch.empty((M, K // 128), dtype=torch.bfloat16, device=DEV)
    rht_quant_pack(xd, sd, out_packed=ref_p, out_scale=ref_s)
    rt = torch.full((rowtiled_rows(M), K // 2), CANARY, dtype=torch.int8, device=DEV)
    sc = torch.empty((M, K // 128), dtype=torch.bfloat16, device=DEV)
    rht_quant_pack_rowtiled(xd, sd, out_packed=rt, out_scale=sc)
    torch.cuda.synchronize()
    rt_h = rt.cpu().numpy()
    assert np.array_equal(untile(rt_h, M), ref_p.cpu().numpy())
    assert np.array_equal(bf16_bits(sc), bf16_bits(ref_s))
    # rows past M of the last block: never written
    full = untile(rt_h, rowtiled_rows(M))
    assert np.all(full[M:] == CANARY)
    # and the codes are the oracle's
    p_ref, s_ref = oracle.rht_quant_pack(bf16_bits(x), signs.numpy())
    assert np.array_equal(untile(rt_h, M), p_ref) and np.array_equal(bf16_bits(sc), s_ref)


@pytest.mark.parametrize("M", [1, 17, 32])
def test_fused_k1_rowtiled_equals_reference_codes(M):
    print(f"[fused-k1-rt] M={M}", flush=True)
    g = torch.Generator().manual_seed(900 + M)
    x = torch.randn((M, 4096), generator=g).to(torch.bfloat16).to(DEV)
    res = torch.randn((M, 4096), generator=g).to(torch.bfloat16).to(DEV)
    w = (1 + 0.1 * torch.randn(4096, generator=g)).to(torch.bfloat16).to(DEV)
    s4 = (torch.randint(0, 2, (4096,), generator=g) * 2 - 1).to(torch.int8).to(DEV)
    for with_res in (False, True):
        r1, r2 = (res.clone(), res.clone()) if with_res else (None, None)
        p_ref, s_ref = rmsnorm_rht_quant_pack(x, w, 1e-6, s4, r1)[:2]
        p_rt, s_rt = rmsnorm_rht_quant_pack(x, w, 1e-6, s4, r2, rowtiled=True)[:2]
        torch.cuda.synchronize()
        assert tuple(p_rt.shape) == (rowtiled_rows(M), 2048)
        assert np.array_equal(untile(p_rt.cpu().numpy(), M), p_ref.cpu().numpy())
        assert np.array_equal(bf16_bits(s_rt), bf16_bits(s_ref))
        if with_res:
            assert torch.equal(r1, r2)
    for K in (4096, 12288):
        gu = torch.randn((M, 2 * K), generator=g).to(torch.bfloat16).to(DEV)
        sk = (torch.randint(0, 2, (K,), generator=g) * 2 - 1).to(torch.int8).to(DEV)
        p_ref, s_ref = silu_mul_rht_quant_pack(gu, sk)
        p_rt, s_rt = silu_mul_rht_quant_pack(gu, sk, rowtiled=True)
        torch.cuda.synchronize()
        assert np.array_equal(untile(p_rt.cpu().numpy(), M), p_ref.cpu().numpy())
        assert np.array_equal(bf16_bits(s_rt), bf16_bits(s_ref))


def gemm_inputs(M, N, K, seed):
    rng = np.random.default_rng(seed)
    qa = rng.integers(-7, 8, (M, K)).astype(np.int8)
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


def run_rowtiled(ap, wp, sa, sw, what, seed=0):
    M, N = ap.shape[0], wp.shape[0]
    exp = oracle.w4a4_gemm(ap, wp, sa, sw)
    exp32 = oracle.w4a4_gemm(ap, wp, sa, sw, out_fp32=True)
    a_rt = torch.from_numpy(rowtile(ap, seed=seed)).to(DEV)
    wt = tile_weights(torch.from_numpy(wp).to(DEV))
    s_a, s_w = bits_to_bf16(sa).to(DEV), bits_to_bf16(sw).to(DEV)
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    w4a4_gemm_rowtiled(a_rt, wt, s_a, s_w, out=out)
    out32 = torch.full((M, N), float("nan"), dtype=torch.float32, device=DEV)
    w4a4_gemm_rowtiled(a_rt, wt, s_a, s_w, out=out32, output_fp32=True)
    torch.cuda.synchronize()
    got = bf16_bits(out)
    assert np.array_equal(got, exp), f"{what}: {int((got != exp).sum())} of {exp.size} bf16 outputs differ"
    assert np.array_equal(out32.cpu().numpy().view(np.uint32), exp32.view(np.uint32)), f"{what}: fp32 differs"
    return a_rt, wt, s_a, s_w, exp


@pytest.mark.parametrize("M,N,K", [
    (1, 4096, 4096), (5, 6144, 4096), (16, 4096, 12288), (17, 4096, 4096), (32, 4096, 4096),
    (32, 6144, 4096), (32, 4096, 12288),                 # o / qkv / down shapes: 16- and 8-wave kernels
    (9, 272, 2176), (32, 144, 640), (24, 4112, 2048),     # partial last rounds, column tails
    (32, 4112, 4096), (1, 6160, 4096),                    # two column blocks per workgroup, odd last block
    (32, 24576, 4096), (3, 24576, 4096), (32, 16384, 2048),  # wide-N kernel
])
def test_gemm_rowtiled_vs_oracle(M, N, K):
    print(f"[k2-rt] M={M} N={N} K={K}", flush=True)
    ap, wp, sa, sw = gemm_inputs(M, N, K, M * 7 + N + K)
    run_rowtiled(ap, wp, sa, sw, f"M={M} N={N} K={K}")
    if M in (5, 32) and N <= 6144:
        run_rowtiled(ap, wp, sa, sw[:, 0].copy(), f"per-channel M={M} N={N} K={K}")


def test_gemm_rowtiled_ignores_rows_past_m():
    """Different garbage in rows 17..31 of the last block gives the same bits."""
    ap, wp, sa, sw = gemm_inputs(17, 4096, 4096, 4242)
    _, wt, s_a, s_w, exp = run_rowtiled(ap, wp, sa, sw, "seed 1", seed=1)
    for seed in (2, 3):
        a_rt = torch.from_numpy(rowtile(ap, seed=seed)).to(DEV)
        out = w4a4_gemm_rowtiled(a_rt, wt, s_a, s_w)
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(out), exp)


def special_scales(rng, shape, frac):
    s = oracle.f32_to_bf16((rng.random(shape) * 0.5 + 0.01).astype(np.float32))
    special = np.array([0x0080, 0x0001, 0x62800000 >> 16, 0x2000, 0x5f80], dtype=np.uint16)
    pick = rng.random(shape) < frac
    s[pick] = special[rng.integers(0, len(special), pick.sum())]
    return s


@pytest.mark.parametrize("which", ["sw_columns", "sa_rows", "none"])
def test_wide_kernel_scale_fold_fallback(which):
    """gate_up shape (the wide-N kernel).  Scales outside [2^-59, 2^63) --
    tiny normals, bf16 subnormals, 2^70, 2^-64, 2^64 -- in a few weight
    columns (some workgroups fold, the others run the literal sequence) or in
    some activation rows (no workgroup folds); bit-exact either way, in the
    reference-layout and the row-tiled calls."""
    M, N, K = 32, 24576, 4096
    print(f"[k2-fold] {which}", flush=True)
    rng = np.random.default_rng(77 + len(which))
    ap, wp, sa, sw = gemm_inputs(M, N, K, 5150)
    G = K // 128
    if which == "sw_columns":
        cols = rng.choice(N, 40, replace=False)
        sw[cols] = special_scales(rng, (40, G), 0.3)
    elif which == "sa_rows":
        sa[5:9] = special_scales(rng, (4, G), 0.3)
    a_rt, wt, s_a, s_w, exp = run_rowtiled(ap, wp, sa, sw, which)
    out = w4a4_grouped_gemm(torch.from_numpy(ap).to(DEV), wt, s_a, s_w, weights_tiled=True)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(out), exp)


@pytest.mark.parametrize("proj", ["o", "qkv", "gate_up", "down"])
@pytest.mark.parametrize("M", [1, 32])
def test_linear_rowtiled_path_vs_oracle_chain(proj, M):
    """W4A4Linear at decode-sized M (row-tiled K1 -> row-tiled GEMM) equals
    the oracle's K1 + GEMM on the same input."""
    case = W.w4a4_case(proj, M)
    _, N, K = case.shape
    print(f"[linear-rt] {proj} M={M}", flush=True)
    lin = W4A4Linear(K, N).to(DEV)
    lin.assign_quantized_(case.w_packed.to(DEV), case.w_scale.to(DEV), case.signs.to(DEV))
    assert lin.uses_rowtiled(M)
    out = lin(case.x.to(DEV))
    torch.cuda.synchronize()
    p_ref, s_ref = oracle.rht_quant_pack(bf16_bits(case.x), case.signs.numpy())
    exp = oracle.w4a4_gemm(p_ref, case.w_packed.numpy(), s_ref, bf16_bits(case.w_scale))
    assert np.array_equal(bf16_bits(out), exp)


@pytest.mark.parametrize("M", [1, 32])
def test_k1_prefetch_tail_changes_nothing(M):
    """The prefetch workgroups of the row-tiled K1 launches (reading the next
    GEMM's weights into the Infinity Cache) write nothing: codes, scales and
    the residual are the same bits with and without a 48 MiB prefetch, for
    the plain, add+RMSNorm and SiLU-mul K1s."""
    print(f"[k1-prefetch] M={M}", flush=True)
    g = torch.Generator().manual_seed(31 + M)
    buf = torch.randint(-128, 128, (48 << 20,), dtype=torch.int8).to(DEV)
    x = torch.randn((M, 4096), generator=g).to(torch.bfloat16).to(DEV)
    s4 = (torch.randint(0, 2, (4096,), generator=g) * 2 - 1).to(torch.int8).to(DEV)
    a = rht_quant_pack_rowtiled(x, s4)
    b = rht_quant_pack_rowtiled(x, s4, prefetch=buf)
    w = (1 + 0.1 * torch.randn(4096, generator=g)).to(torch.bfloat16).to(DEV)
    res = torch.randn((M, 4096), generator=g).to(torch.bfloat16).to(DEV)
    r1, r2 = res.clone(), res.clone()
    c = rmsnorm_rht_quant_pack(x, w, 1e-6, s4, r1, rowtiled=True)
    d = rmsnorm_rht_quant_pack(x, w, 1e-6, s4, r2, rowtiled=True, prefetch=buf[: 12 << 20])
    gu = torch.randn((M, 2 * 12288), generator=g).to(torch.bfloat16).to(DEV)
    s12 = (torch.randint(0, 2, (12288,), generator=g) * 2 - 1).to(torch.int8).to(DEV)
    e = silu_mul_rht_quant_pack(gu, s12, rowtiled=True)
    f = silu_mul_rht_quant_pack(gu, s12, rowtiled=True, prefetch=buf)
    torch.cuda.synchronize()
    for u, v in ((a, b), (c[:2], d[:2]), (e, f)):  # rows past M of the block are never written: not compared
        assert np.array_equal(untile(u[0].cpu().numpy(), M), untile(v[0].cpu().numpy(), M))
        assert torch.equal(u[1].view(torch.int16), v[1].view(torch.int16))
    assert torch.equal(r1.view(torch.int16), r2.view(torch.int16))


@pytest.mark.parametrize("M,N,K", [(1, 24576, 4096), (7, 24576, 4096), (16, 24576, 4096), (17, 24576, 4096),
                                   (32, 24576, 4096), (32, 24544, 4096), (9, 16384, 2048)])
def test_gemm_rowtiled_silu_equals_gemm_then_silu(M, N, K):
    """The gate/up GEMM with SiLU-and-mul in its epilogue gives exactly the
    bits of the row-tiled GEMM (itself bit-exact with the oracle) followed by
    silu_mul: gate columns n < N/2 paired with up columns N/2 + n; M blocks 1
    and 2, a partial last workgroup (N = 24544: 767 output blocks, 3 per
    workgroup), 4 column blocks per workgroup (N = 16384, K = 2048), grouped and
    per-channel weight scales."""
    print(f"[k2-silu] M={M} N={N} K={K}", flush=True)
    assert rowtiled_silu_fits(M, N, K, DEV)
    ap, wp, sa, sw = gemm_inputs(M, N, K, 11 * M + N + K)
    a_rt = torch.from_numpy(rowtile(ap)).to(DEV)
    wt = tile_weights(torch.from_numpy(wp).to(DEV))
    s_a = bits_to_bf16(sa).to(DEV)
    for grouped in (True, False):
        s_w = bits_to_bf16(sw if grouped else sw[:, 0].copy()).to(DEV)
        two = silu_mul(w4a4_gemm_rowtiled(a_rt, wt, s_a, s_w))
        out = torch.full((M, N // 2), float("nan"), dtype=torch.bfloat16, device=DEV)
        got = w4a4_gemm_rowtiled_silu(a_rt, wt, s_a, s_w, out=out)
        torch.cuda.synchronize()
        assert got.data_ptr() == out.data_ptr()
        assert np.array_equal(bf16_bits(out), bf16_bits(two)), f"grouped={grouped}"
    if M == 32 and N == 24576:
        exp = oracle.w4a4_gemm(ap, wp, sa, sw)   # the GEMM half against the oracle once more
        assert np.array_equal(bf16_bits(w4a4_gemm_rowtiled(a_rt, wt, s_a, bits_to_bf16(sw).to(DEV))), exp)
