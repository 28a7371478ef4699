"""GPU parity of the W4A4 linear forward as one operator call (``nv4_w4a4_linear``).

The reference's ``W4A4Linear.forward`` (nanovllm/layers/linear_w4a4.py:27-35)
is rht_quant_pack followed by w4a4_grouped_gemm; the one-call operator must
give the same bits as the oracle chain -- codes, scales and bf16 outputs --
for the four Qwen3-8B projections across the decode and prefill kernels,
repeated calls, a non-default stream and HIP-graph replay after the inputs
change -- with the weights in the reference layout and in the MFMA-tiled
layout that ``W4A4Linear.tile_weights_()`` switches the module to (its
state dict keeps the reference layout).  Bar: bit-exact.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import bf16_bits
from nv4 import W4A4Linear, tile_weights, w4a4_linear
from nv4 import workloads as W

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def expected(case):
    xb = bf16_bits(case.x)
    packed, scale = oracle.rht_quant_pack(xb, case.signs.numpy())
    return packed, scale, oracle.w4a4_gemm(packed, case.w_packed.numpy(), scale, bf16_bits(case.w_scale))


def run(case, stream=None, tiled=False):
    M, N, K = case.shape
    x, signs = case.x.to(DEV), case.signs.to(DEV)
    wp, ws = case.w_packed.to(DEV), case.w_scale.to(DEV)
    if tiled:
        wp = tile_weights(wp)
    packed = torch.full((M, K // 2), 85, dtype=torch.int8, device=DEV)
    scale = torch.full((M, K // 128), float("nan"), dtype=torch.bfloat16, device=DEV)
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    with torch.cuda.stream(stream or torch.cuda.current_stream()):
        w4a4_linear(x, signs, wp, ws, out=out, out_packed=packed, out_scale=scale, weights_tiled=tiled)
    torch.cuda.synchronize()
    return packed, scale, out


def check(case, got, what):
    p_ref, s_ref, o_ref = expected(case)
    packed, scale, out = got
    assert np.array_equal(packed.cpu().numpy(), p_ref), f"{what}: packed codes differ"
    assert np.array_equal(bf16_bits(scale), s_ref), f"{what}: scales differ"
    bad = np.argwhere(bf16_bits(out) != o_ref)
    assert bad.size == 0, f"{what}: {len(bad)} outputs differ, first {bad[:5].tolist()}"


@pytest.mark.parametrize("tiled", [False, True])
@pytest.mark.parametrize("proj", ["o", "qkv", "gate_up", "down"])
@pytest.mark.parametrize("M", [1, 7, 32])
def test_linear_qwen3_shapes(proj, M, tiled):
    print(f"[linear] {proj} M={M} tiled={tiled}", flush=True)
    case = W.w4a4_case(proj, M)
    check(case, run(case, tiled=tiled), f"{proj} M={M} tiled={tiled}")


@pytest.mark.parametrize("M", [16, 17, 33, 48, 64, 65])
def test_linear_m_blocks(M):
    """Every decode row-block count, and M = 65 (the prefill GEMM)."""
    for proj in ("o", "down"):
        print(f"[linear] {proj} M={M}", flush=True)
        case = W.w4a4_case(proj, M, seed=W.BASE_SEED + M)
        check(case, run(case), f"{proj} M={M}")
        check(case, run(case, tiled=True), f"{proj} M={M} tiled")


def test_module_tiled_weights_and_state_dict():
    """W4A4Linear.tile_weights_(): same outputs; state_dict() returns and
    load_state_dict() accepts the reference [out, in/2] layout."""
    case = W.w4a4_case("qkv", 32)
    x = case.x.to(DEV)
    m = W4A4Linear(4096, 6144).to(DEV)
    with torch.no_grad():
        m.packed_weight.copy_(case.w_packed)
        m.weight_scale.copy_(case.w_scale)
        m.signs.copy_(case.signs)
    plain = m(x)
    _, _, o_ref = expected(case)
    assert np.array_equal(bf16_bits(plain), o_ref)
    m.tile_weights_()
    assert m.weights_tiled and not torch.equal(m.packed_weight.cpu(), case.w_packed)
    assert torch.equal(m(x), plain)
    sd = m.state_dict()
    assert torch.equal(sd["packed_weight"].cpu(), case.w_packed)
    m2 = W4A4Linear(4096, 6144).to(DEV).tile_weights_()
    m2.load_state_dict(sd)
    assert m2.weights_tiled and torch.equal(m2.packed_weight, m.packed_weight)
    assert torch.equal(m2(x), plain)


def test_linear_repeated_calls_and_stream():
    case = W.w4a4_case("gate_up", 32)
    for _ in range(3):
        check(case, run(case), "repeat")
    side = torch.cuda.Stream()
    check(case, run(case, stream=side), "side stream")


@pytest.mark.parametrize("proj", ["o", "gate_up"])
def test_linear_graph_replay(proj):
    """Capture once; replay after changing x, with eager work between replays."""
    case = W.w4a4_case(proj, 32)
    M, N, K = case.shape
    x = case.x.to(DEV)
    signs, wp, ws = case.signs.to(DEV), case.w_packed.to(DEV), case.w_scale.to(DEV)
    packed = torch.empty((M, K // 2), dtype=torch.int8, device=DEV)
    scale = torch.empty((M, K // 128), dtype=torch.bfloat16, device=DEV)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        w4a4_linear(x, signs, wp, ws, out=out, out_packed=packed, out_scale=scale)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        w4a4_linear(x, signs, wp, ws, out=out, out_packed=packed, out_scale=scale)
    for step, delta in enumerate((0.0, 0.125, -0.25)):
        new_x = (case.x.float() + delta).to(torch.bfloat16)
        x.copy_(new_x)
        g.replay()
        torch.cuda.synchronize()
        shifted = W.W4A4Case(case.name, new_x, case.signs, case.w_packed, case.w_scale)
        check(shifted, (packed, scale, out), f"{proj} replay {step}")


@pytest.mark.parametrize("proj,M", [("qkv", 2048), ("down", 1024), ("gate_up", 1100)])
def test_linear_prefill_matrix_core_route(proj, M):
    """At prefill-sized M ``w4a4_linear`` runs K1 and then the fp6 matrix-core
    GEMM: its codes, scales and output equal K1 followed by the int8 path, bit
    for bit, in both weight layouts."""
    from nv4 import rht_quant_pack, w4a4_grouped_gemm
    from nv4.kernels.w4a4_grouped import use_prefill_path
    case = W.w4a4_case(proj, M)
    M, N, K = case.shape
    assert use_prefill_path(M, N, K)
    print(f"[linear-prefill] {proj} M={M} N={N} K={K}", flush=True)
    x, signs = case.x.to(DEV), case.signs.to(DEV)
    wpk, wsc = case.w_packed.to(DEV), case.w_scale.to(DEV)
    for tiled in (False, True):
        w = tile_weights(wpk) if tiled else wpk
        packed = torch.empty((M, K // 2), dtype=torch.int8, device=DEV)
        scale = torch.empty((M, K // 128), dtype=torch.bfloat16, device=DEV)
        out = w4a4_linear(x, signs, w, wsc, out_packed=packed, out_scale=scale, weights_tiled=tiled)
        p2 = torch.empty_like(packed)
        s2 = torch.empty_like(scale)
        rht_quant_pack(x, signs, out_packed=p2, out_scale=s2)
        ref = w4a4_grouped_gemm(p2, w, s2, wsc, weights_tiled=tiled, path="int8")
        torch.cuda.synchronize()
        assert torch.equal(packed, p2) and torch.equal(scale.view(torch.int16), s2.view(torch.int16))
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"tiled={tiled}"


def test_linear_module_keeps_fp6_weights():
    """The fp6 form of the weights is opt-in (``keep_weights_f6``): off by
    default; when kept (not for gate_up's size) prefill-sized forwards use it,
    with the bits of converting per call; it stays out of the state dict,
    follows ``load_state_dict``, and is not used once ``packed_weight`` is
    written in place."""
    from nv4 import weights_to_f6
    assert W4A4Linear(4096, 24576, keep_weights_f6=True).to(DEV).tile_weights_().weight_f6 is None
    case = W.w4a4_case("qkv", 1024)
    M, N, K = case.shape
    print(f"[linear-fp6-weights] M={M} N={N} K={K}", flush=True)
    x = case.x.to(DEV)
    plain = W4A4Linear(K, N).to(DEV)
    plain.assign_quantized_(case.w_packed.to(DEV), case.w_scale.to(DEV), case.signs.to(DEV))
    assert plain.weights_tiled and plain.weight_f6 is None and plain._f6() is None
    assert plain.weight_bytes() == N * K // 2 + N * K // 128 * 2 + K
    m = W4A4Linear(K, N, keep_weights_f6=True).to(DEV)
    m.assign_quantized_(case.w_packed.to(DEV), case.w_scale.to(DEV), case.signs.to(DEV))
    assert m.weights_tiled and m._f6() is m.weight_f6 is not None
    assert m.weight_bytes() == plain.weight_bytes() + m.weight_f6.numel()
    assert "weight_f6" not in m.state_dict()
    assert torch.equal(m.weight_f6, weights_to_f6(case.w_packed.to(DEV)))
    out = m(x)
    ref = w4a4_linear(x, m.signs, m.packed_weight, m.weight_scale, weights_tiled=True)   # converts per call
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(plain(x).view(torch.int16), out.view(torch.int16))
    with torch.no_grad():
        m.packed_weight[:64].zero_()                  # in place: the fp6 copy is now stale
    assert m._f6() is None
    out2 = m(x)
    ref2 = w4a4_linear(x, m.signs, m.packed_weight, m.weight_scale, weights_tiled=True)
    torch.cuda.synchronize()
    assert torch.equal(out2.view(torch.int16), ref2.view(torch.int16))
    assert not torch.equal(out2.view(torch.int16), out.view(torch.int16))
    m2 = W4A4Linear(K, N).to(DEV).keep_weights_f6_(True).tile_weights_()
    m2.load_state_dict(m.state_dict())
    assert m2._f6() is not None and torch.equal(m2.weight_f6, weights_to_f6(m.packed_weight, True))
    assert torch.equal(m2(x).view(torch.int16), out2.view(torch.int16))
    m2.keep_weights_f6_(False)
    assert m2.weight_f6 is None and m2._f6() is None


def test_linear_fp6_weights_refused_under_inference_mode():
    """Weights created under torch.inference_mode carry no version counter,
    so an in-place write could not be noticed: such a layer keeps no fp6
    copy even when asked, and a prefill-sized forward after writing new
    weights in place (under inference_mode) follows them, bit for bit with
    the oracle's K1 + GEMM chain on the new weights."""
    case = W.w4a4_case("down", 1024)
    M, N, K = case.shape
    print(f"[linear-fp6-inference-mode] M={M} N={N} K={K}", flush=True)
    rows = np.r_[0:8, 517:521, M - 8:M]
    g = torch.Generator().manual_seed(4321)
    new_w = torch.randint(-128, 128, (N, K // 2), generator=g, dtype=torch.int16).to(torch.int8)
    with torch.inference_mode():
        m = W4A4Linear(K, N, keep_weights_f6=True).to(DEV)
        m.assign_quantized_(case.w_packed.to(DEV), case.w_scale.to(DEV), case.signs.to(DEV))
        assert m.weight_f6 is None and m._f6() is None
        x = case.x.to(DEV)
        out = m(x)
        ref = w4a4_linear(x, m.signs, m.packed_weight, m.weight_scale, weights_tiled=True)
        # new weights written in place, through the tiled layout the module keeps
        m.packed_weight.copy_(tile_weights(new_w.to(DEV)))
        out2 = m(x)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    xb = bf16_bits(case.x)[rows]
    p_ref, s_ref = oracle.rht_quant_pack(xb, case.signs.numpy())
    exp = oracle.w4a4_gemm(p_ref, new_w.numpy(), s_ref, bf16_bits(case.w_scale))
    assert np.array_equal(bf16_bits(out2)[rows], exp)
    assert not torch.equal(out2.view(torch.int16), out.view(torch.int16))
