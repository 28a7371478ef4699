"""GPU parity of K1 (RHT + group-128 quantization + packing) against the oracle.

Restates the reference's kernel checks (benchmarks/bench_rht_a4.py:55-154,
benchmarks/verify_rht_a4_extremes.py): exact codes and BF16 scales over
M in {1,7,17,31,32,33,4096,4097} x K in {4096,12288}, outputs pre-filled with
85/NaN, 64-element canaries on both sides, inputs unchanged, two calls, a
non-default stream, HIP-graph replay after mutating x and the signs, BF16
exponent extremes, and a negative control.  The bar is bit-exact (stricter
than the >=99.9 % / +-1 code agreement allowed for this path).
"""
import math

import numpy as np
import pytest
import torch

import oracle
from conftest import bf16_bits
from nv4 import rht_quant_pack
from nv4 import workloads as W

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def make_input(m, k, seed=W.BASE_SEED):
    return W.special_rows(m, k, seed)


def gold(x_cpu, signs_cpu, layout=oracle.LAYOUT_REFERENCE):
    p, s = oracle.rht_quant_pack(bf16_bits(x_cpu), signs_cpu.numpy(), layout=layout)
    return p, s


def compare(packed, scale, gold_packed, gold_scale):
    got_codes = oracle.unpack_int4(packed.cpu().numpy())
    ref_codes = oracle.unpack_int4(gold_packed)
    bad_codes = int((got_codes != ref_codes).sum())
    bad_scales = int((bf16_bits(scale) != gold_scale).sum())
    assert bad_codes == bad_scales == 0, (
        f"Quantizer parity failed: {bad_codes} codes, {bad_scales} BF16 scales differ")


def check_case(fn, x_cpu, signs_cpu, layout="reference", gold_pair=None):
    m, k = x_cpu.shape
    print(f"[k1] M={m} K={k} layout={layout}", flush=True)
    x = x_cpu.to(DEV)
    signs = signs_cpu.to(DEV)
    x_before, signs_before = x.clone(), signs.clone()
    if gold_pair is None:
        gold_pair = gold(x_cpu, signs_cpu, oracle.LAYOUT_BLOCK128 if layout == "block128" else 0)
    packed_store = torch.full((m * k // 2 + 128,), -69, dtype=torch.int8, device=DEV)
    scale_store = torch.full((m * k // 128 + 128,), -17, dtype=torch.bfloat16, device=DEV)
    packed = packed_store[64:-64].view(m, k // 2)
    scale = scale_store[64:-64].view(m, k // 128)
    for _ in range(2):
        packed.fill_(85)
        scale.fill_(float("nan"))
        kw = {} if layout == "reference" else {"layout": layout}
        ret = fn(x, signs, out_packed=packed, out_scale=scale, **kw)
        torch.cuda.synchronize()
        assert isinstance(ret, tuple) and len(ret) == 2
        assert ret[0].data_ptr() == packed.data_ptr() and ret[1].data_ptr() == scale.data_ptr()
        compare(packed, scale, *gold_pair)
        assert torch.isfinite(scale).all() and (scale > 0).all()
        assert (packed_store[:64] == -69).all() and (packed_store[-64:] == -69).all()
        assert (scale_store[:64] == -17).all() and (scale_store[-64:] == -17).all()
        assert torch.equal(x, x_before) and torch.equal(signs, signs_before)


@pytest.mark.parametrize("k", [4096, 12288])
@pytest.mark.parametrize("m", [1, 7, 17, 31, 32, 33, 64, 65, 200, 256, 257, 4096, 4097])
def test_k1_exact(m, k):
    check_case(rht_quant_pack, make_input(m, k), W.signs(k, 20261108 + k))


@pytest.mark.parametrize("k", [4096, 12288])
@pytest.mark.parametrize("m", [32, 33])
def test_k1_exponent_extremes(m, k):
    # verify_rht_a4_extremes.py:25-37
    exponents = [-130, -126, -120, -80, -30, 0, 30, 80, 100]
    g = torch.Generator("cpu").manual_seed(20261108 + m + k)
    x = torch.randn(m, k, generator=g, dtype=torch.float32)
    e = torch.tensor([exponents[i % len(exponents)] for i in range(m)], dtype=torch.int32)
    x = torch.ldexp(x, e[:, None].float()).to(torch.bfloat16).contiguous()
    x[-1].zero_()
    assert torch.isfinite(x).all()
    check_case(rht_quant_pack, x, W.signs(k, 7 + k))


def coarse_rows(m, k, seed):
    """Rows of a few small integers: their rotated values often sit exactly
    on half-integer multiples of the group scale (quantization ties)."""
    rng = np.random.default_rng(seed)
    pool = np.array([0, 0, 0, 1, -1, 2, -2, 3], np.float32)
    vals = rng.choice(pool, size=(m, k)) if seed % 2 else rng.integers(-1, 2, (m, k)).astype(np.float32)
    return torch.from_numpy(vals).to(torch.bfloat16)


def exact_ties(x_cpu, signs_cpu):
    rotated = oracle.rht_rows(bf16_bits(x_cpu), signs_cpu.numpy())
    _, scales = oracle.quantize_rows(rotated)
    s = np.repeat(oracle.bf16_to_f32(scales).astype(np.float64), 128, axis=1)
    q = rotated.astype(np.float64) / s
    return int((np.abs(q - np.floor(q) - 0.5) == 0).sum())


@pytest.mark.parametrize("seed", [1, 2])
@pytest.mark.parametrize("k", [4096, 12288])
def test_k1_quantization_ties(k, seed):
    """Values exactly halfway between two codes round to the even code (IEEE
    quotient, rint); the kernel's reciprocal fast path must hand them to the
    exact division."""
    x_cpu, signs_cpu = coarse_rows(33, k, seed), W.signs(k, seed)
    if k == 4096:
        assert exact_ties(x_cpu, signs_cpu) >= 50, "input no longer exercises ties"
    check_case(rht_quant_pack, x_cpu, signs_cpu)


@pytest.mark.parametrize("k", [4096, 12288])
def test_k1_workload_activations(k):
    # The benchmark inputs: 1 % x20 outlier channels (configs 0/2) or silu(g)*u (config 3).
    case = W.w4a4_case("down" if k == 12288 else "o", 32)
    check_case(rht_quant_pack, case.x, case.signs)


@pytest.mark.parametrize("k", [128, 512, 4096, 12288])
@pytest.mark.parametrize("m", [1, 3, 33])
def test_k1_block128_layout(m, k):
    check_case(rht_quant_pack, make_input(m, k) if k >= 4096 else
               torch.randn(m, k, generator=torch.Generator("cpu").manual_seed(m + k)).to(torch.bfloat16),
               W.signs(k, 99 + k), layout="block128")


@pytest.mark.parametrize("k", [4096, 12288])
def test_k1_stream_and_graph_replay(k):
    # bench_rht_a4.py:92-115
    print(f"[k1-dynamic] K={k}", flush=True)
    x_cpu = make_input(32, k)
    signs_cpu = W.signs(k, 5 + k)
    x, signs = x_cpu.to(DEV), signs_cpu.to(DEV)
    packed = torch.empty((32, k // 2), dtype=torch.int8, device=DEV)
    scale = torch.empty((32, k // 128), dtype=torch.bfloat16, device=DEV)

    def invoke():
        return rht_quant_pack(x, signs, out_packed=packed, out_scale=scale)
    for _ in range(3):
        invoke()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        packed.fill_(0)
        invoke()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    compare(packed, scale, *gold(x_cpu, signs_cpu))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        invoke()
    for offset in [.125, -.25]:
        x.add_(offset)
        signs.neg_()
        packed.fill_(85)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        compare(packed, scale, *gold(x.cpu(), signs.cpu()))
        # eager work between replays
        invoke()
        torch.cuda.synchronize()
        compare(packed, scale, *gold(x.cpu(), signs.cpu()))


def test_k1_negative_control():
    # bench_rht_a4.py:142-152: a comparison that accepts a corrupted answer is useless.
    x_cpu = make_input(1, 4096)
    signs_cpu = W.signs(4096, 1)

    def corrupt(x, signs, *, out_packed, out_scale):
        rht_quant_pack(x, signs, out_packed=out_packed, out_scale=out_scale)
        out_packed[0, 0].bitwise_xor_(1)
        return out_packed, out_scale
    with pytest.raises(AssertionError, match="Quantizer parity failed"):
        check_case(corrupt, x_cpu, signs_cpu)
