"""GPU checks of K3 (W4A16 GPTQ GEMM) and of the drop-in modules.

K3 has no reference test (nanovllm/layers/linear_w4a16.py is exercised by no
script) and the reference kernel sums split-K partials with BF16 atomics in a
nondeterministic order, so its exact bits are unpinnable.  The dense
dequantization used for prefill-sized M (nv4_w4a16_dequant) is bit-exact with
the oracle's rounded dequantized weights.  The GEMM bar here is
the BF16/FP16 GEMM tolerance: every output within 1e-2 relative of the float64
product of the activations and the oracle's dequantised weights, measured as
|out - ref| <= 1e-2 * max(|ref|, rms(ref)) elementwise, plus bit-exact
determinism across calls.

W4A4Linear / W4A16Linear: same buffers and shapes as the reference modules,
forward equal to the oracle chain, and HIP-graph capture replayed several
times with eager work in between.
"""
import numpy as np
import pytest
import torch

import oracle
from conftest import bf16_bits, f16_bits
from nv4 import W4A4Linear, W4A16Linear, dequant_matmul_w4a16
from nv4.kernels import dequant_w4a16
from nv4 import workloads as W

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-2


def check_close(out, ref):
    out = out.detach().float().cpu().numpy().astype(np.float64)
    rms = np.sqrt((ref ** 2).mean())
    err = np.abs(out - ref)
    bound = TOL * np.maximum(np.abs(ref), rms)
    assert np.all(err <= bound), f"max err {err.max():.3e}, worst ratio {(err / bound).max():.3f}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M", [1, 8, 9, 16, 17, 31, 32, 33, 64, 65, 100, 300])
def test_k3_w4a16_qkv(M, dtype):
    print(f"[k3] M={M} dtype={dtype}", flush=True)
    case = W.w4a16_case(M, dtype=dtype)
    xd = oracle.X_FP16 if dtype == torch.float16 else oracle.X_BF16
    xbits = f16_bits(case.x)
    ref = oracle.w4a16_gemm(xbits, case.qweight.numpy(), case.qzeros.numpy(),
                            case.scales.numpy().view(np.uint16), x_dtype=xd)
    x, qw, qz, sc = (t.to(DEV) for t in (case.x, case.qweight, case.qzeros, case.scales))
    out = dequant_matmul_w4a16(x, qw, qz, sc)
    out2 = dequant_matmul_w4a16(x, qw, qz, sc)
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == (M, 6144)
    check_close(out, ref)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("N,K", [(6144, 4096), (136, 512), (4096, 12288)])
def test_dense_dequant_bit_exact(N, K, dtype):
    case = W.w4a16_case(1, N=N, K=K, dtype=dtype)
    xd = oracle.X_FP16 if dtype == torch.float16 else oracle.X_BF16
    ref = oracle.w4a16_dequant(case.qweight.numpy(), case.qzeros.numpy(), case.scales.numpy().view(np.uint16),
                               x_dtype=xd)
    w = dequant_w4a16(*(t.to(DEV) for t in (case.qweight, case.qzeros, case.scales)), dtype=dtype)
    torch.cuda.synchronize()
    assert w.dtype == dtype and tuple(w.shape) == (K, N)
    assert np.array_equal(w.float().cpu().numpy(), ref.astype(np.float32))


@pytest.mark.parametrize("M", [5, 12])
@pytest.mark.parametrize("N,K", [(64, 128), (136, 512), (4096, 12288), (40, 4096)])
def test_k3_shapes(N, K, M):
    case = W.w4a16_case(M, N=N, K=K, dtype=torch.bfloat16)
    ref = oracle.w4a16_gemm(bf16_bits(case.x), case.qweight.numpy(), case.qzeros.numpy(),
                            case.scales.numpy().view(np.uint16), x_dtype=oracle.X_BF16)
    out = dequant_matmul_w4a16(*(t.to(DEV) for t in (case.x, case.qweight, case.qzeros, case.scales)))
    torch.cuda.synchronize()
    check_close(out, ref)


@pytest.mark.parametrize("M,N,K", [(20, 4104, 2048), (32, 8192, 4096), (17, 6144, 640), (32, 4104, 3968),
                                   (32, 6144, 4096), (3, 264, 8320), (16, 4096, 12288), (9, 24576, 4096),
                                   (1, 8, 128), (16, 136, 4224)])
def test_k3_one_launch_shapes(M, N, K):
    """Shapes the one-launch decode kernel takes: one and two row blocks
    (rows past M repeat row M - 1), a column tail (N = 4104, 136, 264, 8),
    fewer groups than waves (K = 640, 128), several passes over K (K = 8320,
    12288, 4224: a last pass with a single live round), the widest N of the
    model (gate/up); fp16 and bf16 activations; deterministic across calls and
    taken without a workspace."""
    from nv4.kernels.w4a16 import one_launch
    assert one_launch(M, N, K, DEV)
    for dtype in (torch.bfloat16, torch.float16):
        case = W.w4a16_case(M, N=N, K=K, dtype=dtype)
        xd = oracle.X_FP16 if dtype == torch.float16 else oracle.X_BF16
        ref = oracle.w4a16_gemm(f16_bits(case.x), case.qweight.numpy(), case.qzeros.numpy(),
                                case.scales.numpy().view(np.uint16), x_dtype=xd)
        args = [t.to(DEV) for t in (case.x, case.qweight, case.qzeros, case.scales)]
        out = dequant_matmul_w4a16(*args)
        out2 = dequant_matmul_w4a16(*args)
        torch.cuda.synchronize()
        check_close(out, ref)
        assert torch.equal(out, out2)


def test_w4a16_linear_module():
    mod = W4A16Linear(4096, 6144).to(DEV)
    case = W.w4a16_case(6, dtype=torch.bfloat16)
    with torch.no_grad():
        mod.qweight.copy_(case.qweight)
        mod.qzeros.copy_(case.qzeros)
        mod.scales.copy_(case.scales)
    assert {k: tuple(v.shape) for k, v in mod.state_dict().items()} == {
        "qweight": (512, 6144), "qzeros": (32, 768), "scales": (32, 6144)}
    x = case.x.to(DEV).view(2, 3, 4096)
    y = mod(x)
    torch.cuda.synchronize()
    assert y.shape == (2, 3, 6144)
    ref = oracle.w4a16_gemm(bf16_bits(case.x), case.qweight.numpy(), case.qzeros.numpy(),
                            case.scales.numpy().view(np.uint16), x_dtype=oracle.X_BF16)
    check_close(y.view(6, 6144), ref)


def test_tl_dequant_matmul_w4a16_reference_call():
    """The reference's call (linear_w4a16.py:138-146): zeroed C, tiles 16/64/32,
    split 8; C += A @ deq(B).  A second call adds the product again."""
    from nv4.layers import tl_dequant_matmul_w4a16
    case = W.w4a16_case(5, N=512, K=1024, dtype=torch.bfloat16)
    x, qw, qz, sc = (t.to(DEV) for t in (case.x, case.qweight, case.qzeros, case.scales))
    C = torch.zeros((5, 512), device=DEV, dtype=torch.bfloat16)
    assert tl_dequant_matmul_w4a16(x, qw, C, sc, qz, 16, 64, 32, 8, 128) is C
    torch.cuda.synchronize()
    direct = dequant_matmul_w4a16(x, qw, qz, sc)
    assert torch.equal(C, direct)
    tl_dequant_matmul_w4a16(x, qw, C, sc, qz, 16, 64, 32, 8, 128)
    assert torch.equal(C, (direct.float() + direct.float()).to(torch.bfloat16))


def load_w4a4(mod, case):
    with torch.no_grad():
        mod.packed_weight.copy_(case.w_packed)
        mod.weight_scale.copy_(case.w_scale)
        mod.signs.copy_(case.signs)


@pytest.mark.parametrize("proj", ["qkv", "down"])
def test_w4a4_linear_module_and_graph(proj):
    N, K = W.PROJECTIONS[proj]
    mod = W4A4Linear(K, N).to(DEV)
    assert {k: (tuple(v.shape), v.dtype) for k, v in mod.state_dict().items()} == {
        "packed_weight": ((N, K // 2), torch.int8), "weight_scale": ((N, K // 128), torch.bfloat16),
        "signs": ((K,), torch.int8)}
    case = W.w4a4_case(proj, 12)
    load_w4a4(mod, case)
    x = case.x.to(DEV).view(3, 4, K)
    y = mod(x)
    torch.cuda.synchronize()
    assert y.shape == (3, 4, N) and y.dtype == torch.bfloat16
    packed, scale = oracle.rht_quant_pack(bf16_bits(case.x), case.signs.numpy())
    ref = oracle.w4a4_gemm(packed, case.w_packed.numpy(), scale, bf16_bits(case.w_scale))
    assert np.array_equal(bf16_bits(y.view(12, N)), ref)

    # Graph capture of the module forward; replays see updated inputs.
    static_x = x.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            mod(static_x)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_y = mod(static_x)
    for i in range(3):
        static_x.copy_(x * (1.0 + 0.25 * i))
        g.replay()
        torch.cuda.synchronize()
        eager = mod(static_x)
        torch.cuda.synchronize()
        assert torch.equal(static_y, eager), f"graph replay {i} differs from eager"
