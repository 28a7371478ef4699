"""GPU parity of the decode-step LM head (``nv4_lm_head``, the replacement of
ParallelLMHead.forward's F.linear, nanovllm/layers/embed_head.py:56-61, for
M <= 32 rows) against an fp32 reference of the same product: bf16 inputs,
products summed in fp32, the result rounded to bf16.  Bar: within one bf16
rounding of the fp32 reference plus 2^-20 of the sum of |products| (the
difference between two fp32 summation orders).  Shapes: the Qwen3-8B vocabulary
(151936 rows) at M = 1, 7, 16, 17, 32; row counts that are not a multiple
of the 16-row workgroup tile; hidden sizes 2048, 4096, 5120; h rows read as a
strided view.  Repeated calls give the same bits; the model's compute_logits
takes it in decode.
"""
import pytest
import torch

from nv4.kernels.decoder_ops import lm_head, lm_head_fits

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def check(h, w, out):
    ref = h.float() @ w.float().t()
    absum = h.float().abs() @ w.float().abs().t()
    err = (out.float() - ref).abs()
    bound = ref.abs() * 2.0 ** -8 + absum * 2.0 ** -20 + 1e-30
    bad = (err > bound).sum().item()
    assert bad == 0, f"{bad} of {err.numel()} outside the bound, max err {err.max().item():.3e}"


@pytest.mark.parametrize("M,N,K", [(32, 151936, 4096), (1, 151936, 4096), (7, 151936, 4096), (16, 1000, 4096),
                                   (17, 4099, 4096), (32, 16, 2048), (5, 2053, 5120), (32, 30000, 5120), (32, 200000, 4096), (24, 151936, 2048), (32, 5000, 4096)])
def test_lm_head_matches_fp32_reference(M, N, K):
    g = torch.Generator(device=DEV).manual_seed(M * 131 + N + K)
    print(f"[lm_head] M={M} N={N} K={K}", flush=True)
    hp = torch.randn(M, K + 64, generator=g, device=DEV).to(torch.bfloat16)
    h = hp[:, :K]  # strided rows
    w = (torch.randn(N, K, generator=g, device=DEV) * 0.05).to(torch.bfloat16)
    assert lm_head_fits(h, w)
    out = lm_head(h, w)
    torch.cuda.synchronize()
    check(h, w, out)
    again = lm_head(h, w)
    torch.cuda.synchronize()
    assert torch.equal(out, again)


def test_lm_head_strided_unaligned_output():
    """Output rows at an odd stride (element stores instead of 8-byte ones)."""
    g = torch.Generator(device=DEV).manual_seed(5)
    M, N, K = 32, 3000, 4096
    h = torch.randn(M, K, generator=g, device=DEV).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=DEV) * 0.05).to(torch.bfloat16)
    big = torch.full((M, N + 3), -1.0, dtype=torch.bfloat16, device=DEV)
    out = big[:, 1:N + 1]
    lm_head(h, w, out=out)
    torch.cuda.synchronize()
    check(h, w, out)
    assert torch.equal(out, lm_head(h, w))
    assert (big[:, 0] == -1).all() and (big[:, N + 1:] == -1).all()


def test_lm_head_declines_unsupported_shapes():
    h = torch.zeros(33, 4096, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(64, 4096, dtype=torch.bfloat16, device=DEV)
    assert not lm_head_fits(h, w)
    assert not lm_head_fits(h[:4, :3072].contiguous(), w[:, :3072].contiguous())
    with pytest.raises(ValueError):
        lm_head(h, w)
