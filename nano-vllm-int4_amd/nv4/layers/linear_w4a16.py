"""GPTQ W4A16 linear (MI355X).

Drop-in for ``nanovllm.layers.linear_w4a16.W4A16Linear`` (reference
nanovllm/layers/linear_w4a16.py:98-148): same constructor, the same
parameters (``qweight`` int32 [in/8, out], ``qzeros`` int32 [in/128, out/8],
``scales`` fp16 [in/128, out], all ``requires_grad=False``), same forward
shape handling.  The GEMM is the HIP kernel ``nv4_w4a16_gemm``.
"""
import torch
from torch import nn

from ..kernels.w4a16 import dequant_matmul_w4a16


def tl_dequant_matmul_w4a16(A, B, C, scales, qzeros, BLOCK_M, BLOCK_N, BLOCK_K, SPLIT_K, group_size):
    """Same call as the reference kernel (linear_w4a16.py:11-59): ``C += A @ deq(B)``.

    The reference accumulates split-K partials into ``C`` with bf16 atomics and is
    only called with a zeroed ``C`` (linear_w4a16.py:132-146); here the whole-K
    product is computed once and added to ``C``.  The tile and split arguments
    are accepted for compatibility and do not change the result.
    """
    for v in (BLOCK_M, BLOCK_N, BLOCK_K, SPLIT_K):
        if int(v) < 1:
            raise ValueError("tile and split sizes must be positive")
    if C.dtype != torch.bfloat16 or tuple(C.shape) != (A.shape[0], B.shape[1]):
        raise ValueError("C must be BF16 [M, N]")
    C.add_(dequant_matmul_w4a16(A, B, qzeros, scales, group_size))
    return C


class W4A16Linear(nn.Module):

    def __init__(self, in_features, out_features, group_size=128):
        super().__init__()
        assert group_size == 128
        self.in_features = in_features
        self.out_features = out_features
        self.group_size = group_size
        self.qweight = nn.Parameter(torch.empty(in_features // 8, out_features, dtype=torch.int32),
                                    requires_grad=False)
        self.qzeros = nn.Parameter(torch.empty(in_features // group_size, out_features // 8, dtype=torch.int32),
                                   requires_grad=False)
        self.scales = nn.Parameter(torch.empty(in_features // group_size, out_features, dtype=torch.float16),
                                   requires_grad=False)

    def forward(self, x):
        shape = x.shape
        x = x.reshape(-1, self.in_features).contiguous()
        # (after fuse_w4a16 the parameters are column views of the fused
        # tensors; a direct call then reads contiguous copies)
        out = dequant_matmul_w4a16(x, self.qweight.contiguous(), self.qzeros.contiguous(), self.scales.contiguous(),
                                   self.group_size)
        return out.reshape(*shape[:-1], self.out_features)


@torch.no_grad()
def fuse_w4a16(linears) -> W4A16Linear:
    """One GPTQ linear for several that read the same input (q/k/v, gate/up):
    qweight, qzeros and scales concatenated along N (dim 1), which keeps every
    column's packing (qzeros packs 8 output channels per int32, so each part's
    N must be a multiple of 8).  The parts' parameters become views into the
    fused tensors, so nothing is stored twice and their state-dict entries
    keep the reference names and values.  The fused forward equals the
    concatenation of the parts' forwards bit for bit (columns are computed
    independently)."""
    K = linears[0].in_features
    if any(l.in_features != K or l.group_size != 128 or l.out_features % 8 for l in linears):
        raise ValueError("Fused GPTQ linears need the same input width, group 128 and N % 8 == 0")
    fused = W4A16Linear.__new__(W4A16Linear)
    nn.Module.__init__(fused)
    fused.in_features, fused.group_size = K, 128
    fused.out_features = sum(l.out_features for l in linears)
    for name in ("qweight", "qzeros", "scales"):
        setattr(fused, name, nn.Parameter(torch.cat([getattr(l, name).data for l in linears], dim=1),
                                          requires_grad=False))
    off = 0
    for l in linears:
        n = l.out_features
        l.qweight = nn.Parameter(fused.qweight.data[:, off:off + n], requires_grad=False)
        l.qzeros = nn.Parameter(fused.qzeros.data[:, off // 8:(off + n) // 8], requires_grad=False)
        l.scales = nn.Parameter(fused.scales.data[:, off:off + n], requires_grad=False)
        off += n
    return fused
