"""The allocation-free paged decode attention entry point
(``nv4_paged_decode_attention_noalloc``), called through the C ABI.

Its split partials live in the library's per-GPU device scratch
(``NV4_PA_SCRATCH_BYTES``) instead of a caller's workspace; it runs the same
kernels, so its outputs equal those of ``nv4_paged_decode_attention`` bit
for bit.  Checked on two calls in a row on one GPU (the scratch keeps the
first call's partials), the second with a smaller batch and context, and
on a single-split call; sizes beyond the scratch are rejected with
NV4_E_SCRATCH before anything is launched (no GPU needed for that).
"""
import ctypes
import math

import pytest
import torch

from nv4 import _lib

DEV = "cuda:0"
P = ctypes.c_void_p


def call_noalloc(q, kc, vc, bt, cl, out, max_ctx, scale):
    B, Hq, D = q.shape
    nb, bs, Hkv, _ = kc.shape
    lib = _lib.load()
    with torch.cuda.device(q.device):
        return lib.nv4_paged_decode_attention_noalloc(
            P(q.data_ptr()), q.stride(0), P(kc.data_ptr()), P(vc.data_ptr()), P(bt.data_ptr()), bt.shape[1],
            P(cl.data_ptr()), P(out.data_ptr()), B, Hq, Hkv, D, bs, max_ctx, ctypes.c_float(scale),
            P(torch.cuda.current_stream(q.device).cuda_stream))


def call_ws(q, kc, vc, bt, cl, out, max_ctx, scale):
    B, Hq, D = q.shape
    nb, bs, Hkv, _ = kc.shape
    S = (max_ctx + 255) // 256
    ws = torch.empty(B * Hq * S * (D + 2), dtype=torch.float32, device=q.device)
    lib = _lib.load()
    with torch.cuda.device(q.device):
        return lib.nv4_paged_decode_attention(
            P(q.data_ptr()), q.stride(0), P(kc.data_ptr()), P(vc.data_ptr()), P(bt.data_ptr()), bt.shape[1],
            P(cl.data_ptr()), P(out.data_ptr()), P(ws.data_ptr()), ws.numel() * 4, B, Hq, Hkv, D, bs, max_ctx,
            ctypes.c_float(scale), P(torch.cuda.current_stream(q.device).cuda_stream))


def case(B, lens, seed, Hq=32, Hkv=8, bs=256):
    g = torch.Generator(device=DEV).manual_seed(seed)
    max_blocks = max((n + bs - 1) // bs for n in lens)
    nblocks = B * max_blocks + 2
    kc = torch.randn(nblocks, bs, Hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn(nblocks, bs, Hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    bt = torch.randperm(nblocks, generator=g, device=DEV)[:B * max_blocks].to(torch.int32).view(B, max_blocks)
    cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    q = torch.randn(B, Hq, 128, generator=g, device=DEV).to(torch.bfloat16)
    return q, kc, vc, bt.contiguous(), cl


def test_scratch_limit_rejected_before_launch():
    """B * Hq * S * 130 * 4 bytes above the 16 MiB scratch: NV4_E_SCRATCH
    (argument checks only; fake device addresses are never dereferenced)."""
    f = _lib.load().nv4_paged_decode_attention_noalloc
    A = 0x10000
    # 32 x 32 x 32 splits x 520 B = 17 MB > 16 MiB
    assert f(P(A), 4096, P(A), P(A), P(A), 32, P(A), P(A), 32, 32, 8, 128, 256, 8192, 0.1, None) \
        == _lib.NV4_E_SCRATCH
    assert f(None, 4096, P(A), P(A), P(A), 32, P(A), P(A), 32, 32, 8, 128, 256, 8192, 0.1, None) == _lib.NV4_E_NULL
    assert f(P(A), 4096, P(A), P(A), P(A), 32, P(A), P(A), 32, 32, 8, 64, 256, 8192, 0.1, None) == _lib.NV4_E_SHAPE
    assert _lib.strerror(_lib.NV4_E_SCRATCH) not in ("ok", "unknown error")


@pytest.mark.gpu
def test_noalloc_equals_workspace_entry_two_calls():
    scale = 1 / math.sqrt(128)
    # call 1: the end-to-end decode shape (32 sequences, ~4.1k context, 17 splits)
    lens1 = [4096 + (13 * i) % 257 for i in range(32)]
    # call 2: smaller batch and context (3 splits), after call 1 left its partials in the scratch
    lens2 = [1, 300, 700, 513, 256]
    for step, (lens, max_ctx, seed) in enumerate(((lens1, 4352, 1), (lens2, 768, 2))):
        q, kc, vc, bt, cl = case(len(lens), lens, seed)
        out_a = torch.full_like(q, float("nan"))
        out_b = torch.full_like(q, float("nan"))
        print(f"[noalloc] call {step + 1}: B={len(lens)} max_ctx={max_ctx}", flush=True)
        assert call_noalloc(q, kc, vc, bt, cl, out_a, max_ctx, scale) == _lib.NV4_OK
        assert call_ws(q, kc, vc, bt, cl, out_b, max_ctx, scale) == _lib.NV4_OK
        torch.cuda.synchronize()
        assert torch.isfinite(out_a.float()).all()
        assert torch.equal(out_a, out_b), f"call {step + 1}: allocation-free output differs"


@pytest.mark.gpu
def test_noalloc_single_split():
    q, kc, vc, bt, cl = case(3, [1, 100, 256], 5)
    out_a, out_b = torch.empty_like(q), torch.empty_like(q)
    assert call_noalloc(q, kc, vc, bt, cl, out_a, 256, 0.1) == _lib.NV4_OK
    assert call_ws(q, kc, vc, bt, cl, out_b, 256, 0.1) == _lib.NV4_OK
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)
