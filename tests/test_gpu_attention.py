"""GPU parity of the decoder's attention against an fp32 reference.

Paged decode attention (``nv4_paged_decode_attention``, the replacement of
flash_attn_with_kvcache in nanovllm/layers/attention.py:72-74): random bf16
caches behind shuffled block tables, context lengths at and around the
256-token split and block boundaries (1, 255, 256, 257, ..., 4352), GQA
groups 1/2/4, block sizes 256, 16 (one block-table read per 16 tokens) and
24 (one read per token), contexts of more than 64 splits (the merge's
chunked loop), every compile-time split count of the merge (bit-equal to the
chunked form), and queries read as a strided view of a fused qkv tensor;
against softmax(scale q.K^T) V computed in fp32.  Bar:
|out - ref| <= 1e-2 + 1e-2 |ref| (bf16 output).  Rows with an empty context
give zeros.  Prefill attention (``nv4_prefill_attention``, the replacement of
flash_attn_varlen_func in nanovllm/layers/attention.py:64-70: causal GQA over
packed sequences in one launch) against the same fp32 reference and bar:
lengths around its 32-row query tiles, 64-row workgroups and 64-key blocks
up to the 4096-token prompt of the end-to-end workload, query-to-KV head
ratios 1/2/4/8, q/k/v as strided slices of a fused tensor, and large score
peaks that move the running max.
"""
import math

import pytest
import torch

from nv4.attention import paged_decode_attention, prefill_attention

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def reference(q, kc, vc, bt, cl, scale):
    """fp32 attention of each sequence over its first cl[b] slots."""
    B, Hq, D = q.shape
    bs, Hkv = kc.shape[1], kc.shape[2]
    G = Hq // Hkv
    outs = []
    for b in range(B):
        n = int(cl[b])
        slots = torch.tensor([int(bt[b, t // bs]) * bs + t % bs for t in range(n)], device=q.device)
        k = kc.reshape(-1, Hkv, D)[slots].float().repeat_interleave(G, dim=1).contiguous()  # [n, Hq, D]
        v = vc.reshape(-1, Hkv, D)[slots].float().repeat_interleave(G, dim=1).contiguous()
        s = torch.einsum("hd,nhd->hn", q[b].float(), k) * scale
        p = torch.softmax(s, dim=-1)
        outs.append(torch.einsum("hn,nhd->hd", p, v))
    return torch.stack(outs)


def make_case(B, Hq, Hkv, bs, lens, seed, strided=False):
    g = torch.Generator(device=DEV).manual_seed(seed)
    max_blocks = max((n + bs - 1) // bs for n in lens)
    nblocks = B * max_blocks + 3
    kc = torch.randn(nblocks, bs, Hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn(nblocks, bs, Hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    perm = torch.randperm(nblocks, generator=g, device=DEV)[:B * max_blocks].to(torch.int32)
    bt = perm.view(B, max_blocks).contiguous()
    cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    if strided:  # q as the leading slice of a fused [B, (Hq + 2 Hkv) * 128] row
        qkv = torch.randn(B, (Hq + 2 * Hkv) * 128, generator=g, device=DEV).to(torch.bfloat16)
        q = qkv[:, :Hq * 128].view(B, Hq, 128)
    else:
        q = torch.randn(B, Hq, 128, generator=g, device=DEV).to(torch.bfloat16)
    return q, kc, vc, bt, cl


def check(out, ref, what):
    err = (out.float() - ref).abs()
    bound = 1e-2 + 1e-2 * ref.abs()
    bad = (err > bound).sum().item()
    assert bad == 0, f"{what}: {bad} of {err.numel()} outside the bound, max err {err.max().item():.3e}"


@pytest.mark.parametrize("G", [1, 2, 4])
@pytest.mark.parametrize("bs", [256, 16, 24])
def test_paged_decode_attention(G, bs):
    Hkv = 8 // G if G < 8 else 1
    Hq = Hkv * G
    lens = [1, 7, 255, 256, 257, 600, 1000, 4352]
    print(f"[attn] G={G} Hq={Hq} Hkv={Hkv} bs={bs}", flush=True)
    q, kc, vc, bt, cl = make_case(len(lens), Hq, Hkv, bs, lens, seed=G * 100 + bs)
    scale = 1 / math.sqrt(128)
    out = paged_decode_attention(q, kc, vc, bt, cl, scale, max_context=4352)
    torch.cuda.synchronize()
    check(out, reference(q, kc, vc, bt, cl, scale), f"G={G} bs={bs}")


def test_paged_decode_attention_qwen3_batch_strided():
    """The decode shape of the end-to-end workload: 32 sequences, 32 query /
    8 KV heads, contexts near 4096, q read from a fused qkv row."""
    lens = [4096 + (7 * i) % 257 for i in range(32)]
    q, kc, vc, bt, cl = make_case(32, 32, 8, 256, lens, seed=7, strided=True)
    assert q.stride(0) == (32 + 16) * 128
    scale = 1 / math.sqrt(128)
    ws = torch.empty(32 * 32 * 18 * 130, dtype=torch.float32, device=DEV)
    out = paged_decode_attention(q, kc, vc, bt, cl, scale, workspace=ws, max_context=4352)
    torch.cuda.synchronize()
    check(out, reference(q, kc, vc, bt, cl, scale), "qwen3 batch")


def test_paged_decode_attention_many_splits():
    """More than 64 splits of 256 tokens: the merge takes them in chunks of 64."""
    lens = [64 * 256 + 300, 300, 64 * 256 + 1]
    q, kc, vc, bt, cl = make_case(3, 32, 8, 256, lens, seed=13)
    scale = 1 / math.sqrt(128)
    out = paged_decode_attention(q, kc, vc, bt, cl, scale, max_context=max(lens))
    torch.cuda.synchronize()
    check(out, reference(q, kc, vc, bt, cl, scale), "many splits")


@pytest.mark.parametrize("max_ctx", [512, 2304, 4352, 8000, 12000])
def test_merge_split_counts_equal_chunked_form(max_ctx):
    """Each compile-time split count of the merge (S up to 8, 16, 24, 32, 64:
    every load in one round trip) gives the bits of the chunked general form,
    which a block table widened to 65 splits selects for the same contexts."""
    lens = [max_ctx, 1, 257, max_ctx - 255, (2 * max_ctx) // 3]
    q, kc, vc, bt, cl = make_case(len(lens), 32, 8, 256, lens, seed=max_ctx)
    scale = 1 / math.sqrt(128)
    wide = 65 * 256
    pad = torch.zeros(bt.shape[0], wide // 256 - bt.shape[1], dtype=torch.int32, device=DEV)  # never read
    bt_wide = torch.cat([bt, pad], 1).contiguous()
    print(f"[attn] merge max_ctx={max_ctx} splits={(max_ctx + 255) // 256}", flush=True)
    out = paged_decode_attention(q, kc, vc, bt, cl, scale, max_context=max_ctx)
    out_chunked = paged_decode_attention(q, kc, vc, bt_wide, cl, scale, max_context=wide)
    torch.cuda.synchronize()
    check(out, reference(q, kc, vc, bt, cl, scale), f"max_ctx={max_ctx}")
    assert torch.equal(out, out_chunked)


def test_single_split_writes_output_directly():
    lens = [1, 100, 256]
    q, kc, vc, bt, cl = make_case(3, 32, 8, 256, lens, seed=11)
    out = paged_decode_attention(q, kc, vc, bt, cl, 0.1, max_context=256)
    torch.cuda.synchronize()
    check(out, reference(q, kc, vc, bt, cl, 0.1), "one split")


@pytest.mark.parametrize("max_ctx", [256, 4352])
def test_empty_context_rows_are_zero(max_ctx):
    """A row whose context length is 0 (or negative) has nothing to attend
    to: its output is defined as zeros, with one split (no merge pass) and
    with several; the other rows are unaffected."""
    lens = [100, 0, 257, 1]
    q, kc, vc, bt, cl = make_case(4, 32, 8, 256, lens, seed=max_ctx + 1)
    if max_ctx == 256:
        lens[2], cl[2] = 256, 256
    cl[3] = -5
    out = torch.full((4, 32, 128), float("nan"), dtype=torch.bfloat16, device=DEV)
    bt = torch.cat([bt, torch.zeros(4, max(0, max_ctx // 256 - bt.shape[1]), dtype=torch.int32, device=DEV)], 1)
    paged_decode_attention(q, kc, vc, bt.contiguous(), cl, 0.1, out=out, max_context=max_ctx)
    torch.cuda.synchronize()
    assert torch.equal(out[1], torch.zeros_like(out[1])) and torch.equal(out[3], torch.zeros_like(out[3]))
    live = [0, 2]
    check(out[live], reference(q[live], kc, vc, bt[live], cl[live], 0.1), f"live rows max_ctx={max_ctx}")


def prefill_reference(q, k, v, lens, scale):
    """fp32 causal GQA attention of each packed sequence."""
    G = q.shape[1] // k.shape[1]
    outs, start = [], 0
    for n in lens:
        qf = q[start:start + n].float().transpose(0, 1).contiguous()
        kf = k[start:start + n].float().repeat_interleave(G, dim=1).transpose(0, 1).contiguous()
        vf = v[start:start + n].float().repeat_interleave(G, dim=1).transpose(0, 1).contiguous()
        s = torch.matmul(qf, kf.transpose(1, 2).contiguous()) * scale
        s = s + torch.triu(torch.full((n, n), float("-inf"), device=DEV), 1)
        outs.append(torch.matmul(torch.softmax(s, dim=-1), vf).transpose(0, 1))
        start += n
    return torch.cat(outs, 0)


@pytest.mark.parametrize("lens", [[1, 17, 300], [4096, 33], [64, 65, 127, 128, 129], [31, 32, 33, 63, 257, 1000],
                                  [1900], [2000], [8192, 129]])
def test_prefill_attention(lens):
    """nv4_prefill_attention (one launch for all packed sequences) against fp32;
    lengths around the 32-row query tiles, 64-row workgroups and 64-key blocks;
    both workgroup forms (4 waves while 8-wave workgroups would number fewer
    than the CUs, as for 1900 tokens; 8 waves from 2000 tokens on); a prompt
    twice the end-to-end one."""
    print(f"[prefill-attn] lens={lens}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(3 + len(lens))
    T = sum(lens)
    q = torch.randn(T, 32, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(T, 8, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(T, 8, 128, generator=g, device=DEV).to(torch.bfloat16)
    scale = 1 / math.sqrt(128)
    out = torch.full_like(q, float("nan"))
    out.copy_(prefill_attention(q, k, v, lens, scale))
    torch.cuda.synchronize()
    ref = prefill_reference(q, k, v, lens, scale)
    start = 0
    for n in lens:
        check(out[start:start + n], ref[start:start + n], f"prefill n={n}")
        start += n


@pytest.mark.parametrize("G,Hkv,lens", [(1, 8, [5, 300, 129]), (2, 4, [5, 300, 129]), (8, 2, [5, 300, 129]),
                                        (1, 8, [4096, 40]), (2, 4, [4096, 100])])
def test_prefill_attention_gqa_groups(G, Hkv, lens):
    """Other query-to-KV head ratios (the workgroup then covers 256/G rows).
    The short prompts run the 4-wave form; a 4096-token prompt beside a short
    one at G = 1 / Hkv = 8 and G = 2 / Hkv = 4 gives 256 8-wave workgroups, as
    many as the CUs, so those run the 8-wave form with 128-key blocks (256 and
    128 query rows per workgroup)."""
    print(f"[prefill-attn-gqa] G={G} Hkv={Hkv} lens={lens}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(11 * G)
    T = sum(lens)
    q = torch.randn(T, G * Hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(T, Hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(T, Hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    out = prefill_attention(q, k, v, lens, 0.125)
    torch.cuda.synchronize()
    check(out, prefill_reference(q, k, v, lens, 0.125), f"G={G}")


def test_prefill_attention_strided_and_peaked():
    """q, k, v as column slices of one fused [T, (32+8+8)*128] tensor (row
    strides larger than the head block), and scores with large peaks (a
    scale of 0.5: the running max moves often, the rescale runs)."""
    lens = [700, 64]
    print(f"[prefill-attn-strided] lens={lens}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(5)
    T = sum(lens)
    qkv = torch.randn(T, 48 * 128, generator=g, device=DEV).to(torch.bfloat16)
    q = qkv[:, :4096].view(T, 32, 128)
    k = qkv[:, 4096:5120].view(T, 8, 128)
    v = qkv[:, 5120:].view(T, 8, 128)
    out = prefill_attention(q, k, v, lens, 0.5)
    torch.cuda.synchronize()
    check(out, prefill_reference(q, k, v, lens, 0.5), "strided")
