"""GPU parity of the fused decode step attention (``nv4_paged_decode_attention_qkv``).

The decoder's decode step calls one launch for what the reference does in
q_norm/k_norm + rotary_emb (nanovllm/models/qwen3.py:78-94), store_kvcache
(nanovllm/layers/attention.py:10-40) and flash_attn_with_kvcache (:72-74).
Bar: bit-equal to the two launches it replaces, ``qk_norm_rope_store``
followed by ``paged_decode_attention`` on its q (each of those is checked
against fp32 references in test_gpu_decoder_ops.py and
test_gpu_attention.py): the attention output, and every byte of both caches
afterwards.  The step's cache slots start as NaN, so a lane of the fused
kernel that used the slot's old contents instead of the step's key or value
(the token itself, or the lanes clamped onto it past the context's end)
would make the outputs differ.  Cases: contexts at and around the 256-token
split and block boundaries, GQA groups 1/2/4, block sizes 256, 16 and 24,
the end-to-end decode shape with strided qkv rows, and the edge rows: slot
-1, an empty context with and without a slot, a context longer than
max_context, a slot other than the block table's, positions outside the
rotary table.
"""
import math

import pytest
import torch

from nv4.attention import paged_decode_attention, paged_decode_attention_qkv
from nv4.kernels.decoder_ops import qk_norm_rope_store

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
EPS = 1e-6
NAN16 = 0x7FC0  # a bf16 quiet NaN


def rope_table(max_pos, base=1_000_000.0):
    inv = 1.0 / (base ** (torch.arange(0, 128, 2, dtype=torch.float) / 128))
    f = torch.arange(max_pos, dtype=torch.float)[:, None] * inv[None, :]
    return torch.cat((f.cos(), f.sin()), dim=-1).contiguous().to(DEV)


def make_step(B, Hq, Hkv, bs, lens, seed, max_context, pad=64):
    """Caches, block tables and a step's qkv rows; slot_mapping[b] is the
    block-table slot of token lens[b] - 1 (the step's token), set to NaN."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    max_blocks = (max_context + bs - 1) // bs
    nblocks = B * max_blocks + 3
    kc = torch.randn(nblocks, bs, Hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn(nblocks, bs, Hkv, 128, generator=g, device=DEV).to(torch.bfloat16)
    perm = torch.randperm(nblocks, generator=g, device=DEV)[:B * max_blocks].to(torch.int32)
    bt = perm.view(B, max_blocks).contiguous()
    slots = []
    for b, n in enumerate(lens):
        t = max(n, 1) - 1
        slots.append(int(bt[b, t // bs]) * bs + t % bs if t < max_blocks * bs else -1)
    slot_mapping = torch.tensor(slots, dtype=torch.int32, device=DEV)
    cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    width = (Hq + 2 * Hkv) * 128
    qkv = (torch.randn(B, width + pad, generator=g, device=DEV) * 2).to(torch.bfloat16)[:, :width]
    qw = (1 + 0.2 * torch.randn(128, generator=g, device=DEV)).to(torch.bfloat16)
    kw = (1 + 0.2 * torch.randn(128, generator=g, device=DEV)).to(torch.bfloat16)
    positions = torch.tensor([max(n, 1) - 1 for n in lens], dtype=torch.int64, device=DEV)
    return kc, vc, bt, cl, slot_mapping, qkv, qw, kw, positions


def poison(kc, vc, slot_mapping):
    Hkv = kc.shape[2]
    for t in (kc, vc):
        flat = t.view(-1, Hkv, 128).view(torch.int16)
        for s in slot_mapping.tolist():
            if 0 <= s < flat.shape[0]:
                flat[s] = NAN16


def run_both(Hq, Hkv, kc, vc, bt, cl, slot_mapping, qkv, qw, kw, positions, table, max_context, scale):
    kc1, vc1 = kc.clone(), vc.clone()
    q = qk_norm_rope_store(qkv, Hq, Hkv, qw, kw, table, positions, EPS, slot_mapping=slot_mapping, k_cache=kc1,
                           v_cache=vc1)
    out1 = paged_decode_attention(q, kc1, vc1, bt, cl, scale, max_context=max_context)
    kc2, vc2 = kc.clone(), vc.clone()
    out2 = paged_decode_attention_qkv(qkv, Hq, Hkv, qw, kw, table, positions, slot_mapping, EPS, kc2, vc2, bt, cl,
                                      scale, max_context=max_context)
    torch.cuda.synchronize()
    return (out1, kc1, vc1), (out2, kc2, vc2)


def assert_same(a, b, what):
    for x, y, name in zip(a, b, ("out", "k_cache", "v_cache")):
        xi, yi = x.view(torch.int16), y.view(torch.int16)
        bad = (xi != yi).sum().item()
        assert bad == 0, f"{what}: {name} differs in {bad} of {xi.numel()} values"
    assert not torch.isnan(a[0].float()).any(), f"{what}: NaN in the output"


@pytest.mark.parametrize("G", [1, 2, 4])
@pytest.mark.parametrize("bs", [256, 16, 24])
def test_fused_step_equals_two_launches(G, bs):
    Hkv = 8 // G
    Hq = Hkv * G
    lens = [1, 7, 255, 256, 257, 600, 1000, 4352, 4351, 513]
    max_context = 4352
    print(f"[attn-qkv] G={G} bs={bs}", flush=True)
    kc, vc, bt, cl, sm, qkv, qw, kw, pos = make_step(len(lens), Hq, Hkv, bs, lens, G * 31 + bs, max_context)
    poison(kc, vc, sm)
    a, b = run_both(Hq, Hkv, kc, vc, bt, cl, sm, qkv, qw, kw, pos, rope_table(8192), max_context,
                    1 / math.sqrt(128))
    assert_same(a, b, f"G={G} bs={bs}")


def test_fused_step_qwen3_decode_shape():
    """32 sequences, 32 query / 8 KV heads, contexts near 4096, bs 256, qkv
    rows as the fused projection's output (strided)."""
    lens = [4096 + (7 * i) % 257 for i in range(32)]
    kc, vc, bt, cl, sm, qkv, qw, kw, pos = make_step(32, 32, 8, 256, lens, 5, 4352, pad=0)
    poison(kc, vc, sm)
    a, b = run_both(32, 8, kc, vc, bt, cl, sm, qkv, qw, kw, pos, rope_table(40960), 4352, 1 / math.sqrt(128))
    assert_same(a, b, "qwen3 decode")


@pytest.mark.parametrize("max_context", [256, 4352])
def test_fused_step_edge_rows(max_context):
    """Row 1: slot -1 (nothing stored; the old slot is read, as in the two
    launches).  Row 2: empty context with a slot (stored, output zeros).
    Row 3: empty context, slot -1.  Row 4: context longer than max_context
    (stored at its slot, not attended).  Row 5: a slot other than the block
    table's (stored there; the table's slot is read).  Row 6: a position
    outside the rotary table (row 0 of the table)."""
    lens = [200, 150, 0, 0, max_context + 40, 230, 100]
    kc, vc, bt, cl, sm, qkv, qw, kw, pos = make_step(len(lens), 32, 8, 256, lens, max_context, max_context)
    nslots = kc.shape[0] * kc.shape[1]
    used = set(int(x) for x in bt.flatten().tolist())
    free = [blk for blk in range(kc.shape[0]) if blk not in used]
    sm[1] = -1
    sm[2] = free[0] * 256 + 3
    sm[3] = -1
    sm[4] = free[1] * 256 + 17
    sm[5] = free[2] * 256 + 9
    pos[6] = 10 ** 9
    poison(kc, vc, sm[[0, 2, 4, 5, 6]])
    assert int(sm.max()) < nslots
    a, b = run_both(32, 8, kc, vc, bt, cl, sm, qkv, qw, kw, pos, rope_table(4096), max_context, 0.1)
    assert_same(a, b, f"edge rows max_context={max_context}")
    assert torch.equal(a[0][2], torch.zeros_like(a[0][2])) and torch.equal(a[0][3], torch.zeros_like(a[0][3]))


def test_fused_step_repeated_steps():
    """Three decode steps in a row (each appends one token per sequence),
    fused against two launches, from the same starting caches."""
    Hq, Hkv, bs, max_context = 32, 8, 16, 1024
    lens0 = [1, 15, 16, 255, 256, 700]
    kc, vc, bt, cl, sm, qkv, qw, kw, pos = make_step(len(lens0), Hq, Hkv, bs, lens0, 77, max_context)
    table = rope_table(2048)
    kc1, vc1, kc2, vc2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    g = torch.Generator(device=DEV).manual_seed(78)
    for step in range(3):
        lens = [n + step for n in lens0]
        cl = torch.tensor(lens, dtype=torch.int32, device=DEV)
        pos = torch.tensor([n - 1 for n in lens], dtype=torch.int64, device=DEV)
        sm = torch.tensor([int(bt[b, (n - 1) // bs]) * bs + (n - 1) % bs for b, n in enumerate(lens)],
                          dtype=torch.int32, device=DEV)
        qkv = (torch.randn(len(lens), (Hq + 2 * Hkv) * 128, generator=g, device=DEV) * 2).to(torch.bfloat16)
        q = qk_norm_rope_store(qkv, Hq, Hkv, qw, kw, table, pos, EPS, slot_mapping=sm, k_cache=kc1, v_cache=vc1)
        out1 = paged_decode_attention(q, kc1, vc1, bt, cl, 0.1, max_context=max_context)
        out2 = paged_decode_attention_qkv(qkv, Hq, Hkv, qw, kw, table, pos, sm, EPS, kc2, vc2, bt, cl, 0.1,
                                          max_context=max_context)
        torch.cuda.synchronize()
        assert_same((out1, kc1, vc1), (out2, kc2, vc2), f"step {step}")
