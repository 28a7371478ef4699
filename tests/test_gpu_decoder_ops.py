"""GPU parity of the fused decoder elementwise kernels against fp32 PyTorch.

Each kernel is compared with the reference's PyTorch formulation of the
same op, written out below in fp32 with the reference's bf16 rounding
points (nanovllm/layers/layernorm.py:16-50, nanovllm/layers/rotary_embedding.py:
6-48, nanovllm/models/qwen3.py:78-94, nanovllm/layers/activation.py:8-11,
nanovllm/layers/attention.py:10-40):

* bit-exact where no reduction or transcendental is involved (the residual
  sum, the value copy into the cache, untouched cache slots);
* elsewhere within one bf16 ulp, with at most 1% of the elements off by that
  ulp: the kernels sum x^2 in another order than torch's reduction (so the
  reciprocal RMS can differ in its last fp32 bit) and exp may differ by an
  ulp between implementations, which moves a bf16 rounding now and then.
  A rotated output y1 = x1 cos - x2 sin inherits a one-ulp change of the
  normalised x1 or x2 without the cancellation shrinking it, so its bound
  adds 2^-7 (|x1| + |x2|).

The fused producer + K1 kernels (``rmsnorm_rht_quant_pack``,
``silu_mul_rht_quant_pack``) must give exactly the codes and scales of the
producer kernel followed by ``rht_quant_pack`` (whose parity with the
oracle is tested elsewhere), and the same residual.
"""
import pytest
import torch
import torch.nn.functional as F

from nv4 import rht_quant_pack
from nv4.kernels.decoder_ops import (qk_norm_rope_store, rmsnorm, rmsnorm_rht_quant_pack, silu_mul,
                                     silu_mul_rht_quant_pack)

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
EPS = 1e-6


def close_bf16(out, ref, what, frac=0.01, extra=None):
    """|out - ref| <= 1 bf16 ulp of ref (+ ``extra``) everywhere; mismatches <= frac."""
    o, r = out.float(), ref.float()
    ulp = torch.where(r == 0, torch.full_like(r, 2.0 ** -133), r.abs() * 2.0 ** -7)
    if extra is not None:
        ulp = ulp + extra
    bad = (o - r).abs() > ulp * 1.001
    assert not bad.any(), f"{what}: {int(bad.sum())} elements off by more than one ulp"
    mism = (o != r).float().mean().item()
    assert mism <= frac, f"{what}: {mism:.4f} of the elements differ by an ulp"


def ref_rms(x, w, residual=None):
    h = x.float()
    if residual is not None:
        h = h + residual.float()
    res = h.to(torch.bfloat16)
    r = torch.rsqrt(h.pow(2).mean(dim=-1, keepdim=True) + EPS)
    y = ((h * r).to(torch.bfloat16).float() * w.float()).to(torch.bfloat16)
    return y, res


@pytest.mark.parametrize("rows,H", [(1, 4096), (7, 4096), (64, 4096), (300, 1024), (3, 8192), (5, 144)])
@pytest.mark.parametrize("with_residual", [False, True])
def test_rmsnorm(rows, H, with_residual):
    g = torch.Generator(device=DEV).manual_seed(rows * 31 + H)
    x = (torch.randn(rows, H, generator=g, device=DEV) * 3).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(H, generator=g, device=DEV)).to(torch.bfloat16)
    res = torch.randn(rows, H, generator=g, device=DEV).to(torch.bfloat16) if with_residual else None
    ref_y, ref_res = ref_rms(x, w, res)
    if with_residual:
        y, new_res = rmsnorm(x, w, EPS, residual=res)
        assert new_res.data_ptr() == res.data_ptr()
        assert torch.equal(new_res, ref_res)
    else:
        y = rmsnorm(x, w, EPS)
    close_bf16(y, ref_y, f"rmsnorm rows={rows} H={H}")


def test_rmsnorm_in_place_output():
    g = torch.Generator(device=DEV).manual_seed(4)
    x = torch.randn(9, 4096, generator=g, device=DEV).to(torch.bfloat16)
    w = torch.ones(4096, dtype=torch.bfloat16, device=DEV)
    ref_y, _ = ref_rms(x, w)
    y = rmsnorm(x, w, EPS, out=x)
    assert y.data_ptr() == x.data_ptr()
    close_bf16(y, ref_y, "rmsnorm in place")


def ref_qk(qkv, Hq, Hkv, qw, kw, cos_sin, positions):
    D = 128
    T = qkv.shape[0]
    q = qkv[:, :Hq * D].reshape(T, Hq, D)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].reshape(T, Hkv, D)
    v = qkv[:, (Hq + Hkv) * D:(Hq + 2 * Hkv) * D].reshape(T, Hkv, D)
    q, _ = ref_rms(q, qw)
    k, _ = ref_rms(k, kw)
    cos, sin = cos_sin[positions].chunk(2, dim=-1)  # [T, 1, 64]

    def rot(x):
        x1, x2 = x.float().chunk(2, dim=-1)
        return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(torch.bfloat16)

    def slack(x):  # one-ulp change of either rotated input
        x1, x2 = x.float().abs().chunk(2, dim=-1)
        return (x1 + x2).repeat(1, 1, 2) * 2.0 ** -7

    return rot(q), rot(k), v.contiguous(), slack(q), slack(k)


def rope_table(max_pos, base=1_000_000.0):
    inv = 1.0 / (base ** (torch.arange(0, 128, 2, dtype=torch.float) / 128))
    f = torch.arange(max_pos, dtype=torch.float)[:, None] * inv[None, :]
    return torch.cat((f.cos(), f.sin()), dim=-1).unsqueeze_(1).to(DEV)


@pytest.mark.parametrize("T,Hq,Hkv", [(1, 32, 8), (3, 32, 8), (33, 32, 8), (260, 32, 8), (5, 8, 8), (4, 4, 1)])
def test_qk_norm_rope_store(T, Hq, Hkv):
    g = torch.Generator(device=DEV).manual_seed(T * 7 + Hq)
    width = (Hq + 2 * Hkv) * 128
    qkv_full = (torch.randn(T, width + 256, generator=g, device=DEV) * 2).to(torch.bfloat16)
    qkv = qkv_full[:, :width]  # strided rows, as a slice of a wider projection output
    qw = (1 + 0.2 * torch.randn(128, generator=g, device=DEV)).to(torch.bfloat16)
    kw = (1 + 0.2 * torch.randn(128, generator=g, device=DEV)).to(torch.bfloat16)
    table = rope_table(4096)
    positions = torch.randint(0, 4096, (T,), generator=g, device=DEV)
    nb, bs = 6, 64
    kc = torch.zeros(nb, bs, Hkv, 128, dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    slots = torch.randperm(nb * bs, generator=g, device=DEV)[:T].to(torch.int32)
    if T > 2:
        slots[1] = -1  # the reference's padding slot: not stored
    rq, rk, rv, sq, sk = ref_qk(qkv, Hq, Hkv, qw, kw, table, positions)
    q, k, v = qk_norm_rope_store(qkv, Hq, Hkv, qw, kw, table, positions, EPS, slot_mapping=slots, k_cache=kc,
                                 v_cache=vc, return_kv=True)
    close_bf16(q, rq, "q", extra=sq)
    close_bf16(k, rk, "k", extra=sk)
    assert torch.equal(v, rv)
    keep = slots >= 0
    idx = slots[keep].long()
    flat_k, flat_v = kc.view(-1, Hkv, 128), vc.view(-1, Hkv, 128)
    assert torch.equal(flat_k[idx], k[keep]) and torch.equal(flat_v[idx], v[keep])
    mask = torch.ones(nb * bs, dtype=torch.bool, device=DEV)
    mask[idx] = False
    assert not flat_k[mask].any() and not flat_v[mask].any()
    # decode form: no k/v outputs, same queries and cache contents
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    q2 = qk_norm_rope_store(qkv, Hq, Hkv, qw, kw, table, positions, EPS, slot_mapping=slots, k_cache=kc2,
                            v_cache=vc2)
    assert torch.equal(q2, q) and torch.equal(kc2, kc) and torch.equal(vc2, vc)


def test_qk_norm_rope_store_out_of_table_positions_read_row_zero():
    """Positions outside [0, max_position) are documented to rotate with row
    0 of the table (cos 1, sin 0: no rotation) instead of reading past it;
    callers keep positions inside the table."""
    g = torch.Generator(device=DEV).manual_seed(77)
    Hq, Hkv, T = 8, 2, 4
    qkv = (torch.randn(T, (Hq + 2 * Hkv) * 128, generator=g, device=DEV) * 2).to(torch.bfloat16)
    qw = (1 + 0.2 * torch.randn(128, generator=g, device=DEV)).to(torch.bfloat16)
    kw = (1 + 0.2 * torch.randn(128, generator=g, device=DEV)).to(torch.bfloat16)
    table = rope_table(64)
    bad = torch.tensor([64, 1000, -1, 2**40], dtype=torch.int64, device=DEV)
    zero = torch.zeros(T, dtype=torch.int64, device=DEV)
    q_bad, k_bad, v_bad = qk_norm_rope_store(qkv, Hq, Hkv, qw, kw, table, bad, EPS, return_kv=True)
    q_0, k_0, v_0 = qk_norm_rope_store(qkv, Hq, Hkv, qw, kw, table, zero, EPS, return_kv=True)
    assert torch.equal(q_bad, q_0) and torch.equal(k_bad, k_0) and torch.equal(v_bad, v_0)


def test_qk_norm_rope_store_rejects_bad_norm_weights():
    qkv = torch.zeros(2, (4 + 2) * 128, dtype=torch.bfloat16, device=DEV)
    table = rope_table(16)
    pos = torch.zeros(2, dtype=torch.int64, device=DEV)
    good = torch.ones(128, dtype=torch.bfloat16, device=DEV)
    for bad in (torch.ones(128, dtype=torch.float32, device=DEV), torch.ones(64, dtype=torch.bfloat16, device=DEV),
                torch.ones(256, dtype=torch.bfloat16, device=DEV)[::2]):
        with pytest.raises(TypeError):
            qk_norm_rope_store(qkv, 4, 1, bad, good, table, pos, EPS)
        with pytest.raises(TypeError):
            qk_norm_rope_store(qkv, 4, 1, good, bad, table, pos, EPS)


@pytest.mark.parametrize("rows,I", [(1, 12288), (32, 12288), (70, 12288), (3, 8)])
def test_silu_mul(rows, I):
    g = torch.Generator(device=DEV).manual_seed(rows + I)
    gu = (torch.randn(rows, 2 * I, generator=g, device=DEV) * 4).to(torch.bfloat16)
    gate, up = gu.float().chunk(2, -1)
    ref = (F.silu(gate).to(torch.bfloat16).float() * up).to(torch.bfloat16)
    close_bf16(silu_mul(gu), ref, f"silu_mul rows={rows}")


def test_silu_mul_extremes():
    vals = torch.tensor([0.0, -0.0, 1.0, -1.0, 20.0, -20.0, 88.0, -88.0, 100.0, -100.0, 3e38, -3e38, 1e-30, -1e-30,
                         float("inf"), float("-inf")], device=DEV)
    g = vals.repeat(8)[:128 // 2 * 2]
    gu = torch.cat([g, torch.full_like(g, 1.5)]).view(1, -1).to(torch.bfloat16)
    gate, up = gu.float().chunk(2, -1)
    ref = (F.silu(gate).to(torch.bfloat16).float() * up).to(torch.bfloat16)
    out = silu_mul(gu)
    fin = torch.isfinite(ref.float())
    close_bf16(out[fin], ref[fin], "silu extremes", frac=0.05)
    assert torch.equal(out[~fin].float().nan_to_num(0.0), ref[~fin].float().nan_to_num(0.0))


@pytest.mark.parametrize("rows", [1, 32, 300, 2500])
@pytest.mark.parametrize("with_residual", [False, True])
def test_rmsnorm_rht_quant_pack_equals_two_step(rows, with_residual):
    g = torch.Generator(device=DEV).manual_seed(rows + 77)
    x = (torch.randn(rows, 4096, generator=g, device=DEV) * 3).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(4096, generator=g, device=DEV)).to(torch.bfloat16)
    signs = (torch.randint(0, 2, (4096,), generator=g, device=DEV) * 2 - 1).to(torch.int8)
    res = torch.randn(rows, 4096, generator=g, device=DEV).to(torch.bfloat16) if with_residual else None
    if with_residual:
        res2 = res.clone()
        y, res2 = rmsnorm(x, w, EPS, residual=res2)
        packed, scale, res = rmsnorm_rht_quant_pack(x, w, EPS, signs, residual=res)
        assert torch.equal(res, res2)
    else:
        y = rmsnorm(x, w, EPS)
        packed, scale = rmsnorm_rht_quant_pack(x, w, EPS, signs)
    p2, s2 = k1(y, signs)
    torch.cuda.synchronize()
    assert torch.equal(packed, p2) and torch.equal(scale.view(torch.int16), s2.view(torch.int16))


def k1(x, signs):
    M, K = x.shape
    return rht_quant_pack(x, signs, out_packed=torch.empty((M, K // 2), dtype=torch.int8, device=DEV),
                          out_scale=torch.empty((M, K // 128), dtype=torch.bfloat16, device=DEV))


@pytest.mark.parametrize("K", [4096, 12288])
@pytest.mark.parametrize("rows", [1, 32, 65, 2500])
def test_silu_mul_rht_quant_pack_equals_two_step(K, rows):
    g = torch.Generator(device=DEV).manual_seed(rows + K)
    gu = (torch.randn(rows, 2 * K, generator=g, device=DEV) * 2).to(torch.bfloat16)
    signs = (torch.randint(0, 2, (K,), generator=g, device=DEV) * 2 - 1).to(torch.int8)
    packed, scale = silu_mul_rht_quant_pack(gu, signs)
    p2, s2 = k1(silu_mul(gu), signs)
    torch.cuda.synchronize()
    assert torch.equal(packed, p2) and torch.equal(scale.view(torch.int16), s2.view(torch.int16))


def silu_bf16_reference(g32):
    """round_bf16(g / (1 + e)) in fp32 arithmetic with e the correctly rounded
    fp32 exp(-g): exp in float64 rounded to fp32 (overflowing to inf past
    88.72), the fp32 sum, and the correctly rounded fp32 quotient."""
    import numpy as np
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        g = g32.astype(np.float64)  # signaling NaN patterns raise "invalid" here
        e = np.exp(-g).astype(np.float32)
        d = (np.float32(1.0) + e).astype(np.float32)
        s = (g / d.astype(np.float64)).astype(np.float32)
    return s


def test_silu_every_bf16_gate():
    """silu_mul with up = 1 over every bf16 gate value (all 65536 patterns):
    bf16(silu(g)) equals the fp32 formula with a correctly rounded exp, bit
    for bit (any NaN for NaN gates)."""
    import numpy as np
    bits = np.arange(65536, dtype=np.uint32)
    g32 = (bits << 16).view(np.float32)
    ref = silu_bf16_reference(g32)
    rb = ref.view(np.uint32)
    # bf16 round-to-nearest-even of the fp32 result
    rnd = ((rb + 0x7FFF + ((rb >> 16) & 1)) >> 16).astype(np.uint16)
    gate = torch.from_numpy(bits.astype(np.uint16).view(np.int16)).view(torch.bfloat16).to(DEV)
    gu = torch.cat([gate, torch.ones_like(gate)]).view(1, -1)
    out = silu_mul(gu).view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    nan_g = np.isnan(g32)
    out_f = (out.astype(np.uint32) << 16).view(np.float32)
    assert np.isnan(out_f[nan_g]).all()
    ok = nan_g | (out == rnd)
    bad = np.nonzero(~ok)[0]
    assert bad.size == 0, f"{bad.size} gates differ, e.g. g bits {[hex(b) for b in bad[:8]]}: " \
                          f"{[hex(out[b]) for b in bad[:8]]} vs {[hex(rnd[b]) for b in bad[:8]]}"
