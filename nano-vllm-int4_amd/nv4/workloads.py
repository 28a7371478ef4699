"""Seeded synthetic inputs of the Qwen3-8B quantized-linear workloads.

All tensors come from ``torch.Generator("cpu")`` seeded from the reference's
standard base seed (benchmarks/rht_a4_bench_common.py:104), so the same
values are produced on any host and can feed both the GPU kernels and the
CPU oracle.  Shapes follow the reference's fused projections
(benchmarks/rht_a4_bench_common.py:13-18): qkv (6144, 4096), o (4096, 4096),
gate_up (24576, 4096), down (4096, 12288), written (N, K).

Recipes:
* W4A4 activations: randn fp32, 1 % of channels (a seeded permutation) x20 as
  outliers, rounded to bf16.  down_proj inputs are bf16(silu(g) * u) of two
  randn bf16 tensors instead (a heavy-tailed distribution).
* RHT signs: randint(0, 2) * 2 - 1, int8.
* W4A4 weights: codes randint(-8, 8) packed two per byte (even k in the low
  nibble), group-128 bf16 scales uniform in [0.005, 0.02].
* W4A16 weights: codes randint(0, 16) packed 8 per int32 along K, zero points
  randint(0, 16) packed 8 per int32 along N, fp16 scales uniform in
  [0.005, 0.02]; fp16 activations randn.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

BASE_SEED = 20261108
PROJECTIONS = {  # name -> (N, K)
    "qkv": (6144, 4096),
    "o": (4096, 4096),
    "gate_up": (24576, 4096),
    "down": (4096, 12288),
}


def _gen(seed: int) -> torch.Generator:
    return torch.Generator("cpu").manual_seed(int(seed))


def pack_int4(codes: torch.Tensor) -> torch.Tensor:
    """int8 codes [..., K] in [-8, 7] -> int8 [..., K/2], even k in the low nibble."""
    c = codes.to(torch.int16)
    return ((c[..., ::2] & 15) | ((c[..., 1::2] & 15) << 4)).to(torch.uint8).view(torch.int8).contiguous()


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    p = packed.view(torch.uint8).to(torch.int16)
    lo, hi = p & 15, (p >> 4) & 15
    lo = torch.where(lo >= 8, lo - 16, lo)
    hi = torch.where(hi >= 8, hi - 16, hi)
    return torch.stack((lo, hi), dim=-1).flatten(-2).to(torch.int8)


def activations(M: int, K: int, seed: int, outlier_fraction: float = 0.01) -> torch.Tensor:
    x = torch.randn(M, K, generator=_gen(seed), dtype=torch.float32)
    count = int(round(K * outlier_fraction))
    if count:
        idx = torch.randperm(K, generator=_gen(seed + 1))[:count]
        x[:, idx] *= 20.0
    return x.to(torch.bfloat16).contiguous()


def silu_mul_activations(M: int, K: int, seed_g: int, seed_u: int) -> torch.Tensor:
    g = torch.randn(M, K, generator=_gen(seed_g), dtype=torch.float32).to(torch.bfloat16)
    u = torch.randn(M, K, generator=_gen(seed_u), dtype=torch.float32).to(torch.bfloat16)
    gf = g.float()
    return (gf * torch.sigmoid(gf) * u.float()).to(torch.bfloat16).contiguous()


def special_rows(m: int, k: int, seed: int = BASE_SEED) -> torch.Tensor:
    """Seeded randn bf16 rows carrying the reference's special rows
    (benchmarks/rht_a4_bench_common.py:104-120: a zero row, an impulse of
    1000 at k/12 or 5, a row of ones, alternating +-1, x1e-9 and x1e4), drawn
    from a CPU generator with the reference's seed formula."""
    x = torch.randn(m, k, generator=_gen(seed + m * 17 + k), dtype=torch.float32).to(torch.bfloat16)
    x[0].zero_()
    if m > 1:
        x[1].zero_()
        x[1, k // 12 if k == 12288 else 5] = 1000
    if m > 2:
        x[2].fill_(1)
    if m > 3:
        x[3, ::2] = 1
        x[3, 1::2] = -1
    if m > 4:
        x[4].mul_(1e-9)
    if m > 5:
        x[5].mul_(1e4)
    return x.contiguous()


def signs(K: int, seed: int) -> torch.Tensor:
    return (torch.randint(0, 2, (K,), generator=_gen(seed), dtype=torch.int8) * 2 - 1).contiguous()


def w4a4_weights(N: int, K: int, seed_q: int, seed_s: int):
    """(packed int8 [N, K/2], scale bf16 [N, K/128])."""
    q = torch.randint(-8, 8, (N, K), generator=_gen(seed_q), dtype=torch.int8)
    sw = (0.005 + 0.015 * torch.rand(N, K // 128, generator=_gen(seed_s))).to(torch.bfloat16)
    return pack_int4(q), sw.contiguous()


def pack_qweight(q: torch.Tensor) -> torch.Tensor:
    """codes [K, N] in [0, 16) -> int32 [K/8, N] with code k%8 at bits 4*(k%8)."""
    K, N = q.shape
    q = q.to(torch.int64).reshape(K // 8, 8, N)
    shifts = (4 * torch.arange(8, dtype=torch.int64)).view(1, 8, 1)
    word = (q << shifts).sum(dim=1)
    return ((word + 2**31) % 2**32 - 2**31).to(torch.int32).contiguous()


def pack_qzeros(z: torch.Tensor) -> torch.Tensor:
    """zero points [G, N] in [0, 16) -> int32 [G, N/8] with z[g, n] at bits 4*(n%8)."""
    G, N = z.shape
    z = z.to(torch.int64).reshape(G, N // 8, 8)
    shifts = (4 * torch.arange(8, dtype=torch.int64)).view(1, 1, 8)
    word = (z << shifts).sum(dim=2)
    return ((word + 2**31) % 2**32 - 2**31).to(torch.int32).contiguous()


def w4a16_weights(K: int, N: int, seed_q: int, seed_z: int, seed_s: int, group: int = 128):
    """(qweight int32 [K/8, N], qzeros int32 [K/group, N/8], scales fp16 [K/group, N])."""
    q = torch.randint(0, 16, (K, N), generator=_gen(seed_q), dtype=torch.int64)
    z = torch.randint(0, 16, (K // group, N), generator=_gen(seed_z), dtype=torch.int64)
    s = (0.005 + 0.015 * torch.rand(K // group, N, generator=_gen(seed_s))).to(torch.float16)
    return pack_qweight(q), pack_qzeros(z), s.contiguous()


@dataclass
class W4A4Case:
    name: str
    x: torch.Tensor        # bf16 [M, K]
    signs: torch.Tensor    # int8 [K]
    w_packed: torch.Tensor  # int8 [N, K/2]
    w_scale: torch.Tensor  # bf16 [N, K/128]

    @property
    def shape(self):
        return self.x.shape[0], self.w_packed.shape[0], self.x.shape[1]


def w4a4_case(projection: str, M: int, seed: int = BASE_SEED) -> W4A4Case:
    """The W4A4 workload of one fused projection at M rows.

    o (config 0, seeds S..S+4), gate_up (config 2, S+20..S+24), down (config 3,
    S+30..S+34, silu(g)*u activations), qkv (S+40..S+44)."""
    N, K = PROJECTIONS[projection]
    off = {"o": 0, "gate_up": 20, "down": 30, "qkv": 40}[projection]
    s = seed + off
    if projection == "down":
        x = silu_mul_activations(M, K, s, s + 1)
    else:
        x = activations(M, K, s)
    wp, sw = w4a4_weights(N, K, s + 3, s + 4)
    return W4A4Case(projection, x, signs(K, s + 2), wp, sw)


@dataclass
class W4A16Case:
    x: torch.Tensor        # fp16 [M, K]
    qweight: torch.Tensor
    qzeros: torch.Tensor
    scales: torch.Tensor


def w4a16_case(M: int, N: int = 6144, K: int = 4096, seed: int = BASE_SEED,
               dtype: torch.dtype = torch.float16) -> W4A16Case:
    """Config 1: W4A16 fused QKV (N = 4096 q + 2 x 1024 kv), seeds S+10..S+13."""
    x = torch.randn(M, K, generator=_gen(seed + 10), dtype=torch.float32).to(dtype).contiguous()
    qw, qz, sc = w4a16_weights(K, N, seed + 11, seed + 12, seed + 13)
    return W4A16Case(x, qw, qz, sc)
