// Paged decode attention for the Qwen3 decoder (GQA, head_dim 128, bf16 KV
// cache), gfx950.  Replaces flash_attn_with_kvcache in the reference's
// decode branch (nanovllm/layers/attention.py:72-74): for every sequence b
// and query head h, o = softmax(scale * q . K^T) V over the first
// context_lens[b] cache slots of the sequence, found through its block table.
//
// Decode attention reads the whole KV context of every sequence once per
// step, so it is bound by HBM bandwidth.  Layout:
//  * pass 1: one workgroup (4 waves) per (sequence, KV head, split of
//    PA_SPLIT = 256 context tokens); wave w takes tokens 64w..64w+63 of the
//    split as two 32-token halves, and issues every K and V load of both
//    halves (q first) before any arithmetic.  The products run on the matrix
//    cores (v_mfma_f32_16x16x32_bf16; lane = (k-octet kq, row/column rc)):
//      - scores S^T[token][head] = K . q^T: A = K rows (lane: token
//        h0 + 16c + rc, 16-byte chunks kq, kq+4, kq+8, kq+12 -- a 64-byte
//        piece of the 256-byte row per load), B = q of head rc (zero past the
//        group's G heads), four 32-dim steps per 16-token tile;
//      - online softmax in the score layout: lane (kq, rc) holds head rc's
//        scores for tokens h0 + 16c + 4kq + r, so every exponential is taken
//        once; the max over the half is shared by the four k-octet rows
//        (scores in raw units, exponentials in base 2 with scale*log2(e));
//      - O[head][dim] += P . V: A = P (bf16, as flash attention rounds P for
//        P.V), B = V: each lane loads 256-byte V rows (chunk rc of its own
//        score tokens) and an 8x8 transpose of bf16 pairs (v_perm) turns
//        them into the operand of tile t = dims 8rc + t.
//    The four wave states (m, l, o per head) are merged through LDS and
//    written to the split workspace (or, for a single split, normalised
//    into out).
//  * pass 2: one wave per (sequence, query head) merges the splits: lane s
//    reads split s's (m, l), M = max m_s, w_s = 2^(m_s - M) (broadcast with
//    lane reads), o = sum w_s o_s / sum w_s l_s with lane i owning dims 2i,
//    2i+1 and every split's loads issued before the sums.
#include "norm_ops.h"
#include "qk_ops.h"

#include <mutex>

namespace nv4 {
namespace {

constexpr int PA_D = 128;        // head dim
constexpr int PA_SPLIT = 256;    // context tokens per pass-1 workgroup
constexpr int PA_THREADS = 256;  // 4 waves x 64 tokens
constexpr int PA_KT_ROW = 272;   // bytes per K row in the transposing LDS buffer

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

// The step's q/k RMSNorm, rotary embedding and KV store, fused into the
// decode attention (FUSED): q is then the raw fused qkv row of the step's
// token, [Hq q heads | Hkv k heads | Hkv v heads] x 128.
struct QkvStep {
    const uint16_t* qw;        // q_norm weight [128]
    const uint16_t* kw;        // k_norm weight [128]
    const float* cos_sin;      // [max_position, 128]: cos of dims 0..63, then sin
    const int64_t* positions;  // [B]
    const int32_t* slots;      // [B] cache slot of the step's token (-1: none)
    uint16_t* k_cache;         // the caches kc / vc, written at the slots
    uint16_t* v_cache;
    int64_t max_position, num_slots;
    float eps;
};

// FUSED prologue.  Every wave normalises and rotates the group's G q heads
// itself, sixteen lanes per head as qk_norm_rope_store does (qk_head16: lane
// j of a head holds dims 4j .. 4j+3 and 64 + 4j .. 64 + 4j+3), into LDS rows
// of its own, so no workgroup barrier couples the four waves.  Loads of one
// head's values and norm weights for lane offset j4 = 4j:
struct Head16 {
    uint2 xa, xb, wa, wb;
};
__device__ __forceinline__ Head16 head16_loads(const uint16_t* src, const uint16_t* w, int j4) {
    return Head16{*reinterpret_cast<const uint2*>(src + j4), *reinterpret_cast<const uint2*>(src + 64 + j4),
                  *reinterpret_cast<const uint2*>(w + j4), *reinterpret_cast<const uint2*>(w + 64 + j4)};
}
// cos and sin of dims j4 .. j4+3 at position pos (row 0 outside the table).
__device__ __forceinline__ void rope_cs(const QkvStep& qs, int64_t pos, int j4, v4f& c, v4f& sn) {
    if (pos < 0 || pos >= qs.max_position) pos = 0;
    c = *reinterpret_cast<const v4f*>(qs.cos_sin + pos * PA_D + j4);
    sn = *reinterpret_cast<const v4f*>(qs.cos_sin + pos * PA_D + 64 + j4);
}
// Orders one wave's LDS accesses (the LDS unit runs them in order) without a
// workgroup barrier.
__device__ __forceinline__ void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// The step's key (norm + rotary, by all four sixteen-lane groups alike) into
// ko1 / ko2, and the value chunk loaded by the caller (lane (kq, rc): dims
// 8 rc .. 8 rc + 7); lanes 0-15 store the key (store_k) and the value
// (store_v) at the slot.
__device__ __forceinline__ void kv_step(const QkvStep& qs, const Head16& kh, v4u vch, const v4f& c, const v4f& sn,
                                        int64_t slot, bool store_k, bool store_v, int Hkv, int kvh, int lane,
                                        uint2& ko1, uint2& ko2) {
    const int j4 = (lane & 15) * 4;
    qk_head16(kh.xa, kh.xb, kh.wa, kh.wb, c, sn, qs.eps, ko1, ko2);
    if (store_k && lane < 16) {
        uint16_t* dst = qs.k_cache + (slot * Hkv + kvh) * PA_D;
        *reinterpret_cast<uint2*>(dst + j4) = ko1;
        *reinterpret_cast<uint2*>(dst + 64 + j4) = ko2;
    }
    if (store_v && lane < 16) *reinterpret_cast<v4u*>(qs.v_cache + (slot * Hkv + kvh) * PA_D + 8 * lane) = vch;
}

// The arguments the first loads need (q, the caches, the block table, the
// context lengths, max_blocks, bs, Hkv, max_ctx) come first: they fill the 14
// argument dwords preloaded into SGPRs at wave launch, so the context length
// and block-table loads issue before any wait.  BLK: 0 for any block size, 16 for block
// sizes that are multiples of 16, PA_SPLIT for blocks of exactly PA_SPLIT.
template <int G, int BLK, bool FUSED>
__global__ void __launch_bounds__(PA_THREADS)
pa_split(const uint16_t* __restrict__ q, const uint16_t* kc, const uint16_t* vc,
         const int32_t* __restrict__ block_tables, const int32_t* __restrict__ context_lens, int max_blocks, int bs,
         int Hkv, int max_ctx, int64_t q_row, uint16_t* __restrict__ out, float* __restrict__ part_o,
         float* __restrict__ part_ml, int S, float qscale, QkvStep qs) {
    constexpr bool BLK16 = BLK != 0;
    const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int Hq = Hkv * G;
    const int start = s * PA_SPLIT;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int32_t* bt = block_tables + (int64_t)b * max_blocks;
    const int clen = context_lens[b];
    // Blocks of PA_SPLIT tokens (BLK == PA_SPLIT): the split is block s, whose
    // entry goes out with the context length, in one round trip (clamped
    // into the row; for a split that runs, start < ctx <= max_blocks * bs, so
    // s < max_blocks and every token of the split, clamped runs included,
    // lies in block s).
    int bt_split = 0;
    if constexpr (BLK == PA_SPLIT) {
        bt_split = bt[min(s, max_blocks - 1)];
        // Issued with the context length, ahead of the wait on the other
        // (non-preloaded) arguments.
        asm volatile("" ::"s"(bt_split), "s"(clen));
    }
    const int ctx = min(clen, max_ctx);  // never past the block table's row
    const uint16_t* qrow = q + (int64_t)b * q_row;
    int64_t slot = -1, pos = 0;
    bool kv_wg = false, slot_ok = false;
    if constexpr (FUSED) {
        // Read with the context length, in one round trip.
        pos = qs.positions[b];
        slot = qs.slots[b];
        slot_ok = slot >= 0 && slot < qs.num_slots;
        kv_wg = s == (ctx > 0 ? (ctx - 1) / PA_SPLIT : 0);
    }
    if (start >= ctx) {
        if constexpr (FUSED) {
            if (kv_wg) {  // an empty context: only the store
                const int j4 = (lane & 15) * 4;
                v4f c, sn;
                rope_cs(qs, pos, j4, c, sn);
                const Head16 kh = head16_loads(qrow + (int64_t)(Hq + kvh) * PA_D, qs.kw, j4);
                const v4u vch =
                    *reinterpret_cast<const v4u*>(qrow + (int64_t)(Hq + Hkv + kvh) * PA_D + 8 * (lane & 15));
                uint2 ko1, ko2;
                kv_step(qs, kh, vch, c, sn, slot, slot_ok && wave == 3, slot_ok && wave == 2, Hkv, kvh, lane, ko1,
                        ko2);
            }
        }
        // Nothing of this sequence here; pass 2 skips the split.  An empty
        // context (ctx <= 0) with a single split has no pass 2: its output
        // is defined as zeros.
        if (S == 1)
            for (int e = threadIdx.x; e < G * PA_D; e += PA_THREADS)
                out[((int64_t)b * Hq + kvh * G + e / PA_D) * PA_D + e % PA_D] = 0;
        return;
    }
    const int end = min(start + PA_SPLIT, ctx);
    const int kq = lane >> 4, rc = lane & 15;  // MFMA k-octet and row/column of the lane

    __shared__ float sm_m[4][G], sm_l[4][G];
    __shared__ float sm_o[4][G][PA_D];
    // Per wave: one half's K rows (2 runs x 16 tokens) on their way to the
    // operand layout.
    __shared__ __align__(16) uint8_t s_kt[4][2 * 16 * PA_KT_ROW];
    // FUSED: per wave, the G normalised, rotated q heads, then the step's key.
    __shared__ __align__(16) uint16_t s_qk[FUSED ? 4 : 1][G + 1][PA_D];

    const uint32_t row = (uint32_t)Hkv * PA_D;  // elements between consecutive slots
    const uint16_t* kbase = kc + kvh * PA_D + 8 * rc;
    const uint16_t* vbase = vc + kvh * PA_D + 8 * rc;
    // First token of half hh (32 tokens) of this wave; a half is two 16-token
    // runs, 16-aligned.
    auto half0 = [&](int hh) { return start + 64 * wave + 32 * hh; };
    // A run of 16 tokens starting at t0 (wave-uniform), clamped into the
    // sequence: token t0 + d is token t0c + min(d, ctx - 1 - t0c).  With
    // block_size % 16 == 0 the run lies in one block, whose block-table entry
    // run_of reads ahead of its use (read at entry for BLK == PA_SPLIT).
    struct Run {
        int t0c, blk;
    };
    auto run_of = [&](int t0) {
        Run r;
        r.t0c = min(t0, ctx - 1);
        if constexpr (BLK == PA_SPLIT)
            r.blk = bt_split;
        else
            r.blk = BLK16 ? bt[r.t0c / bs] : 0;
        return r;
    };
    auto slot_of = [&](const Run& r, int d) -> uint32_t {
        const int c = r.t0c + min(d, ctx - 1 - r.t0c);
        if constexpr (BLK16)
            return (uint32_t)(r.blk * bs + c % bs);
        else
            return (uint32_t)(bt[c / bs] * bs + c % bs);
    };
    // Loads of one half (non-temporal: each K/V byte is read once per step;
    // 2 % faster than plain loads at bs32 x 4.1k tokens).  K and V alike, as
    // rows: lane (kq, rc) holds chunk rc (16 bytes) of tokens h0 + 16c + 4kq
    // + r, so every instruction reads four whole 256-byte rows (K read as
    // 16 tokens x 64 bytes per instruction, in the operand order, streamed
    // at 5.2 against 7.0 TB/s for whole rows).  k_operand then turns K into
    // the A operand of the score MFMA through LDS: lane (kq, rc) holds chunks
    // kq, kq+4, kq+8, kq+12 of token h0 + 16c + rc.
    auto issue = [&](v4u (&kx)[8], v4u (&vx)[8], const Run& r0, const Run& r1) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const Run& r = c ? r1 : r0;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                kx[4 * c + i] =
                    __builtin_nontemporal_load(reinterpret_cast<const v4u*>(kbase + (uint64_t)slot_of(r, 4 * kq + i) * row));
        }
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const Run& r = c ? r1 : r0;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                vx[4 * c + i] =
                    __builtin_nontemporal_load(reinterpret_cast<const v4u*>(vbase + (uint64_t)slot_of(r, 4 * kq + i) * row));
        }
    };
    // Row-layout K of one half -> A-operand layout, through this wave's LDS
    // rows (272-byte stride: the transposed reads spread over the banks).
    // LDS accesses of one wave run in order, so the next half may reuse them.
    uint8_t* kt = reinterpret_cast<uint8_t*>(s_kt[wave]);
    auto k_operand = [&](v4u (&kx)[8]) {
        wave_lds_order();
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<v4u*>(kt + c * 16 * PA_KT_ROW + (4 * kq + i) * PA_KT_ROW + 16 * rc) = kx[4 * c + i];
        wave_lds_order();
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int st = 0; st < 4; ++st)
                kx[4 * c + st] = *reinterpret_cast<const v4u*>(kt + c * 16 * PA_KT_ROW + rc * PA_KT_ROW + 16 * (kq + 4 * st));
    };

    // B operand of the score MFMA: q of head rc (zero past the group's G
    // heads), 8 dims per k-octet in the chunk order of the K operand.  Loaded
    // first and unconditionally (a clamped head, then zeroed), so that the
    // first half's waits leave the second half's loads in flight.
    v8bf qb[4];
    // FUSED: the q head of this lane's sixteen-lane group (clamped to the
    // group's G), rotary factors, norm weights; in the storing workgroup also
    // the step's key head and the value chunk of the V operand's layout.
    const int j4 = (lane & 15) * 4;
    Head16 qh{}, kh;
    v4u vch;
    v4f c{}, sn{};
    const int tl = ctx - 1;                       // the last context token
    const int w_last = (tl - start) >> 6;         // the wave holding it (kv_wg)
    bool subst = false;      // FUSED: see below
    if constexpr (FUSED) {
        // Ahead of the K and V loads, like q in the plain form: they arrive
        // first, and the q products below overlap the K and V loads.
        qh = head16_loads(qrow + (int64_t)(kvh * G + min(lane >> 4, G - 1)) * PA_D, qs.qw, j4);
        rope_cs(qs, pos, j4, c, sn);
        if (kv_wg) {
            kh = head16_loads(qrow + (int64_t)(Hq + kvh) * PA_D, qs.kw, j4);
            vch = *reinterpret_cast<const v4u*>(qrow + (int64_t)(Hq + Hkv + kvh) * PA_D + 8 * rc);
        }
    } else {
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            v4u w = *reinterpret_cast<const v4u*>(qrow + (int64_t)(kvh * G + min(rc, G - 1)) * PA_D +
                                                  8 * (kq + 4 * st));
            if (rc >= G) w = v4u{0u, 0u, 0u, 0u};
            qb[st] = __builtin_bit_cast(v8bf, w);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    v4u ka[8], va[8], kb[8], vb[8];
    {
        const Run a0 = run_of(half0(0)), a1 = run_of(half0(0) + 16);
        const Run b0 = run_of(half0(1)), b1 = run_of(half0(1) + 16);
        issue(ka, va, a0, a1);
        __builtin_amdgcn_sched_barrier(0);
        issue(kb, vb, b0, b1);
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (FUSED) {
        // (Read after the K and V loads are issued, its wait overlaps them.)
        subst = kv_wg && slot_ok && clen == ctx &&
                (int64_t)(block_tables[(int64_t)b * max_blocks + tl / bs] * bs + tl % bs) == slot;
        uint16_t (*sq)[PA_D] = s_qk[wave];
        {
            uint2 o1, o2;
            qk_head16(qh.xa, qh.xb, qh.wa, qh.wb, c, sn, qs.eps, o1, o2);
            if ((lane >> 4) < G) {
                *reinterpret_cast<uint2*>(&sq[lane >> 4][j4]) = o1;
                *reinterpret_cast<uint2*>(&sq[lane >> 4][64 + j4]) = o2;
            }
        }
        // The wave holding the last context token computes and stores the
        // step's key and value; only it needs the key (past the token every
        // lane is masked out of the scores).
        if (kv_wg && wave == w_last) {
            uint2 ko1, ko2;
            kv_step(qs, kh, vch, c, sn, slot, slot_ok, slot_ok, Hkv, kvh, lane, ko1, ko2);
            if (lane < 16) {
                *reinterpret_cast<uint2*>(&sq[G][j4]) = ko1;
                *reinterpret_cast<uint2*>(&sq[G][64 + j4]) = ko2;
            }
        }
        wave_lds_order();
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            v4u w = *reinterpret_cast<const v4u*>(&sq[min(rc, G - 1)][8 * (kq + 4 * st)]);
            if (rc >= G) w = v4u{0u, 0u, 0u, 0u};
            qb[st] = __builtin_bit_cast(v8bf, w);
        }
    }
    // FUSED: the cache slot of the last context token was loaded before this
    // step's key and value reached it: every operand lane that holds that
    // token (the clamped lanes past the end too) takes them instead, right
    // before the half's products (which wait for its loads anyway).  Only
    // when the token is the step's own (context not cut by max_ctx) and its
    // block-table slot is the one just stored.
    v4u knew[4];
    if constexpr (FUSED) {
        if (subst && wave == w_last) {
#pragma unroll
            for (int st = 0; st < 4; ++st)
                knew[st] = *reinterpret_cast<const v4u*>(&s_qk[wave][G][8 * (kq + 4 * st)]);
        }
    }
    // Waves past w_last take only the value (a finite one for the masked
    // lanes, as the two-launch form reads there).
    auto take = [&](v4u (&kx)[8], v4u (&vx)[8], int h0) {
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const int t0 = h0 + 16 * cc;
            if (wave == w_last && t0 + rc >= tl)
#pragma unroll
                for (int st = 0; st < 4; ++st) kx[4 * cc + st] = knew[st];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (t0 + 4 * kq + i >= tl) vx[4 * cc + i] = vch;
        }
    };

    // Softmax state of head rc (the same in the four k-octet rows): running
    // max m (raw score units), partial sum l over this lane's tokens.  Output
    // accumulators: tile t holds O[head 4kq + r][dim 8rc + t].
    float m = -__builtin_inff(), l = 0.0f;
    v4f acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](const v4u (&kx)[8], const v4u (&vx)[8], int h0) {
        // Scores S[token h0 + 16c + 4kq + r][head rc].
        v4f sv[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            sv[c] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < 4; ++st)
                sv[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, kx[4 * c + st]), qb[st],
                                                                  sv[c], 0, 0, 0);
        }
        float sc[8];
        float mx = -__builtin_inff();
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int tk = h0 + 16 * (e >> 2) + 4 * kq + (e & 3);
            sc[e] = tk < end ? sv[e >> 2][e & 3] : -__builtin_inff();
            mx = fmaxf(mx, sc[e]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);
        // no live token yet: the state stays m = -inf, l = 0, o = 0
        const bool any = mn != -__builtin_inff();
        const float off = any ? -mn * qscale : 0.0f;
        const float corr = any ? __builtin_amdgcn_exp2f(__builtin_fmaf(m, qscale, off)) : 1.0f;
        m = mn;
        float p[8], ls = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[e], qscale, off));
            ls += p[e];
        }
        l = l * corr + ls;
        // A operand of the output MFMA: P[head rc][token (kq, e)], bf16
        // (as flash attention rounds P for its P.V product); zero past G.
        v4u pw;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const v2bf pp = __builtin_convertvector((v2f){p[2 * w], p[2 * w + 1]}, v2bf);
            pw[w] = rc < G ? __builtin_bit_cast(uint32_t, pp) : 0u;
        }
        const v8bf pa = __builtin_bit_cast(v8bf, pw);
        // Rescale rows 0..G-1 (heads 0..G-1 sit in the kq = 0 lanes; other
        // rows are unused) when a head's max moved.
        float cr[G];
        bool moved = false;
#pragma unroll
        for (int h = 0; h < G; ++h) {
            cr[h] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, corr), h));
            moved |= cr[h] != 1.0f;
        }
        if (moved) {
#pragma unroll
            for (int t = 0; t < 8; ++t)
#pragma unroll
                for (int h = 0; h < G; ++h) acc[t][h] *= cr[h];
        }
        // B operand of tile t: V[token (kq, e)][dim 8rc + t], e = 0..7, from
        // this lane's 8 rows (an 8 x 8 transpose of bf16 pairs).
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t sel = (t & 1) ? 0x07060302u : 0x05040100u;
            v4u bw;
#pragma unroll
            for (int w = 0; w < 4; ++w) bw[w] = __builtin_amdgcn_perm(vx[2 * w + 1][t >> 1], vx[2 * w][t >> 1], sel);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, __builtin_bit_cast(v8bf, bw), acc[t], 0, 0, 0);
        }
    };

    k_operand(ka);
    if (subst && wave >= w_last) take(ka, va, half0(0));
    compute(ka, va, half0(0));
    k_operand(kb);
    if (subst && wave >= w_last) take(kb, vb, half0(1));
    compute(kb, vb, half0(1));

    // Merge the four wave states of the workgroup.
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (kq == 0) {
        if (rc < G) {
            sm_m[wave][rc] = m;
            sm_l[wave][rc] = l;
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
            *reinterpret_cast<v4f*>(&sm_o[wave][h][8 * rc]) = v4f{acc[0][h], acc[1][h], acc[2][h], acc[3][h]};
            *reinterpret_cast<v4f*>(&sm_o[wave][h][8 * rc + 4]) = v4f{acc[4][h], acc[5][h], acc[6][h], acc[7][h]};
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < G * PA_D; e += PA_THREADS) {
        const int h = e / PA_D, d = e % PA_D;
        float M = -__builtin_inff();
#pragma unroll
        for (int w = 0; w < 4; ++w) M = fmaxf(M, sm_m[w][h]);
        float Lw = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float wt = sm_m[w][h] == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f((sm_m[w][h] - M) * qscale);
            Lw = __builtin_fmaf(wt, sm_l[w][h], Lw);
            O = __builtin_fmaf(wt, sm_o[w][h][d], O);
        }
        const int hq = kvh * G + h;
        if (S == 1) {
            out[((int64_t)b * Hq + hq) * PA_D + d] = (uint16_t)f32_to_bf16_rne(O / Lw);
        } else {
            const int64_t ps = ((int64_t)b * Hq + hq) * S + s;
            part_o[ps * PA_D + d] = O;
            if (d == 0) {
                part_ml[ps * 2] = M * qscale;  // base-2 units for the merge
                part_ml[ps * 2 + 1] = Lw;
            }
        }
    }
}

// Split merge, one wave per (sequence, query head).  SMAX > 0 (S <= SMAX
// <= 64 splits): the split maxima and every partial row are loaded with the
// context length, in one round trip to memory (rows past S repeat row S-1
// and are not used), then merged with the operation sequence of the general
// form below for a single chunk, so the result has the same bits.  SMAX = 0:
// any S, in chunks of 64 splits.
template <int SMAX>
__global__ void __launch_bounds__(64)
pa_merge(const int32_t* __restrict__ context_lens, const float* __restrict__ part_o,
         const float* __restrict__ part_ml, uint16_t* __restrict__ out, int Hq, int S, int max_ctx) {
    const int hq = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
    const int64_t base = ((int64_t)b * Hq + hq) * S;
    if constexpr (SMAX > 0) {
        const int clen = context_lens[b];
        const float2 ml = *reinterpret_cast<const float2*>(part_ml + (base + min(lane, S - 1)) * 2);
        float2 v[SMAX];
#pragma unroll
        for (int u = 0; u < SMAX; ++u)
            v[u] = *reinterpret_cast<const float2*>(part_o + (base + min(u, S - 1)) * PA_D + 2 * lane);
        // Every row is used only under u < n below; without these pins the
        // compiler may move each load into its branch, one round trip per row.
#pragma unroll
        for (int u = 0; u < SMAX; ++u) asm volatile("" : "+v"(v[u].x), "+v"(v[u].y));
        const int n = min(S, (min(clen, max_ctx) + PA_SPLIT - 1) / PA_SPLIT);
        const float ms = lane < n ? ml.x : -__builtin_inff(), ls = lane < n ? ml.y : 0.0f;
        float M = ms;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
        const float w = lane < n ? __builtin_amdgcn_exp2f(ms - M) : 0.0f;
        float L = w * ls;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) L += __shfl_xor(L, off);
        L = 0.0f + L;
        float O0 = 0.0f, O1 = 0.0f;
#pragma unroll
        for (int u = 0; u < SMAX; ++u) {
            if (u < n) {
                const float wk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), u));
                O0 = __builtin_fmaf(wk, v[u].x, O0);
                O1 = __builtin_fmaf(wk, v[u].y, O1);
            }
        }
        uint16_t* o = out + ((int64_t)b * Hq + hq) * PA_D + 2 * lane;
        // n == 0 (an empty context): L == 0 and the output is zeros.
        *reinterpret_cast<uint32_t*>(o) = n > 0 ? f32_to_bf16_rne(O0 / L) | (f32_to_bf16_rne(O1 / L) << 16) : 0u;
        return;
    }
    const int n = min(S, (min(context_lens[b], max_ctx) + PA_SPLIT - 1) / PA_SPLIT);
    float O0 = 0.0f, O1 = 0.0f, L = 0.0f;
    // Splits in chunks of 64 (one per lane); the running max M rescales
    // earlier chunks when a later one raises it.
    float M = -__builtin_inff();
    for (int c0 = 0; c0 < n; c0 += 64) {
        const int sidx = c0 + lane;
        float ms = -__builtin_inff(), ls = 0.0f;
        if (sidx < n) {
            const float2 ml = *reinterpret_cast<const float2*>(part_ml + (base + sidx) * 2);
            ms = ml.x;
            ls = ml.y;
        }
        float cm = ms;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) cm = fmaxf(cm, __shfl_xor(cm, off));
        const float Mn = fmaxf(M, cm);
        const float corr = M == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(M - Mn);
        O0 *= corr;
        O1 *= corr;
        L *= corr;
        M = Mn;
        const float w = sidx < n ? __builtin_amdgcn_exp2f(ms - M) : 0.0f;
        float wl = w * ls;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) wl += __shfl_xor(wl, off);
        L += wl;
        const int cnt = min(64, n - c0);
        constexpr int U = 8;
        for (int k0 = 0; k0 < cnt; k0 += U) {
            float2 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int k = min(k0 + u, cnt - 1);
                v[u] = *reinterpret_cast<const float2*>(part_o + (base + c0 + k) * PA_D + 2 * lane);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (k0 + u < cnt) {
                    const float wk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w),
                                                                                         k0 + u));
                    O0 = __builtin_fmaf(wk, v[u].x, O0);
                    O1 = __builtin_fmaf(wk, v[u].y, O1);
                }
            }
        }
    }
    uint16_t* o = out + ((int64_t)b * Hq + hq) * PA_D + 2 * lane;
    *reinterpret_cast<uint32_t*>(o) = n > 0 ? f32_to_bf16_rne(O0 / L) | (f32_to_bf16_rne(O1 / L) << 16) : 0u;
}

template <int G, bool FUSED>
hipError_t pa_launch(const void* q, int64_t q_row, const void* kc, const void* vc, const int32_t* bt, int max_blocks,
                     const int32_t* cl, void* out, float* ws, int B, int Hkv, int bs, int S, int max_ctx,
                     float qscale, const QkvStep& qs, hipStream_t st) {
    float* part_o = ws;
    float* part_ml = ws + (int64_t)B * Hkv * G * S * PA_D;
    const dim3 grid((unsigned)S, (unsigned)Hkv, (unsigned)B);
    if (bs == PA_SPLIT)
        hipLaunchKernelGGL((pa_split<G, PA_SPLIT, FUSED>), grid, dim3(PA_THREADS), 0, st,
                           static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(kc),
                           static_cast<const uint16_t*>(vc), bt, cl, max_blocks, bs, Hkv, max_ctx, q_row,
                           static_cast<uint16_t*>(out), part_o, part_ml, S, qscale, qs);
    else if (bs % 16 == 0)
        hipLaunchKernelGGL((pa_split<G, 16, FUSED>), grid, dim3(PA_THREADS), 0, st,
                           static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(kc),
                           static_cast<const uint16_t*>(vc), bt, cl, max_blocks, bs, Hkv, max_ctx, q_row,
                           static_cast<uint16_t*>(out), part_o, part_ml, S, qscale, qs);
    else
        hipLaunchKernelGGL((pa_split<G, 0, FUSED>), grid, dim3(PA_THREADS), 0, st,
                           static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(kc),
                           static_cast<const uint16_t*>(vc), bt, cl, max_blocks, bs, Hkv, max_ctx, q_row,
                           static_cast<uint16_t*>(out), part_o, part_ml, S, qscale, qs);
    if (S > 1) {
        const dim3 mg((unsigned)(Hkv * G), (unsigned)B);
        auto* o16 = static_cast<uint16_t*>(out);
        if (S <= 8)
            hipLaunchKernelGGL(pa_merge<8>, mg, dim3(64), 0, st, cl, part_o, part_ml, o16, Hkv * G, S, max_ctx);
        else if (S <= 16)
            hipLaunchKernelGGL(pa_merge<16>, mg, dim3(64), 0, st, cl, part_o, part_ml, o16, Hkv * G, S, max_ctx);
        else if (S <= 24)
            hipLaunchKernelGGL(pa_merge<24>, mg, dim3(64), 0, st, cl, part_o, part_ml, o16, Hkv * G, S, max_ctx);
        else if (S <= 32)
            hipLaunchKernelGGL(pa_merge<32>, mg, dim3(64), 0, st, cl, part_o, part_ml, o16, Hkv * G, S, max_ctx);
        else if (S <= 64)
            hipLaunchKernelGGL(pa_merge<64>, mg, dim3(64), 0, st, cl, part_o, part_ml, o16, Hkv * G, S, max_ctx);
        else
            hipLaunchKernelGGL(pa_merge<0>, mg, dim3(64), 0, st, cl, part_o, part_ml, o16, Hkv * G, S, max_ctx);
    }
    return hipGetLastError();
}

}  // namespace
}  // namespace nv4

// Device scratch of the allocation-free entry point
// (nv4_paged_decode_attention_noalloc): the split partials live here instead
// of in a caller's workspace.  Each device holds its own copy for the life of
// the process; its address on a device comes from hipGetSymbolAddress (the
// name itself is a host-side stand-in that must never reach a kernel).
static __device__ __align__(256) float scratch[NV4_PA_SCRATCH_BYTES / sizeof(float)];

namespace nv4 {
namespace {

// Argument rules shared by both entry points; on success *splits is S.
int pa_check(const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache,
             const int32_t* block_tables, int64_t max_blocks, const int32_t* context_lens, const void* out,
             int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t block_size, int64_t max_context,
             int64_t* splits) {
    if (!q || !k_cache || !v_cache || !block_tables || !context_lens || !out) return NV4_E_NULL;
    // Every factor is bounded before any product, so no size computation
    // below can wrap (max_blocks * block_size <= 2^46, Hq * D <= 2^25).
    if (D != PA_D || B < 1 || Hkv < 1 || Hq < 1 || Hq % Hkv || block_size < 1 || block_size > (1 << 16) ||
        max_blocks < 1 || max_blocks > (1 << 30) || max_context < 1 || max_context > (1 << 30) ||
        max_context > max_blocks * block_size || B > 65535 || Hkv > 65535 || Hq > 4 * 65535 ||
        q_row_stride < Hq * D)
        return NV4_E_SHAPE;
    const int64_t G = Hq / Hkv;
    if (G != 1 && G != 2 && G != 4) return NV4_E_SHAPE;  // the merge keeps 16 x G x 128 fp32 in LDS
    if (reinterpret_cast<uintptr_t>(q) % 16 || reinterpret_cast<uintptr_t>(k_cache) % 16 ||
        reinterpret_cast<uintptr_t>(v_cache) % 16 || reinterpret_cast<uintptr_t>(out) % 4 || q_row_stride % 8)
        return NV4_E_ALIGN;
    *splits = (max_context + PA_SPLIT - 1) / PA_SPLIT;
    return NV4_OK;
}

// Bytes of the split partials, B * Hq * S rows of D + 2 floats, or -1 when
// the product does not fit in int64.
int64_t pa_partials_bytes(int64_t B, int64_t Hq, int64_t S, int64_t D) {
    int64_t n = 0;
    if (__builtin_mul_overflow(B, Hq, &n) || __builtin_mul_overflow(n, S, &n) ||
        __builtin_mul_overflow(n, D + 2, &n) || __builtin_mul_overflow(n, (int64_t)4, &n))
        return -1;
    return n;
}

int pa_run(const void* q, int64_t q_row_stride, const void* k_cache, const void* v_cache,
           const int32_t* block_tables, int64_t max_blocks, const int32_t* context_lens, void* out, float* ws,
           int64_t B, int64_t Hq, int64_t Hkv, int64_t block_size, int64_t max_context, int64_t S, float scale,
           const QkvStep* fused, void* stream) {
    const float qscale = scale * 1.4426950408889634f;  // log2(e): softmax in base 2
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int b = (int)B, hkv = (int)Hkv, bs = (int)block_size, s = (int)S, mb = (int)max_blocks;
    const QkvStep none{};
    auto run = [&](auto g, auto f) {
        constexpr int G = decltype(g)::value;
        constexpr bool F = decltype(f)::value;
        return (int)pa_launch<G, F>(q, q_row_stride, k_cache, v_cache, block_tables, mb, context_lens, out, ws, b,
                                    hkv, bs, s, (int)max_context, qscale, F ? *fused : none, st);
    };
    using T = std::true_type;
    using F = std::false_type;
    switch (Hq / Hkv) {
        case 1: return fused ? run(std::integral_constant<int, 1>{}, T{}) : run(std::integral_constant<int, 1>{}, F{});
        case 2: return fused ? run(std::integral_constant<int, 2>{}, T{}) : run(std::integral_constant<int, 2>{}, F{});
        default:
            return fused ? run(std::integral_constant<int, 4>{}, T{}) : run(std::integral_constant<int, 4>{}, F{});
    }
}

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
constexpr int PA_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[PA_MAX_DEVICES] = {};

int scratch_on_current_device(float** ptr) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= PA_MAX_DEVICES) return NV4_E_SHAPE;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!p) return NV4_E_NULL;
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *ptr = g_scratch_ptr[dev];
    return NV4_OK;
}

}  // namespace
}  // namespace nv4

extern "C" int nv4_paged_decode_attention(const void* q, int64_t q_row_stride, const void* k_cache,
                                          const void* v_cache, const int32_t* block_tables, int64_t max_blocks,
                                          const int32_t* context_lens, void* out, float* workspace,
                                          int64_t workspace_bytes, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                          int64_t block_size, int64_t max_context, float scale, void* stream) {
    using namespace nv4;
    int64_t S = 0;
    const int rc = pa_check(q, q_row_stride, k_cache, v_cache, block_tables, max_blocks, context_lens, out, B, Hq,
                            Hkv, D, block_size, max_context, &S);
    if (rc != NV4_OK) return rc;
    if (!workspace) return NV4_E_NULL;
    const int64_t need = pa_partials_bytes(B, Hq, S, D);
    if (need < 0 || workspace_bytes < need) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(workspace) % 8) return NV4_E_ALIGN;
    return pa_run(q, q_row_stride, k_cache, v_cache, block_tables, max_blocks, context_lens, out, workspace, B, Hq,
                  Hkv, block_size, max_context, S, scale, nullptr, stream);
}

extern "C" int nv4_paged_decode_attention_noalloc(const void* q, int64_t q_row_stride, const void* k_cache,
                                                  const void* v_cache, const int32_t* block_tables,
                                                  int64_t max_blocks, const int32_t* context_lens, void* out,
                                                  int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t block_size,
                                                  int64_t max_context, float scale, void* stream) {
    using namespace nv4;
    int64_t S = 0;
    int rc = pa_check(q, q_row_stride, k_cache, v_cache, block_tables, max_blocks, context_lens, out, B, Hq, Hkv, D,
                      block_size, max_context, &S);
    if (rc != NV4_OK) return rc;
    // Only the split partials (S > 1) use the scratch; their size is checked
    // before anything is launched.
    if (S > 1) {
        const int64_t need = pa_partials_bytes(B, Hq, S, D);
        if (need < 0 || need > NV4_PA_SCRATCH_BYTES) return NV4_E_SCRATCH;
    }
    float* ws = nullptr;
    rc = scratch_on_current_device(&ws);
    if (rc != NV4_OK) return rc;
    return pa_run(q, q_row_stride, k_cache, v_cache, block_tables, max_blocks, context_lens, out, ws, B, Hq, Hkv,
                  block_size, max_context, S, scale, nullptr, stream);
}

extern "C" int nv4_paged_decode_attention_qkv(const void* qkv, int64_t qkv_row_stride, const void* q_norm_w,
                                              const void* k_norm_w, const float* cos_sin, int64_t max_position,
                                              const int64_t* positions, const int32_t* slot_mapping,
                                              int64_t num_slots, void* k_cache, void* v_cache,
                                              const int32_t* block_tables, int64_t max_blocks,
                                              const int32_t* context_lens, void* out, float* workspace,
                                              int64_t workspace_bytes, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                              int64_t block_size, int64_t max_context, float eps, float scale,
                                              void* stream) {
    using namespace nv4;
    int64_t S = 0;
    const int rc = pa_check(qkv, qkv_row_stride, k_cache, v_cache, block_tables, max_blocks, context_lens, out, B,
                            Hq, Hkv, D, block_size, max_context, &S);
    if (rc != NV4_OK) return rc;
    if (!q_norm_w || !k_norm_w || !cos_sin || !positions || !slot_mapping || !workspace) return NV4_E_NULL;
    if (qkv_row_stride < (Hq + 2 * Hkv) * D || max_position < 1 || max_position > ((int64_t)1 << 40) ||
        num_slots < 0)
        return NV4_E_SHAPE;
    const int64_t need = pa_partials_bytes(B, Hq, S, D);
    if (need < 0 || workspace_bytes < need) return NV4_E_SHAPE;
    if (reinterpret_cast<uintptr_t>(workspace) % 8 || reinterpret_cast<uintptr_t>(q_norm_w) % 2 ||
        reinterpret_cast<uintptr_t>(k_norm_w) % 2 || reinterpret_cast<uintptr_t>(cos_sin) % 4 ||
        reinterpret_cast<uintptr_t>(positions) % 8 || reinterpret_cast<uintptr_t>(slot_mapping) % 4)
        return NV4_E_ALIGN;
    const QkvStep qs{static_cast<const uint16_t*>(q_norm_w), static_cast<const uint16_t*>(k_norm_w), cos_sin,
                     positions, slot_mapping, static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
                     max_position, num_slots, eps};
    return pa_run(qkv, qkv_row_stride, k_cache, v_cache, block_tables, max_blocks, context_lens, out, workspace, B,
                  Hq, Hkv, block_size, max_context, S, scale, &qs, stream);
}
