// Paged causal / chunked / non-causal prefill attention, ping-pong form (gfx950, bf16
// MFMA, dense bf16 cache, head_dim 128, power-of-two pages of >= 16 tokens).
//
// Reference: attention_prefill_kernel / prefill_body (src/ops/tile/attention.jl:130-177).
// Query t of the step sits at position start + t (start = positions of the sequence's
// first query, read on the device) and sees keys 0 .. start + t; with causal = 0 it sees
// all start + n keys (attention.jl:155-157).
//
// Why a second prefill kernel. Per 32-key step a wave holding 32 packed query rows
// issues 16 v_mfma_f32_32x32x16_bf16 (about 512 matrix-core cycles) and about 100 VALU
// instructions of softmax (16 of them v_exp_f32; about 500 issue cycles). When every wave
// of a SIMD enters each phase together the two costs add up. Here a work-group is 8 waves
// in two teams of 4 (team A = waves 0-3, team B = waves 4-7; wave w runs on SIMD w % 4,
// so each SIMD holds one wave of each team). Work-group barriers split time into
// phases; in every phase one team runs its MFMAs (QK^T of tile i and PV of tile i-1) while
// the other runs the softmax of its last score tile, so each SIMD's matrix core and VALU
// work at the same time. Team B runs one phase behind team A:
//
//   phase      0      1      2      3      4     ...
//   team A    X0     Y0     X1     Y1     X2
//   team B    --     X0     Y0     X1     Y1
//
//   X_i = S_i = K_i Q^T (8 MFMAs) and O += V_{i-1} P_{i-1} (8 MFMAs)
//   Y_i = online softmax of S_i -> P_i (bf16), lazy rescale of O; K/V staging duties
//
// All 8 waves share every 32-key K/V tile in LDS (256 packed query rows per tile, twice
// the reuse of a 4-wave group). Each thread moves one 16-byte chunk of K and one of V per
// tile: global loads are issued three steps before the tile's V part is needed, K goes to
// LDS two steps ahead, V one step ahead; K and V each live in a three-tile LDS ring (a
// buffer is rewritten only after both teams have read it). Team A's threads carry keys
// 0-15 of a tile and team B's keys 16-31, so a tile's halves are stored in consecutive
// phases and each wave's block-table lookup is a single scalar load.
//
// The per-wave MFMA layouts, the exp2-domain online softmax with lazy rescale, the
// transposing V reads and the output / split-partial formats are those of the
// four-wave prefill kernel (pa_prefill.hip).
#include <stdlib.h>

#include <type_traits>

#include "common.hpp"

using namespace ti;

namespace {

constexpr int D = 128;
constexpr int KT = 32;                 // keys per tile
constexpr int NW = 8;                  // waves per work-group
constexpr int ROWS = 32 * NW;          // packed query rows per work-group
constexpr int NBUF = 3;                // LDS ring depth (K and V each)
constexpr int KROW = D + 8;            // K row stride (bf16): 16-B reads by 16 keys hit 64 banks
constexpr int VROW = D + 32;           // V row stride: transposing reads bank-disjoint
constexpr float RESCALE_LOG2 = 8.0f;   // lazy-rescale threshold

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

struct PPParams {
    const uint16_t *q;
    uint16_t *out;
    const uint16_t *kp, *vp;
    const int32_t *positions, *qsl, *bt;
    float *part;                       // split partials [B][Hk][splits][M][D + 2]
    int bt_stride, num_pages, P, pshift, Hk, Hq, G, TQ, nmax, qtiles, causal, splits, M;
    float scale_log2;
};

struct PPSmem {
    uint16_t k[NBUF][KT * KROW];
    uint16_t v[NBUF][KT * VROW];
};

__device__ __forceinline__ u32x2 lds_tr16(const uint16_t *p) {
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4 *)(__attribute__((address_space(3))) uint16_t *)p);
    return __builtin_bit_cast(u32x2, v);
}

template <int I> using IC = std::integral_constant<int, I>;

__global__ void __launch_bounds__(64 * NW) prefill_pp_kernel(PPParams p) {
    constexpr int NQB = D / 16;        // score MFMAs per tile (16 head-dim elements each)
    constexpr int NDB = D / 32;        // 32-row blocks of O^T
    __shared__ __attribute__((aligned(16))) PPSmem sm;

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int team = w >> 2;                       // 0: A, 1: B
    const int r32 = lane & 31, kg = lane >> 5;
    const int h = blockIdx.x;
    const int qt = p.qtiles - 1 - (int)blockIdx.y / p.splits;   // heaviest q-tiles first
    const int split = (int)blockIdx.y % p.splits;
    const int b = blockIdx.z;
    const int tok0 = p.qsl ? sload(p.qsl, b) : b * p.nmax;
    const int nb = p.qsl ? min(sload(p.qsl, b + 1) - tok0, p.nmax) : p.nmax;   // at most max_query_len
    const int start = max(sload(p.positions, nb > 0 ? tok0 : 0), 0), len = start + nb;   // a negative position reads as 0
    const int t_first = qt * p.TQ;
    if (t_first >= nb) return;
    const int t_last = min(t_first + p.TQ, nb) - 1;
    const int kend = p.causal ? start + t_last + 1 : len;
    const int nkt = (kend + KT - 1) / KT;
    const int per = (nkt + p.splits - 1) / p.splits;
    const int kt_lo = min(split * per, nkt), kt_hi = min(kt_lo + per, nkt);
    const int N = kt_hi - kt_lo;                   // key tiles of this work-group
    const size_t unit = ((size_t)b * p.Hk + h) * p.splits + split;
    const int32_t *bt = p.bt + (size_t)b * p.bt_stride;
    const int mask_from = p.causal ? start + t_first : len - 1;
    if (N == 0) {
        // A split with no keys: neutral partials (m = -big, l = 0, acc = 0).
        for (int idx = tid; idx < ROWS * (D + 2); idx += 64 * NW) {
            const int rr = idx / (D + 2), c = idx - rr * (D + 2);
            const int ttl = rr / p.G, gg = rr - ttl * p.G, tt = t_first + ttl;
            if (ttl < p.TQ && tt < nb)
                p.part[(unit * p.M + (size_t)tt * p.G + gg) * (D + 2) + c] = c == D ? NEG_BIG : 0.0f;
        }
        return;
    }

    // This thread's staging chunk of every tile: key ckey (team A: 0-15, team B: 16-31),
    // 16-byte chunk cch of the head dimension.
    const int ckey = tid >> 4, cch = tid & 15;
    const int half = team;                         // == ckey >> 4, wave-uniform
    const long long chunk_off = (long long)(ckey & 15) * D + cch * 8;

    // This wave's half of tile j (clamped to the last tile, so loads past the end re-read
    // it and are never stored): its block-table entry (raw_half, a scalar load, looked up a
    // step before use so its wait does not fall right after it) and its row base in
    // elements (half_base: page clamped into the pool, 32-bit page stride and head offset).
    const uint32_t pstride = (uint32_t)p.Hk * p.P * D, hoff = (uint32_t)h * p.P * D;
    auto half_pos = [&](int j) { return (kt_lo + min(j, N - 1)) * KT + 16 * half; };
    auto raw_half = [&](int j) { return sload(bt, min(half_pos(j) >> p.pshift, p.bt_stride - 1)); };
    auto half_base = [&](int raw, int j) -> long long {
        return (long long)((uint64_t)(uint32_t)clamp_page(raw, p.num_pages) * pstride + hoff +
                           (uint32_t)((half_pos(j) & (p.P - 1)) * D));
    };

    struct Stage {
        u32x4 k, v;
    };
    Stage st[NBUF];
    auto load = [&](Stage &s, long long base) {
        s.k = *reinterpret_cast<const u32x4 *>(p.kp + base + chunk_off);
        s.v = *reinterpret_cast<const u32x4 *>(p.vp + base + chunk_off);
    };
    auto store_k = [&](const Stage &s, int buf) {
        *reinterpret_cast<u32x4 *>(&sm.k[buf][ckey * KROW + cch * 8]) = s.k;
    };
    auto store_v = [&](const Stage &s, int buf, int j) {
        // Keys past kend in the last tile may hold any bits (even NaN) of an allocated
        // page: their probabilities are 0 and their values must be finite. Branch-free,
        // so the stage registers are never rewritten while loads are pending.
        const uint32_t keep = (kt_lo + j) * KT + ckey < kend ? ~0u : 0u;
        *reinterpret_cast<u32x4 *>(&sm.v[buf][ckey * VROW + cch * 8]) = s.v & keep;
    };

    // Query rows (B operand of S^T = K Q^T): wave w holds rows 32 w .. 32 w + 31.
    const int r = w * 32 + r32, tl = r / p.G, g = r - tl * p.G, t = t_first + tl;
    const bool row_ok = tl < p.TQ && t < nb;
    const int qpos = p.causal && row_ok ? start + t : len - 1;
    bf16x8 qreg[NQB];
    {
        const uint16_t *qr = p.q + ((size_t)(tok0 + (row_ok ? t : 0)) * p.Hq + h * p.G + g) * D;
#pragma unroll
        for (int i = 0; i < NQB; i++)
            qreg[i] = row_ok ? as_bf16x8(*reinterpret_cast<const u32x4 *>(qr + i * 16 + kg * 8))
                             : as_bf16x8((u32x4){0u, 0u, 0u, 0u});
    }

    // Prologue: tiles 0-2 in flight; tile 0's K and V and tile 1's K in LDS; tile 3 in
    // flight in stage 0.
    // (Scheduling fences keep the loads in tile order, so the waits before each LDS
    // store count exactly the younger tiles still in flight.)
    int r0 = raw_half(0), r1 = raw_half(1), r2 = raw_half(2), r3 = raw_half(3);
    long long nbase = half_base(r0, 0);
    load(st[0], nbase);
    nbase = half_base(r1, 1);
    __builtin_amdgcn_sched_barrier(0);
    load(st[1], nbase);
    nbase = half_base(r2, 2);
    __builtin_amdgcn_sched_barrier(0);
    load(st[2], nbase);
    nbase = half_base(r3, 3);
    int nraw = raw_half(4);
    __builtin_amdgcn_sched_barrier(0);
    store_k(st[0], 0);
    store_v(st[0], 0, 0);
    // Unconditional (with one tile, tile 1 is a re-read of tile 0 that is never used):
    // a branch here would let the compiler sink the next load into it and leave the
    // loop with two different counts of loads in flight, which costs conservative waits.
    store_k(st[1], 1);
    load(st[0], nbase);
    nbase = half_base(nraw, 4);
    nraw = raw_half(5);

    f32x16 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; db++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[db][e] = 0.0f;
    float m = NEG_BIG, l = 0.0f;
    bf16x8 pb[2];
    pb[0] = pb[1] = as_bf16x8((u32x4){0u, 0u, 0u, 0u});
    f32x16 sc;

    const int c16 = lane >> 4, s16 = lane & 15;
    const int tr_row = 4 * (c16 >> 1) + (s16 >> 2), tr_col = 16 * (c16 & 1) + 4 * (s16 & 3);

    // O^T += V^T P^T for the tile in V buffer vb.
    auto pv = [&](int vb) {
        const uint16_t *vbase = &sm.v[vb][tr_row * VROW + tr_col];
#pragma unroll
        for (int db = 0; db < NDB; db++)
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const u32x2 lo = lds_tr16(vbase + (16 * hh) * VROW + 32 * db);
                const u32x2 hi = lds_tr16(vbase + (16 * hh + 8) * VROW + 32 * db);
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8((u32x4){lo[0], lo[1], hi[0], hi[1]}),
                                                               pb[hh], o[db], 0, 0, 0);
            }
    };
    // S^T = K Q^T for the tile in K buffer kb (one accumulation chain: dependent MFMAs
    // issue back to back).
    auto qk = [&](int kb) {
#pragma unroll
        for (int e = 0; e < 16; e++) sc[e] = 0.0f;
        const uint16_t *krow = &sm.k[kb][r32 * KROW + kg * 8];
#pragma unroll
        for (int i = 0; i < NQB; i++)
            sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(*reinterpret_cast<const u32x4 *>(krow + i * 16)),
                                                         qreg[i], sc, 0, 0, 0);
    };
    // Online softmax of tile j's scores (exp2 domain, lazy rescale) -> pb. Only tiles
    // reaching past mask_from (the diagonal / last tiles) compare key positions.
    auto softmax = [&](int j, auto need_mask) {
        const int kt = kt_lo + j;
        if (need_mask) {
            // A real branch (the empty asm keeps the compiler from if-converting the
            // selects into every tile): key 8 (e / 4) + 4 kg + e % 4 is visible iff
            // it is <= qpos - kt * KT.
            asm volatile("");
            const int lim = qpos - kt * KT - 4 * kg;
#pragma unroll
            for (int e = 0; e < 16; e++)
                sc[e] = 8 * (e >> 2) + (e & 3) <= lim ? sc[e] : -INFINITY;
        }
        float x[16];
        float mt = -INFINITY;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            x[e] = sc[e];
            mt = fmaxf(mt, x[e]);
        }
        mt *= p.scale_log2;
        if (__any(mt > m + RESCALE_LOG2)) {
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float mn = fmaxf(m, mt);
            const float alpha = fast_exp2(m - mn);
            m = mn;
            l *= alpha;
#pragma unroll
            for (int db = 0; db < NDB; db++) o[db] *= alpha;
        }
        float pe[16], ps = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            pe[e] = fast_exp2(__builtin_fmaf(x[e], p.scale_log2, -m));
            ps += pe[e];
        }
        l += ps;
#pragma unroll
        for (int hh = 0; hh < 2; hh++)
            pb[hh] = as_bf16x8((u32x4){pack_bf16x2(pe[8 * hh + 0], pe[8 * hh + 1]), pack_bf16x2(pe[8 * hh + 2], pe[8 * hh + 3]),
                                       pack_bf16x2(pe[8 * hh + 4], pe[8 * hh + 5]), pack_bf16x2(pe[8 * hh + 6], pe[8 * hh + 7])});
    };

    // Phase boundary: no instruction is scheduled across it, so each phase keeps only its
    // own work (the matrix-core phase must not absorb softmax VALU work).
    auto phase_barrier = [] {
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
    };
    // One step i (ring slot S = i % 3): phase X_i, barrier, phase Y_i, barrier.
    auto step = [&](int i, auto slot, auto need_mask) {
        constexpr int S = decltype(slot)::value;
        constexpr int S1 = (S + 1) % NBUF, S2 = (S + 2) % NBUF;
        qk(S);
        if (i > 0) pv(S2);                           // tile i - 1
        phase_barrier();
        softmax(i, need_mask);
        if (i + 2 < N) store_k(st[S2], S2);          // tile i + 2 (loaded at step i - 2)
        if (i + 1 < N) store_v(st[S1], S1, i + 1);   // tile i + 1 (loaded at step i - 3)
        load(st[S1], nbase);                         // tile i + 4
        nbase = half_base(nraw, i + 5);
        nraw = raw_half(i + 6);
        phase_barrier();
    };
    // First tile (relative) whose keys reach past mask_from.
    const int jm = max(0, (mask_from + 1) / KT - kt_lo);
    auto step_m = [&](int i, auto slot) { step(i, slot, i >= jm); };

    phase_barrier();
    if (team == 1) phase_barrier();                  // team B runs one phase behind
    for (int i = 0; i < N; i += 3) {
        step_m(i, IC<0>{});
        if (i + 1 >= N) break;
        step_m(i + 1, IC<1>{});
        if (i + 2 >= N) break;
        step_m(i + 2, IC<2>{});
    }
    pv((N - 1) % NBUF);                              // last tile's PV
    if (team == 0) phase_barrier();

    l += __shfl_xor(l, 32);
    if (!row_ok) return;
    if (p.splits > 1) {
        float *dst = p.part + (unit * p.M + (size_t)t * p.G + g) * (D + 2);
#pragma unroll
        for (int db = 0; db < NDB; db++)
#pragma unroll
            for (int e4 = 0; e4 < 4; e4++)
                *reinterpret_cast<f32x4 *>(dst + 32 * db + 8 * e4 + 4 * kg) =
                    (f32x4){o[db][4 * e4], o[db][4 * e4 + 1], o[db][4 * e4 + 2], o[db][4 * e4 + 3]};
        if (kg == 0) *reinterpret_cast<float2 *>(dst + D) = make_float2(m, l);
        return;
    }
    const float inv = 1.0f / l;
    uint16_t *orow = p.out + ((size_t)(tok0 + t) * p.Hq + h * p.G + g) * D;
#pragma unroll
    for (int db = 0; db < NDB; db++)
#pragma unroll
        for (int e4 = 0; e4 < 4; e4++) {
            const int d = 32 * db + 8 * e4 + 4 * kg;
            const uint32_t w0 = pack_bf16x2(o[db][4 * e4 + 0] * inv, o[db][4 * e4 + 1] * inv);
            const uint32_t w1 = pack_bf16x2(o[db][4 * e4 + 2] * inv, o[db][4 * e4 + 3] * inv);
            *reinterpret_cast<u32x2 *>(orow + d) = (u32x2){w0, w1};
        }
}

}  // namespace

// The ping-pong kernel takes dense bf16 caches with head_dim 128, power-of-two pages of at
// least 16 tokens and G dividing 256 (each work-group holds 256 packed rows).
bool ti_prefill_pp_eligible(const ti_attention_args *a, const ti_kv_cache *c) {
    const int G = a->q_heads / c->kv_heads;
    const int P = c->page_size;
    return c->kind == TI_KV_DENSE && a->dtype == TI_BF16 && c->head_dim == D && P >= 16 &&
           (P & (P - 1)) == 0 && ROWS % G == 0;
}

int ti_launch_prefill_pp(const ti_attention_args *a, const ti_kv_cache *c, const ti_prefill_plan &pl,
                         hipStream_t s) {
    PPParams p;
    p.q = (const uint16_t *)a->q;
    p.out = (uint16_t *)a->out;
    p.kp = (const uint16_t *)c->k_pages;
    p.vp = (const uint16_t *)c->v_pages;
    p.positions = a->positions;
    p.qsl = a->query_start_loc;
    p.bt = a->block_tables;
    p.bt_stride = a->block_table_stride;
    p.num_pages = c->num_pages;
    p.P = c->page_size;
    p.pshift = __builtin_ctz(c->page_size);
    p.Hk = c->kv_heads;
    p.Hq = a->q_heads;
    p.G = a->q_heads / c->kv_heads;
    p.nmax = a->max_query_len;
    p.causal = a->causal;
    p.scale_log2 = a->scale * LOG2E;
    p.part = (float *)a->workspace;
    p.splits = pl.splits;
    p.M = pl.rows;
    p.TQ = pl.TQ;
    p.qtiles = pl.qtiles;
    dim3 grid(c->kv_heads, p.qtiles * pl.splits, a->num_seqs);
    prefill_pp_kernel<<<grid, 64 * NW, 0, s>>>(p);
    if (hipGetLastError() != hipSuccess) return TI_ERR_LAUNCH;
    return pl.splits > 1 ? ti_launch_combine(a, c, pl.rows, pl.splits, s) : TI_OK;
}
