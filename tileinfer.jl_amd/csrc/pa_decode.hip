#include <stdlib.h>

#include "pa_decode.hpp"

using namespace ti;
using namespace ti_decode;

namespace {

// Merge the splits of packed rows: grid (ceil(M / 4), Hk, B), four waves, one row per
// wave; lane owns head-dim elements lane + 64 k. The running maxima and sums are
// wave-uniform loads; the partial rows are read coalesced, with no LDS and no barrier.
template <int D, typename T, int SB>
__global__ void __launch_bounds__(256) combine_kernel(DecodeParams p) {
    constexpr int PER = D / 64;
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = blockIdx.y, b = blockIdx.z;
    // The partial loads wait only for what fixes their addresses: nothing beyond the
    // arguments, or the flat table's entry, loaded together with the sequence's token range
    // (query_start_loc); the row and token checks come before the store.
    const int rr = min(r, p.M - 1);
    int tok0 = b * p.nmax, tok1 = tok0 + p.nmax;
    int2 mt = make_int2(0, p.splits);
    if (p.qsl && p.flat) {
        tok0 = p.qsl[b];
        tok1 = p.qsl[b + 1];
        mt = *reinterpret_cast<const int2 *>(p.meta + 2 * b);
    } else if (p.qsl) {
        tok0 = p.qsl[b];
        tok1 = p.qsl[b + 1];
    } else if (p.flat) {
        mt = *reinterpret_cast<const int2 *>(p.meta + 2 * b);
    }
    const int t = r / p.G, g = r - t * p.G;
    const size_t stride = (size_t)p.M * (D + 2);
    // flat mode: the sequence's pieces are partial slots lo .. lo + n - 1 of the KV head; a
    // sequence of one piece (or none) had its output written by the decode kernel
    int splits = p.flat ? mt.y : p.splits;
    const size_t first = p.flat ? (size_t)h * p.flat + mt.x : ((size_t)b * p.Hk + h) * p.splits;
    if (!p.flat && p.min_tiles > 0) {
        // only the splits that held keys wrote partials; one alone wrote the output itself
        const int n = min(tok1 - tok0, p.nmax);   // an empty sequence reads no position
        const int len = n > 0 ? max(p.positions[tok0], 0) + n : 0;
        splits = f32_active_splits((len + 15) >> 4, p.splits, p.min_tiles).active;
    }
    const int last = max(splits, 1) - 1;   // loads stay inside the sequence's slots
    const float *base = p.part + first * stride + (size_t)rr * (D + 2);
    // Splits in batches of SB (2, 4, 8 or 16: the launch takes the smallest that holds all
    // splits): every load of a batch (m, l and the row) is issued before any arithmetic,
    // and batches merge online, so up to SB splits cost one round trip.
    float mx = NEG_BIG, lsum = 0.0f, acc[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) acc[k] = 0.0f;
    for (int sp0 = 0; sp0 < splits; sp0 += SB) {
        float2 ml[SB];
        float dv[SB][PER];
#pragma unroll
        for (int j = 0; j < SB; j++) {
            const float *src = base + min(sp0 + j, last) * stride;
            ml[j] = *reinterpret_cast<const float2 *>(src + D);
#pragma unroll
            for (int k = 0; k < PER; k++) dv[j][k] = src[lane + 64 * k];
        }
        float bm = mx;
#pragma unroll
        for (int j = 0; j < SB; j++)
            if (sp0 + j < splits) bm = fmaxf(bm, ml[j].x);
        const float alpha = fast_exp2(mx - bm);
        mx = bm;
        lsum *= alpha;
#pragma unroll
        for (int k = 0; k < PER; k++) acc[k] *= alpha;
#pragma unroll
        for (int j = 0; j < SB; j++) {
            const float wgt = sp0 + j < splits ? fast_exp2(ml[j].x - mx) : 0.0f;
            lsum += ml[j].y * wgt;
#pragma unroll
            for (int k = 0; k < PER; k++) acc[k] += dv[j][k] * wgt;
        }
    }
    const int nb = min(tok1 - tok0, p.nmax);   // at most max_query_len
    if (r >= p.M || t >= nb || splits <= 1) return;
    const float inv = 1.0f / lsum;
    T *o = reinterpret_cast<T *>(p.out) + ((size_t)(tok0 + t) * p.Hq + h * p.G + g) * D;
#pragma unroll
    for (int k = 0; k < PER; k++) Elt<T>::st(o, lane + 64 * k, acc[k] * inv);
}

template <int D, typename T>
void launch_combine_sb(const DecodeParams &p, int sb, dim3 grid, hipStream_t s) {
    switch (sb) {
        case 2: combine_kernel<D, T, 2><<<grid, 256, 0, s>>>(p); break;
        case 4: combine_kernel<D, T, 4><<<grid, 256, 0, s>>>(p); break;
        case 8: combine_kernel<D, T, 8><<<grid, 256, 0, s>>>(p); break;
        default: combine_kernel<D, T, 16><<<grid, 256, 0, s>>>(p); break;
    }
}

template <int D, bool INT8, bool PG16, int NW>
void launch_decode_d(const DecodeParams &p, int rowb, dim3 grid, hipStream_t s) {
    // 8-wave groups only for up to 32 packed rows (their merge slabs must fit the LDS).
    // 33-64 rows: 4-wave groups of two wave pairs, each pair splitting the rows over the
    // same keys (32 rows per wave keeps the accumulators in VGPRs at 2 waves per SIMD).
    switch (rowb) {
        case 1: decode_kernel<D, 1, INT8, PG16, NW, 1><<<grid, NW * 64, 0, s>>>(p); break;
        case 2: decode_kernel<D, 2, INT8, PG16, NW, 1><<<grid, NW * 64, 0, s>>>(p); break;
        default: decode_kernel<D, 2, INT8, PG16, 4, 2><<<grid, 256, 0, s>>>(p); break;
    }
}

template <int D, bool INT8>
void launch_decode_p(const DecodeParams &p, int rowb, int waves, dim3 grid, hipStream_t s) {
    if (p.P % 16 == 0 && p.pshift >= 0) {
        if (waves == 8) launch_decode_d<D, INT8, true, 8>(p, rowb, grid, s);
        else launch_decode_d<D, INT8, true, 4>(p, rowb, grid, s);
    } else {
        if (waves == 8) launch_decode_d<D, INT8, false, 8>(p, rowb, grid, s);
        else launch_decode_d<D, INT8, false, 4>(p, rowb, grid, s);
    }
}

}  // namespace

// Work-groups per (sequence, KV head) and waves per group. Large batches take one split of
// 4 waves per (sequence, KV head), which writes the output directly (no partials, no
// combine launch); smaller ones split the keys into a power of two of 4-wave groups (at
// most 16, about 8 waves per CU over the 256 CUs) merged by the combine kernel. Depends only
// on host shapes, never on context length, so a captured graph stays valid.
ti_decode_plan ti_plan_decode(const ti_attention_args *a, const ti_kv_cache *c) {
    ti_decode_plan pl;
    const int G = a->q_heads / c->kv_heads;
    pl.rows = G * a->max_query_len;
    const long long pairs = (long long)a->num_seqs * c->kv_heads;
    // Split target: 256 work-groups of 4 waves, one wave per SIMD (B = 8: 4 splits against
    // 8, same box: INT8 x 32768 101.6 vs 102.9 us, bf16 x 4096 29.4 vs 30.0 us).
    constexpr long long target = 256;
    // At most 16 splits: at B = 1 (8 KV heads) 16 splits beat 32 at every context
    // measured (1024 positions 7.7 vs 8.8 us, 2048 8.6 vs 9.9, 4096 11.0 vs 11.5): fewer
    // idle waves on short contexts and half the partials to merge.
    constexpr int max_splits = 16;
    // Batches of at least 256 (sequence, KV head) pairs: one split of 4 waves per pair, one
    // wave per SIMD (measured against 8 waves, same process: B = 32 x 4096 91.1 vs 91.8 us,
    // ragged B = 32 132.0 vs 133.9 us; two tiles per step or three register sets in flight
    // per wave made no difference).
    int sp = 1, nw = 4;
    if (pairs < 256 || pl.rows > 32) {
        while (sp < max_splits && pairs * sp < target) sp <<= 1;
    }
    // Split batches of 4-64 sequences with at least 4 splits each share their work-groups out
    // by length (flat mode): the same B x splits work-groups per KV head, cut in proportion
    // to each sequence's keys. Measured on
    // lengths drawn from [1024, 8192] against the fixed splits (separate processes, same
    // box): B = 8 (4 splits) 31.0 -> 27.5 us, B = 4 (8 splits) 21.3 vs 21.3 us, but B = 2
    // (16 splits) 16.0 -> 16.9 us and B = 16 (2 splits) 60.8 -> 63.0 us, where the shares
    // balance little and the device-side prefix costs its latency.
    pl.flat = sp >= 4 && a->num_seqs >= 4 && a->num_seqs <= 64 ? sp * a->num_seqs : 0;
    pl.splits = sp;
    pl.waves = nw;
    pl.bytes = sp == 1 ? 0 : (size_t)pairs * sp * pl.rows * (c->head_dim + 2) * sizeof(float);
    pl.meta = pl.bytes;   // per-sequence {first work-group, pieces} after the partials
    if (pl.flat) pl.bytes += (size_t)a->num_seqs * 2 * sizeof(int);
    return pl;
}

int ti_launch_decode(const ti_attention_args *a, const ti_kv_cache *c, const ti_decode_plan &pl,
                     hipStream_t s) {
    DecodeParams p;
    p.q = (const uint16_t *)a->q;
    p.out = (uint16_t *)a->out;
    p.kp = (const uint16_t *)c->k_pages;
    p.vp = (const uint16_t *)c->v_pages;
    p.lq = c->layer_q;
    p.ls = c->layer_scale;
    p.smooth = c->smooth;
    p.positions = a->positions;
    p.qsl = a->query_start_loc;
    p.bt = a->block_tables;
    p.part = (float *)a->workspace;
    p.meta = pl.flat ? reinterpret_cast<int *>((char *)a->workspace + pl.meta) : nullptr;
    p.B = a->num_seqs;
    p.flat = pl.flat;
    p.bt_stride = a->block_table_stride;
    p.num_pages = c->num_pages;
    p.P = c->page_size;
    p.pshift = (c->page_size & (c->page_size - 1)) == 0 ? __builtin_ctz(c->page_size) : -1;
    p.Hk = c->kv_heads;
    p.Hq = a->q_heads;
    p.G = a->q_heads / c->kv_heads;
    p.nmax = a->max_query_len;
    p.M = pl.rows;
    p.splits = pl.splits;
    p.causal = a->causal;
    p.scale_log2 = a->scale * LOG2E;
    const int rowb = (pl.rows + 15) / 16;
    const dim3 grid = pl.flat ? dim3(pl.flat, c->kv_heads, 1) : dim3(pl.splits, c->kv_heads, a->num_seqs);
    const bool int8 = c->kind == TI_KV_INT8;
    if (c->head_dim == 128) {
        if (int8) launch_decode_p<128, true>(p, rowb, pl.waves, grid, s);
        else launch_decode_p<128, false>(p, rowb, pl.waves, grid, s);
    } else {
        if (int8) launch_decode_p<64, true>(p, rowb, pl.waves, grid, s);
        else launch_decode_p<64, false>(p, rowb, pl.waves, grid, s);
    }
    if (hipGetLastError() != hipSuccess) return TI_ERR_LAUNCH;
    if (pl.splits == 1) return TI_OK;
    // the combine batches its loads by the mean pieces per sequence
    return ti_launch_combine(a, c, pl.rows, pl.flat ? pl.flat / a->num_seqs : pl.splits, s, pl.flat, p.meta);
}

int ti_launch_combine(const ti_attention_args *a, const ti_kv_cache *c, int rows, int splits,
                      hipStream_t s, int flat, int *meta, int min_tiles) {
    DecodeParams p{};
    p.min_tiles = min_tiles;
    p.positions = a->positions;
    p.out = (uint16_t *)a->out;
    p.part = (float *)a->workspace;
    p.flat = flat;
    p.meta = meta;
    p.qsl = a->query_start_loc;
    p.Hk = c->kv_heads;
    p.Hq = a->q_heads;
    p.G = a->q_heads / c->kv_heads;
    p.nmax = a->max_query_len;
    p.M = rows;
    p.splits = splits;
    dim3 cgrid((rows + 3) / 4, c->kv_heads, a->num_seqs);
    const bool f32 = a->dtype == TI_F32;
    const int sb = splits <= 2 ? 2 : (splits <= 4 ? 4 : (splits <= 8 ? 8 : 16));
    if (c->head_dim == 128) {
        if (f32) launch_combine_sb<128, float>(p, sb, cgrid, s);
        else launch_combine_sb<128, uint16_t>(p, sb, cgrid, s);
    } else {
        if (f32) launch_combine_sb<64, float>(p, sb, cgrid, s);
        else launch_combine_sb<64, uint16_t>(p, sb, cgrid, s);
    }
    return hipGetLastError() == hipSuccess ? TI_OK : TI_ERR_LAUNCH;
}
