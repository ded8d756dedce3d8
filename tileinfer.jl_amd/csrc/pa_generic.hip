// Float32 paged attention on the vector ALUs (no MFMA): the path for fp32 activations,
// whose tolerance (1e-4 abs against the double-accumulated oracle) rules out rounding the
// operands to bf16 for the matrix cores. It also accepts bf16 and INT8 caches, which makes
// it an independent cross-check of the MFMA kernels. Probabilities stay in Float32.
//
// Grid (max_query_len x splits, Hq, B), one wave per (query token, query head, key split):
// the split's keys are walked 64 at a time, lane = key for QK^T (a full dot product per
// lane), then lane = head-dim element for PV with the probabilities broadcast through LDS.
// With one split the wave writes the output row; otherwise it writes a Float32 partial
// (acc[D], m, l) in the decode kernel's layout (packed row g + G t of its KV head) and the
// combine kernel merges the splits.
// Semantics as attention(::RefBackend) (src/ops/reference.jl:95-121): key i visible to
// query t iff i <= start + t (causal) or i < start + n (not causal).
#include "common.hpp"

using namespace ti;

namespace {

struct GenericParams {
    const void *q;
    void *out;
    const void *kp, *vp;
    const int8_t *lq;
    const float *ls, *smooth;
    const int32_t *positions, *qsl, *bt;
    float *part;                 // split partials [B][Hk][splits][G nmax][D + 2]
    int bt_stride, num_pages, P, Hk, Hq, G, nmax, causal, splits;
    float scale_log2;
};

template <typename T, bool INT8, int D>
__global__ void __launch_bounds__(64) generic_attention_kernel(GenericParams p) {
    using E = Elt<T>;
    const int t = blockIdx.x / p.splits, split = blockIdx.x % p.splits;
    const int hq = blockIdx.y, b = blockIdx.z, lane = threadIdx.x;
    const int tok0 = p.qsl ? p.qsl[b] : b * p.nmax;
    const int nb = p.qsl ? min(p.qsl[b + 1] - tok0, p.nmax) : p.nmax;   // at most max_query_len
    if (t >= nb) return;
    const int start = max(p.positions[tok0], 0), len = start + nb;   // a negative position reads as 0
    const int last = p.causal ? start + t : len - 1;
    // this split's keys: [k0, k1) of the sequence's len, cut at the query's last key
    const int per = (len + p.splits - 1) / p.splits;
    const int k0 = split * per, k1 = min(k0 + per, last + 1);
    const int g = hq / p.G;
    const int32_t *bt = p.bt + (size_t)b * p.bt_stride;
    const size_t half_q = (size_t)p.num_pages * p.Hk * p.P * D;
    const size_t half_s = (size_t)p.num_pages * p.Hk * p.P;

    __shared__ float qs[D];
    __shared__ float ps[WAVE];
    __shared__ long long rows[WAVE];
    const T *q = (const T *)p.q + ((size_t)(tok0 + t) * p.Hq + hq) * D;
    for (int d = lane; d < D; d += WAVE) qs[d] = E::ld(q, d);
    __syncthreads();

    constexpr int PER = (D + WAVE - 1) / WAVE;
    float acc[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) acc[j] = 0.0f;
    float m = NEG_BIG, l = 0.0f;
    for (int c0 = k0; c0 < k1; c0 += WAVE) {
        const int key = c0 + lane;
        const bool valid = key < k1;
        float s = -INFINITY;
        long long row = 0;
        if (valid) {
            const int pg = page_of(bt, key / p.P, p.bt_stride, p.num_pages);
            row = ((long long)pg * p.Hk + g) * p.P + key % p.P;
            float dot = 0.0f;
            if (INT8) {
                const int8_t *kr = p.lq + row * D;
                const float sk = p.ls[row];
                for (int d = 0; d < D; d++) dot += ((float)kr[d] * sk) * p.smooth[d] * qs[d];
            } else {
                const T *kr = (const T *)p.kp + row * D;
                for (int d = 0; d < D; d++) dot += E::ld(kr, d) * qs[d];
            }
            s = dot * p.scale_log2;
        }
        const float m_new = fmaxf(m, wave_max(s));
        const float alpha = fast_exp2(m - m_new);
        const float pr = valid ? fast_exp2(s - m_new) : 0.0f;
        l = l * alpha + wave_sum(pr);
        m = m_new;
        ps[lane] = pr;
        rows[lane] = row;
        __syncthreads();
        const int cnt = min(WAVE, k1 - c0);
#pragma unroll
        for (int j = 0; j < PER; j++) acc[j] *= alpha;
        for (int kk = 0; kk < cnt; kk++) {
            const float pk = ps[kk];
            const long long r = rows[kk];
#pragma unroll
            for (int j = 0; j < PER; j++) {
                const int d = lane + WAVE * j;
                if (d < D) {
                    const float v = INT8 ? (float)p.lq[half_q + r * D + d] * p.ls[half_s + r]
                                         : E::ld((const T *)p.vp + r * D, d);
                    acc[j] += pk * v;
                }
            }
        }
        __syncthreads();
    }
    if (p.splits > 1) {
        // (acc, m, l) of packed row (hq mod G) + G t of KV head g; a split without keys
        // leaves m = NEG_BIG, l = 0, acc = 0, which the combine weights to zero.
        const int M = p.G * p.nmax, r = (hq - g * p.G) + p.G * t;
        float *dst = p.part + ((((size_t)b * p.Hk + g) * p.splits + split) * M + r) * (D + 2);
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int d = lane + WAVE * j;
            if (d < D) dst[d] = acc[j];
        }
        if (lane == 0) {
            dst[D] = m;
            dst[D + 1] = l;
        }
        return;
    }
    T *o = (T *)p.out + ((size_t)(tok0 + t) * p.Hq + hq) * D;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int d = lane + WAVE * j;
        if (d < D) E::st(o, d, acc[j] / l);
    }
}

// Float32 attention on the fp32 matrix cores (v_mfma_f32_16x16x4_f32: fp32 products and
// sums, within the fp32 path's 1e-4 tolerance), for dense fp32 pools with 16-key tiles in one
// page (P a power of two >= 16) and D = 64 or 128: decode, prefill and multi-token steps.
// Packed query rows g + G t (as the bf16 kernels) form q-tiles of 16 rows. Work-group = (key
// split, q-tile, KV head, sequence); its keys end after the q-tile's last token (causal), and
// four waves take every fourth 16-key tile of the split. Per tile and wave (lane l: row r16 =
// l % 16 of the q-tile, k-group kg = l / 16):
//   S^T = K Q^T     D/4 MFMAs; MFMA (j, c) sums head-dim elements 16 j + 4 kg' + c over kg'
//                   (lane: key r16's and row r16's element 16 j + 4 kg + c, from float4 loads);
//                   the lane gets its row's scores of keys 4 kg + e.
//   softmax         exp2 domain, lane-local per row (two xor shuffles for a row max; lazy
//                   rescale as the bf16 kernel).
//   O^T += V^T P^T  4 D/16 MFMAs; MFMA (e, db): A = V[key 4 kg + e][16 db + r16] (a
//                   coalesced row read), B = the lane's probability of key 4 kg + e.
// The waves merge through LDS; one split writes the output, more write Float32 partials in
// the decode kernel's layout for the combine kernel.
struct F32Params {
    const float *q;
    float *out;
    const float *kp, *vp;
    const int32_t *positions, *qsl, *bt;
    float *part;
    int bt_stride, num_pages, P, pshift, Hk, Hq, G, nmax, M, splits, causal;
    int B, qtiles;   // sequences; 16-row q-tiles per (sequence, KV head)
    int sshift;      // log2(splits)
    int xcd;         // 1-D grid, work-groups of one (sequence, KV head) on one XCD (pairs % 8 == 0)
    float scale_log2;
};

// Each split takes at least this many 16-key tiles (one per wave), so short contexts run on
// fewer work-groups than the launch holds.
constexpr int F32_MIN_TILES = 4;

template <int D, bool QT>   // QT: more than one q-tile per (sequence, KV head)
__global__ void __launch_bounds__(256) attn_f32_kernel(F32Params p) {
    constexpr int NJ = D / 16, NDB = D / 16, NW = 4, MROW = D + 4;
    __shared__ __attribute__((aligned(16))) float slab[NW * 16 * MROW];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, kg = lane >> 4;
    // Work item: key split s, q-tile qt, KV head h, sequence b. Grid (splits x q-tiles, Hk, B),
    // or with xcd a 1-D grid: work-groups are dealt to the 8 XCDs round-robin by index, so
    // the items of one (sequence, KV head) pair take indices that share their residue mod 8,
    // run on one XCD and read the pair's keys and values through one L2.
    int item, h, b;
    if (QT && p.xcd) {
        const int QX = p.splits * p.qtiles, k = blockIdx.x >> 3;
        const int pair = (int)(blockIdx.x & 7) + 8 * (k / QX);
        item = k % QX;
        h = pair % p.Hk;
        b = pair / p.Hk;
    } else {
        item = blockIdx.x;
        h = blockIdx.y;
        b = blockIdx.z;
    }
    // q-tiles in fold order (the heavier causal half descending, then the lighter half
    // ascending): work-groups dispatched half a round apart, which tend to share a CU, then
    // pair a heavy and a light q-tile (a placement hint only; any order is correct)
    const int s = QT ? item & (p.splits - 1) : item;
    int qt = 0;
    if (QT) {
        const int u = item >> p.sshift, half = (p.qtiles + 1) >> 1;
        qt = u < half ? p.qtiles - 1 - u : u - half;
    }
    const int tok0 = p.qsl ? p.qsl[b] : b * p.nmax;
    const int nb = p.qsl ? min(p.qsl[b + 1] - tok0, p.nmax) : p.nmax;   // at most max_query_len
    const int t_first = QT ? 16 * qt / p.G : 0;
    if (t_first >= nb) return;   // the q-tile holds no token of this sequence
    const int start = max(p.positions[tok0], 0), len = start + nb;   // a negative position reads as 0
    // splits cut the sequence's 16-key tiles (the combine derives the same count); this
    // q-tile's keys end after its last token's position
    const ActiveSplits as = f32_active_splits((len + 15) >> 4, p.splits, F32_MIN_TILES);
    if (s >= as.active) return;   // no keys for this split
    const int t_last = QT ? min((16 * qt + 15) / p.G, nb - 1) : nb - 1;
    const int kend = p.causal ? start + t_last + 1 : len;
    const int j0 = s * as.per, j1 = min(j0 + as.per, (kend + 15) >> 4);   // may be empty: (m, l) = (NEG_BIG, 0)
    const int r = 16 * qt + r16, t = r / p.G, g = r - t * p.G;
    const bool ok = r < p.M && t < nb;
    const int qpos = p.causal && ok ? start + t : len - 1;
    const int mask_from = p.causal ? start + t_first : len - 1;   // keys up to here are visible to every row
    f32x4 qv[NJ];
    {
        const float *qr = p.q + ((size_t)(tok0 + (ok ? t : 0)) * p.Hq + h * p.G + g) * D + 4 * kg;
#pragma unroll
        for (int j = 0; j < NJ; j++)
            qv[j] = ok ? *reinterpret_cast<const f32x4 *>(qr + 16 * j) : (f32x4){0.f, 0.f, 0.f, 0.f};
    }
    f32x4 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; db++) o[db] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m = NEG_BIG, l = 0.0f;
    const int32_t *bt = p.bt + (size_t)b * p.bt_stride;
    struct Tile {
        f32x4 k[NJ];
        float v[4][NDB];
    };
    auto load = [&](int j, Tile &tl) {
        const int pos0 = j * 16, last = len - 1 - pos0;   // keys past len read the last key's row
        const int pg = page_of_s(bt, pos0 >> p.pshift, p.bt_stride, p.num_pages);
        const long long rbase = ((long long)pg * p.Hk + h) * p.P + (pos0 & (p.P - 1));
        const float *krow = p.kp + (rbase + min(r16, last)) * D + 4 * kg;
#pragma unroll
        for (int jj = 0; jj < NJ; jj++) tl.k[jj] = *reinterpret_cast<const f32x4 *>(krow + 16 * jj);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float *vrow = p.vp + (rbase + min(4 * kg + e, last)) * D + r16;
#pragma unroll
            for (int db = 0; db < NDB; db++) tl.v[e][db] = vrow[16 * db];
        }
    };
    auto compute = [&](int j, const Tile &tl) {
        const int pos0 = j * 16;
        f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jj = 0; jj < NJ; jj++)
#pragma unroll
            for (int c = 0; c < 4; c++) sc = __builtin_amdgcn_mfma_f32_16x16x4f32(tl.k[jj][c], qv[jj][c], sc, 0, 0, 0);
        const bool need_mask = pos0 + 15 > mask_from;
        float x[4], mt = -INFINITY;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int kpos = pos0 + 4 * kg + e;
            x[e] = need_mask && kpos > qpos ? -INFINITY : sc[e];
            mt = fmaxf(mt, x[e]);
        }
        mt *= p.scale_log2;
        if (__any(mt > m + 8.0f)) {
            mt = fmaxf(mt, __shfl_xor(mt, 16));
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float mn = fmaxf(m, mt);
            const float alpha = fast_exp2(m - mn);
            m = mn;
            l *= alpha;
#pragma unroll
            for (int db = 0; db < NDB; db++) o[db] *= alpha;
        }
        float pe[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            pe[e] = fast_exp2(__builtin_fmaf(x[e], p.scale_log2, -m));
            l += pe[e];
        }
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
            for (int db = 0; db < NDB; db++) o[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(tl.v[e][db], pe[e], o[db], 0, 0, 0);
    };
    if constexpr (QT) {
        // multi-token q-tiles walk many tiles per wave: the next tile's loads are issued
        // before this one's arithmetic (two register sets; past the last tile the prefetch
        // re-reads it, unused)
        Tile ta, tb;
        int j = j0 + w;
        if (j < j1) {
            load(j, ta);
            while (true) {
                load(min(j + NW, j1 - 1), tb);
                compute(j, ta);
                j += NW;
                if (j >= j1) break;
                load(min(j + NW, j1 - 1), ta);
                compute(j, tb);
                j += NW;
                if (j >= j1) break;
            }
        }
    } else {
        for (int j = j0 + w; j < j1; j += NW) {
            Tile tl;
            load(j, tl);
            compute(j, tl);
        }
    }
    // merge the four waves' states (same rows, disjoint keys) through LDS
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    {
        float *my = slab + ((size_t)w * 16 + r16) * MROW;
#pragma unroll
        for (int db = 0; db < NDB; db++) *reinterpret_cast<f32x4 *>(my + 16 * db + 4 * kg) = o[db];
        if (kg == 0) {
            my[D] = m;
            my[D + 1] = l;
        }
    }
    __syncthreads();
    const size_t unit = ((size_t)b * p.Hk + h) * p.splits + s;
    const int mrows = QT ? 16 : p.M;   // one q-tile: the M <= 16 rows
    for (int it = threadIdx.x; it < mrows * (D / 4); it += NW * 64) {
        const int rr = it / (D / 4), d4 = (it % (D / 4)) * 4, r = 16 * qt + rr;
        if (r >= p.M) continue;
        float mx = NEG_BIG;
#pragma unroll
        for (int wi = 0; wi < NW; wi++) mx = fmaxf(mx, slab[((size_t)wi * 16 + rr) * MROW + D]);
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        float lsum = 0.0f;
#pragma unroll
        for (int wi = 0; wi < NW; wi++) {
            const float *src = slab + ((size_t)wi * 16 + rr) * MROW;
            const float wgt = fast_exp2(src[D] - mx);
            lsum += src[D + 1] * wgt;
            acc += *reinterpret_cast<const f32x4 *>(src + d4) * wgt;
        }
        const int tr = r / p.G, gr = r - tr * p.G;
        if (tr >= nb) continue;
        if (as.active == 1) {
            const float inv = 1.0f / lsum;
            *reinterpret_cast<f32x4 *>(p.out + ((size_t)(tok0 + tr) * p.Hq + h * p.G + gr) * D + d4) = acc * inv;
        } else {
            float *dst = p.part + (unit * (size_t)p.M + r) * (D + 2);
#pragma unroll
            for (int e = 0; e < 4; e++) dst[d4 + e] = acc[e];
            if (d4 == 0) {
                dst[D] = mx;
                dst[D + 1] = lsum;
            }
        }
    }
}

template <typename T, bool INT8>
void launch(const GenericParams &p, int D, dim3 grid, hipStream_t s) {
    if (D == 128) generic_attention_kernel<T, INT8, 128><<<grid, 64, 0, s>>>(p);
    else generic_attention_kernel<T, INT8, 64><<<grid, 64, 0, s>>>(p);
}

}  // namespace

// fp32 steps that the matrix-core kernel takes: dense fp32 pools, pages of 2^k >= 16 tokens,
// D = 64 or 128. Its key splits: while the (sequence, KV head, q-tile) items times splits are
// fewer than F32_TARGET work-groups, double (at most 32); short contexts then use fewer of
// them (F32_MIN_TILES).
constexpr int F32_TARGET = 512, F32_MAX_SPLITS = 32;
static bool f32_mfma(const ti_attention_args *a, const ti_kv_cache *c) {
    return a->dtype == TI_F32 && c->kind == TI_KV_DENSE && (c->head_dim == 64 || c->head_dim == 128) &&
           c->page_size >= 16 && (c->page_size & (c->page_size - 1)) == 0;
}
static int f32_qtiles(const ti_attention_args *a, const ti_kv_cache *c) {
    return (a->q_heads / c->kv_heads * a->max_query_len + 15) / 16;
}
static int f32_splits(const ti_attention_args *a, const ti_kv_cache *c) {
    const long long items = (long long)a->num_seqs * c->kv_heads * f32_qtiles(a, c);
    int sp = 1;
    while (sp < F32_MAX_SPLITS && items * sp < F32_TARGET) sp <<= 1;
    return sp;
}

// Key splits for the fp32 path: while the waves (tokens x query heads x sequences) are
// fewer than about 1024, double the splits (at most 32). Host shapes only (graph-safe).
int ti_plan_generic(const ti_attention_args *a, const ti_kv_cache *c, size_t *bytes) {
    if (f32_mfma(a, c)) {
        const int sp = f32_splits(a, c);
        const int rows = a->q_heads / c->kv_heads * a->max_query_len;
        *bytes = sp == 1 ? 0 : (size_t)a->num_seqs * c->kv_heads * sp * rows * (c->head_dim + 2) * sizeof(float);
        return sp;
    }
    const long long waves = (long long)a->max_query_len * a->q_heads * a->num_seqs;
    int sp = 1;
    while (sp < 32 && waves * sp < 1024) sp <<= 1;
    const int rows = a->q_heads / c->kv_heads * a->max_query_len;
    *bytes = sp == 1 ? 0 : (size_t)a->num_seqs * c->kv_heads * sp * rows * (c->head_dim + 2) * sizeof(float);
    return sp;
}

int ti_launch_generic(const ti_attention_args *a, const ti_kv_cache *c, hipStream_t s) {
    if (f32_mfma(a, c)) {
        F32Params f;
        f.q = (const float *)a->q;
        f.out = (float *)a->out;
        f.kp = (const float *)c->k_pages;
        f.vp = (const float *)c->v_pages;
        f.positions = a->positions;
        f.qsl = a->query_start_loc;
        f.bt = a->block_tables;
        f.bt_stride = a->block_table_stride;
        f.num_pages = c->num_pages;
        f.P = c->page_size;
        f.pshift = __builtin_ctz(c->page_size);
        f.Hk = c->kv_heads;
        f.Hq = a->q_heads;
        f.G = a->q_heads / c->kv_heads;
        f.nmax = a->max_query_len;
        f.M = f.G * a->max_query_len;
        f.causal = a->causal;
        f.scale_log2 = a->scale * LOG2E;
        size_t bytes = 0;
        f.splits = ti_plan_generic(a, c, &bytes);
        if (bytes > 0 && (!a->workspace || a->workspace_bytes < bytes)) f.splits = 1;   // runs unsplit
        f.part = (float *)a->workspace;
        f.B = a->num_seqs;
        f.qtiles = f32_qtiles(a, c);
        const long long pairs = (long long)a->num_seqs * c->kv_heads;
        const long long wgs = pairs * f.qtiles * f.splits;
        if (wgs > 0x7fffffffLL) return TI_ERR_UNSUPPORTED;
        f.sshift = __builtin_ctz(f.splits);
        f.xcd = pairs % 8 == 0 && f.qtiles > 1;   // decode (one q-tile) reuses no tile across work-groups
        const dim3 grid = f.xcd ? dim3((unsigned)wgs) : dim3((unsigned)(f.splits * f.qtiles), c->kv_heads, a->num_seqs);
        if (f.qtiles > 1) {
            if (c->head_dim == 128) attn_f32_kernel<128, true><<<grid, 256, 0, s>>>(f);
            else attn_f32_kernel<64, true><<<grid, 256, 0, s>>>(f);
        } else {
            if (c->head_dim == 128) attn_f32_kernel<128, false><<<grid, 256, 0, s>>>(f);
            else attn_f32_kernel<64, false><<<grid, 256, 0, s>>>(f);
        }
        if (hipGetLastError() != hipSuccess) return TI_ERR_LAUNCH;
        return f.splits > 1 ? ti_launch_combine(a, c, f.M, f.splits, s, 0, nullptr, F32_MIN_TILES) : TI_OK;
    }
    GenericParams p;
    p.q = a->q;
    p.out = a->out;
    p.kp = c->k_pages;
    p.vp = c->v_pages;
    p.lq = c->layer_q;
    p.ls = c->layer_scale;
    p.smooth = c->smooth;
    p.positions = a->positions;
    p.qsl = a->query_start_loc;
    p.bt = a->block_tables;
    p.bt_stride = a->block_table_stride;
    p.num_pages = c->num_pages;
    p.P = c->page_size;
    p.Hk = c->kv_heads;
    p.Hq = a->q_heads;
    p.G = a->q_heads / c->kv_heads;
    p.nmax = a->max_query_len;
    p.causal = a->causal;
    p.scale_log2 = a->scale * LOG2E;
    size_t bytes = 0;
    p.splits = ti_plan_generic(a, c, &bytes);
    if (bytes > 0 && (!a->workspace || a->workspace_bytes < bytes)) p.splits = 1;   // runs unsplit
    p.part = (float *)a->workspace;
    dim3 grid(a->max_query_len * p.splits, a->q_heads, a->num_seqs);
    const bool int8 = c->kind == TI_KV_INT8;
    if (a->dtype == TI_BF16) {
        if (int8) launch<uint16_t, true>(p, c->head_dim, grid, s);
        else launch<uint16_t, false>(p, c->head_dim, grid, s);
    } else {
        if (int8) launch<float, true>(p, c->head_dim, grid, s);
        else launch<float, false>(p, c->head_dim, grid, s);
    }
    if (hipGetLastError() != hipSuccess) return TI_ERR_LAUNCH;
    return p.splits > 1 ? ti_launch_combine(a, c, a->q_heads / c->kv_heads * a->max_query_len, p.splits, s)
                        : TI_OK;
}
