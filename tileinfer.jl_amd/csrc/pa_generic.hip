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

template <typename T, bool INT8>
void launch(const GenericParams &p, int D, dim3 grid, hipStream_t s) {
    if (D == 128) generic_attention_kernel<T, INT8, 128><<<grid, 64, 0, s>>>(p);
    else generic_attention_kernel<T, INT8, 64><<<grid, 64, 0, s>>>(p);
}

}  // namespace

// Key splits for the fp32 path: while the waves (tokens x query heads x sequences) are
// fewer than about 1024, double the splits (at most 32). Host shapes only (graph-safe).
int ti_plan_generic(const ti_attention_args *a, const ti_kv_cache *c, size_t *bytes) {
    const long long waves = (long long)a->max_query_len * a->q_heads * a->num_seqs;
    int sp = 1;
    while (sp < 32 && waves * sp < 1024) sp <<= 1;
    const int rows = a->q_heads / c->kv_heads * a->max_query_len;
    *bytes = sp == 1 ? 0 : (size_t)a->num_seqs * c->kv_heads * sp * rows * (c->head_dim + 2) * sizeof(float);
    return sp;
}

int ti_launch_generic(const ti_attention_args *a, const ti_kv_cache *c, hipStream_t s) {
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
