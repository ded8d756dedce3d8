// Float32 paged attention on the vector ALUs (no MFMA): the path for fp32 activations,
// whose tolerance (1e-4 abs against the double-accumulated oracle) rules out rounding the
// operands to bf16 for the matrix cores. It also accepts bf16 and INT8 caches, which makes
// it an independent cross-check of the MFMA kernels. Probabilities stay in Float32.
//
// Grid (max_query_len, Hq, B), one wave per (query token, query head): the keys of the
// step are walked 64 at a time, lane = key for QK^T (a full dot product per lane), then
// lane = head-dim element for PV with the probabilities broadcast through LDS.
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
    int bt_stride, num_pages, P, Hk, Hq, G, nmax, causal;
    float scale_log2;
};

template <typename T, bool INT8, int D>
__global__ void __launch_bounds__(64) generic_attention_kernel(GenericParams p) {
    using E = Elt<T>;
    const int t = blockIdx.x, hq = blockIdx.y, b = blockIdx.z, lane = threadIdx.x;
    const int tok0 = p.qsl ? p.qsl[b] : b * p.nmax;
    const int nb = p.qsl ? p.qsl[b + 1] - tok0 : p.nmax;
    if (t >= nb) return;
    const int start = p.positions[tok0], len = start + nb;
    const int last = p.causal ? start + t : len - 1;
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
    for (int c0 = 0; c0 <= last; c0 += WAVE) {
        const int key = c0 + lane;
        const bool valid = key <= last;
        float s = -INFINITY;
        long long row = 0;
        if (valid) {
            const int pg = page_of(bt, key / p.P, p.num_pages);
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
        const int cnt = min(WAVE, last + 1 - c0);
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
    dim3 grid(a->max_query_len, a->q_heads, a->num_seqs);
    const bool int8 = c->kind == TI_KV_INT8;
    if (a->dtype == TI_BF16) {
        if (int8) launch<uint16_t, true>(p, c->head_dim, grid, s);
        else launch<uint16_t, false>(p, c->head_dim, grid, s);
    } else {
        if (int8) launch<float, true>(p, c->head_dim, grid, s);
        else launch<float, false>(p, c->head_dim, grid, s);
    }
    return hipGetLastError() == hipSuccess ? TI_OK : TI_ERR_LAUNCH;
}
