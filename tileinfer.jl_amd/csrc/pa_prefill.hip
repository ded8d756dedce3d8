// Paged causal / chunked / non-causal prefill attention on bf16 MFMA (gfx950), dense bf16
// or INT8 cache.
//
// Reference: attention_prefill_kernel / prefill_body (src/ops/tile/attention.jl:130-177)
// and attention_prefill_int8_kernel (:139-147). Query t of the step sits at position
// start + t (start = positions of the sequence's first query, read on the device) and sees
// keys 0 .. start + t; with causal = 0 it sees all start + n keys (attention.jl:155-157).
// Chunked prefill over a cached prefix is the same kernel with start > 0.
//
// Work decomposition. A work-group (4 waves, 256 threads) owns 64 packed query rows of
// one (sequence, KV head): the G query heads of the KV head times TQ = 64 / G consecutive
// query positions, row r = g + G t as in the decode kernel, so every K/V tile loaded into
// LDS serves all G heads. Query tiles are issued heaviest first (the last positions see
// the most keys). Keys stream through LDS in 32-key tiles, double-buffered: global loads
// of tile j+1 are in flight while the waves compute tile j. K is kept row-major (the A
// operand of S^T = K Q^T), V transposed (the A operand of O^T = V^T P^T).
//
// Per wave (16 rows) and 32-key tile:
//   S^T = K Q^T        2 x (D/32) v_mfma_f32_16x16x32_bf16 (two 16-key blocks)
//   online softmax     exp2 domain, lane-local per row + two xor shuffles for the max
//   O^T += V^T P^T     D/16 v_mfma_f32_16x16x32_bf16; P^T is the S^T registers of both
//                      key blocks rounded to bf16 (k slots: keys 4k..4k+3 and 16+4k..+3),
//                      V^T read with the same key order.
// INT8: keys and values enter LDS converted to bf16 (exact), their scales beside them; a
// key's scale multiplies its scores, a value's scale its probability; queries are
// multiplied by the keys' smoothing and rounded to bf16 (attention.jl:68-95).
#include "common.hpp"

using namespace ti;

namespace {

struct PrefillParams {
    const uint16_t *q;
    uint16_t *out;
    const uint16_t *kp, *vp;
    const int8_t *lq;
    const float *ls, *smooth;
    const int32_t *positions, *qsl, *bt;
    int bt_stride, num_pages, P, Hk, Hq, G, TQ, nmax, qtiles, causal;
    float scale_log2;
};

constexpr int KT = 32;  // keys per LDS tile

template <int D>
struct Smem {
    static constexpr int KROW = D + 8;   // padded K row (uint16)
    static constexpr int VROW = KT + 4;  // padded V^T row (uint16)
    uint16_t k[2][KT * KROW];
    uint16_t vt[2][D * VROW];
    float sk[2][KT], sv[2][KT];
};

// Registers holding one key tile between its global load and its LDS store.
template <int D, bool INT8>
struct Stage {
    static constexpr int KCH = KT * D / 8;                    // 16 B (8-element) K chunks
    static constexpr int KPT = (KCH + 255) / 256;             // K chunks per thread
    uint4 k[KPT];          // bf16 K chunks (INT8: 8 bytes in .x/.y)
    uint4 v[2];            // two V rows' chunk (key pair)
    float s;               // a key or value scale (INT8)
};

__device__ __forceinline__ uint4 i8x8_to_bf16x8(uint2 v) {
    uint4 r;
    i8x4_to_bf16(v.x, r.x, r.y);
    i8x4_to_bf16(v.y, r.z, r.w);
    return r;
}

template <int D, bool INT8>
__device__ __forceinline__ long long key_row(const PrefillParams &p, const int32_t *bt, int h,
                                             int pos) {
    const int pg = page_of(bt, pos / p.P, p.num_pages);
    return ((long long)pg * p.Hk + h) * p.P + pos % p.P;
}

template <int D, bool INT8>
__device__ __forceinline__ void load_tile(Stage<D, INT8> &st, const PrefillParams &p,
                                          const int32_t *bt, int h, int kt, int kend) {
    const int tid = threadIdx.x;
    const size_t half_q = (size_t)p.num_pages * p.Hk * p.P * D;
    const size_t half_s = (size_t)p.num_pages * p.Hk * p.P;
    constexpr int CPR = D / 8;
#pragma unroll
    for (int u = 0; u < Stage<D, INT8>::KPT; u++) {
        const int c = tid + 256 * u, key = c / CPR, ch = c % CPR, pos = kt * KT + key;
        st.k[u] = make_uint4(0, 0, 0, 0);
        if (c < Stage<D, INT8>::KCH && pos < kend) {
            const long long row = key_row<D, INT8>(p, bt, h, pos);
            if (!INT8) {
                st.k[u] = *reinterpret_cast<const uint4 *>(p.kp + row * D + ch * 8);
            } else {
                const uint2 raw = *reinterpret_cast<const uint2 *>(p.lq + row * D + ch * 8);
                st.k[u] = make_uint4(raw.x, raw.y, 0, 0);
            }
        }
    }
    // V: unit = (key pair, chunk); KT/2 * CPR units (256 for D = 128).
    {
        const int kp2 = tid / CPR, ch = tid % CPR;
        st.v[0] = st.v[1] = make_uint4(0, 0, 0, 0);
        if (kp2 < KT / 2) {
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int pos = kt * KT + 2 * kp2 + e;
                if (pos < kend) {
                    const long long row = key_row<D, INT8>(p, bt, h, pos);
                    if (!INT8) {
                        st.v[e] = *reinterpret_cast<const uint4 *>(p.vp + row * D + ch * 8);
                    } else {
                        const uint2 raw = *reinterpret_cast<const uint2 *>(p.lq + half_q + row * D + ch * 8);
                        st.v[e] = make_uint4(raw.x, raw.y, 0, 0);
                    }
                }
            }
        }
    }
    if (INT8) {
        st.s = 0.0f;
        if (tid < 2 * KT) {
            const int pos = kt * KT + (tid % KT);
            if (pos < kend) {
                const long long row = key_row<D, INT8>(p, bt, h, pos);
                st.s = tid < KT ? p.ls[row] : p.ls[half_s + row];
            }
        }
    }
}

template <int D, bool INT8>
__device__ __forceinline__ void store_tile(const Stage<D, INT8> &st, Smem<D> &sm, int buf) {
    const int tid = threadIdx.x;
    constexpr int CPR = D / 8;
#pragma unroll
    for (int u = 0; u < Stage<D, INT8>::KPT; u++) {
        const int c = tid + 256 * u, key = c / CPR, ch = c % CPR;
        if (c < Stage<D, INT8>::KCH) {
            const uint4 val = INT8 ? i8x8_to_bf16x8(make_uint2(st.k[u].x, st.k[u].y)) : st.k[u];
            *reinterpret_cast<uint4 *>(&sm.k[buf][key * Smem<D>::KROW + ch * 8]) = val;
        }
    }
    const int kp2 = tid / CPR, ch = tid % CPR;
    if (kp2 < KT / 2) {
        uint4 a = st.v[0], b = st.v[1];
        if (INT8) {
            a = i8x8_to_bf16x8(make_uint2(a.x, a.y));
            b = i8x8_to_bf16x8(make_uint2(b.x, b.y));
        }
        const uint32_t wa[4] = {a.x, a.y, a.z, a.w}, wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int dd = 0; dd < 8; dd++) {
            const uint32_t lo = (wa[dd / 2] >> (16 * (dd & 1))) & 0xffff;
            const uint32_t hi = (wb[dd / 2] >> (16 * (dd & 1))) & 0xffff;
            *reinterpret_cast<uint32_t *>(&sm.vt[buf][(ch * 8 + dd) * Smem<D>::VROW + 2 * kp2]) = lo | (hi << 16);
        }
    }
    if (INT8 && tid < 2 * KT) {
        if (tid < KT) sm.sk[buf][tid] = st.s;
        else sm.sv[buf][tid - KT] = st.s;
    }
}

template <int D, bool INT8>
__global__ void __launch_bounds__(256) prefill_kernel(PrefillParams p) {
    constexpr int NKB = D / 32;
    constexpr int NDT = D / 16;
    __shared__ __attribute__((aligned(16))) Smem<D> sm;

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
    const int r16 = lane & 15, kg = lane >> 4;
    const int qt = p.qtiles - 1 - (int)blockIdx.x;   // heaviest tiles first
    const int h = blockIdx.y, b = blockIdx.z;
    const int tok0 = p.qsl ? p.qsl[b] : b * p.nmax;
    const int nb = p.qsl ? p.qsl[b + 1] - tok0 : p.nmax;
    const int t_first = qt * p.TQ;
    if (t_first >= nb) return;
    const int start = p.positions[tok0], len = start + nb;
    const int t_last = min(t_first + p.TQ, nb) - 1;
    const int kend = p.causal ? start + t_last + 1 : len;
    const int nkt = (kend + KT - 1) / KT;
    const int32_t *bt = p.bt + (size_t)b * p.bt_stride;

    // This lane's query row (B operand of S^T = K Q^T).
    const int r = w * 16 + r16, tl = r / p.G, g = r - tl * p.G, t = t_first + tl;
    const bool row_ok = tl < p.TQ && t < nb;
    const int qpos = p.causal && row_ok ? start + t : len - 1;
    bf16x8 qreg[NKB];
    {
        const uint16_t *qr = p.q + ((size_t)(tok0 + t) * p.Hq + h * p.G + g) * D;
#pragma unroll
        for (int i = 0; i < NKB; i++) {
            const int d0 = i * 32 + kg * 8;
            if (!row_ok) {
                qreg[i] = as_bf16x8((u32x4){0u, 0u, 0u, 0u});
            } else if (!INT8) {
                qreg[i] = as_bf16x8(*reinterpret_cast<const u32x4 *>(qr + d0));
            } else {
                const u32x4 raw = *reinterpret_cast<const u32x4 *>(qr + d0);
                u32x4 w;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    w[e] = pack_bf16x2(__uint_as_float(raw[e] << 16) * p.smooth[d0 + 2 * e],
                                       __uint_as_float(raw[e] & 0xffff0000u) * p.smooth[d0 + 2 * e + 1]);
                qreg[i] = as_bf16x8(w);
            }
        }
    }

    f32x4 o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) o[dt] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m = NEG_BIG, l = 0.0f;

    Stage<D, INT8> st;
    load_tile<D, INT8>(st, p, bt, h, 0, kend);
    store_tile<D, INT8>(st, sm, 0);
    __syncthreads();

    for (int kt = 0; kt < nkt; kt++) {
        const int buf = kt & 1;
        const bool more = kt + 1 < nkt;
        if (more) load_tile<D, INT8>(st, p, bt, h, kt + 1, kend);

        // S^T for two 16-key blocks.
        f32x4 sc[2];
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            sc[kb] = (f32x4){0.f, 0.f, 0.f, 0.f};
            const uint16_t *krow = &sm.k[buf][(kb * 16 + r16) * Smem<D>::KROW];
#pragma unroll
            for (int i = 0; i < NKB; i++) {
                const bf16x8 a = as_bf16x8(*reinterpret_cast<const u32x4 *>(krow + i * 32 + kg * 8));
                sc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qreg[i], sc[kb], 0, 0, 0);
            }
        }
        float x[8];
        float mt = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int key = kb * 16 + kg * 4 + e, kpos = kt * KT + key;
                float v = sc[kb][e];
                if (INT8) v *= sm.sk[buf][key];
                v *= p.scale_log2;
                const float xv = (kpos <= qpos && kpos < kend) ? v : -INFINITY;
                x[kb * 4 + e] = xv;
                mt = fmaxf(mt, xv);
            }
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float mn = fmaxf(m, mt);
        const float alpha = fast_exp2(m - mn);
        m = mn;
        float ps = 0.0f, pe[8];
#pragma unroll
        for (int k8 = 0; k8 < 8; k8++) {
            pe[k8] = fast_exp2(x[k8] - mn);
            ps += pe[k8];
            if (INT8) pe[k8] *= sm.sv[buf][(k8 / 4) * 16 + kg * 4 + (k8 & 3)];
        }
        const bf16x8 pb = as_bf16x8((u32x4){pack_bf16x2(pe[0], pe[1]), pack_bf16x2(pe[2], pe[3]),
                                            pack_bf16x2(pe[4], pe[5]), pack_bf16x2(pe[6], pe[7])});
        l = l * alpha + ps;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            const uint16_t *vrow = &sm.vt[buf][(dt * 16 + r16) * Smem<D>::VROW];
            const u32x2 lo = *reinterpret_cast<const u32x2 *>(vrow + kg * 4);
            const u32x2 hi = *reinterpret_cast<const u32x2 *>(vrow + 16 + kg * 4);
            const bf16x8 a = as_bf16x8((u32x4){lo[0], lo[1], hi[0], hi[1]});
            o[dt] *= alpha;
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, o[dt], 0, 0, 0);
        }
        if (more) store_tile<D, INT8>(st, sm, buf ^ 1);
        __syncthreads();
    }

    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (!row_ok) return;
    const float inv = 1.0f / l;
    uint16_t *orow = p.out + ((size_t)(tok0 + t) * p.Hq + h * p.G + g) * D;
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) {
        const int d = dt * 16 + kg * 4;
        const uint32_t w0 = (uint32_t)f2bf(o[dt][0] * inv) | ((uint32_t)f2bf(o[dt][1] * inv) << 16);
        const uint32_t w1 = (uint32_t)f2bf(o[dt][2] * inv) | ((uint32_t)f2bf(o[dt][3] * inv) << 16);
        *reinterpret_cast<u32x2 *>(orow + d) = (u32x2){w0, w1};
    }
}

}  // namespace

int ti_launch_prefill(const ti_attention_args *a, const ti_kv_cache *c, hipStream_t s) {
    PrefillParams p;
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
    p.bt_stride = a->block_table_stride;
    p.num_pages = c->num_pages;
    p.P = c->page_size;
    p.Hk = c->kv_heads;
    p.Hq = a->q_heads;
    p.G = a->q_heads / c->kv_heads;
    p.TQ = 64 / p.G;
    p.nmax = a->max_query_len;
    p.qtiles = (a->max_query_len + p.TQ - 1) / p.TQ;
    p.causal = a->causal;
    p.scale_log2 = a->scale * LOG2E;
    dim3 grid(p.qtiles, c->kv_heads, a->num_seqs);
    const bool int8 = c->kind == TI_KV_INT8;
    if (c->head_dim == 128) {
        if (int8) prefill_kernel<128, true><<<grid, 256, 0, s>>>(p);
        else prefill_kernel<128, false><<<grid, 256, 0, s>>>(p);
    } else {
        if (int8) prefill_kernel<64, true><<<grid, 256, 0, s>>>(p);
        else prefill_kernel<64, false><<<grid, 256, 0, s>>>(p);
    }
    return hipGetLastError() == hipSuccess ? TI_OK : TI_ERR_LAUNCH;
}
