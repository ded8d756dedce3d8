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
#include <stdlib.h>

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
    int bt_stride, num_pages, P, pshift, Hk, Hq, G, TQ, nmax, qtiles, causal;
    float scale_log2;
};

constexpr int KT = 32;                 // keys per LDS tile
constexpr float RESCALE_LOG2 = 8.0f;   // lazy-rescale threshold (see the decode kernel)

template <int D>
struct Smem {
    static constexpr int KROW = D + 8;   // padded K row (uint16)
    static constexpr int VROW = KT + 4;  // padded V^T row (uint16)
    uint16_t k[2][KT * KROW];
    uint16_t vt[2][D * VROW];
    float sk[2][KT], sv[2][KT];
};

// Registers holding one key tile between its global load and its LDS store (per thread
// of a 256-thread key group).
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

// Pool row of key position pos (clamped into the step's keys: rows past kend hold finite
// cache data whose probabilities are masked to 0).
__device__ __forceinline__ long long key_row(const PrefillParams &p, const int32_t *bt, int h,
                                             int pos, int kend) {
    pos = min(pos, kend - 1);
    const int idx = p.pshift >= 0 ? pos >> p.pshift : pos / p.P;
    const int off = p.pshift >= 0 ? pos & (p.P - 1) : pos % p.P;
    const int pg = page_of(bt, idx, p.num_pages);
    return ((long long)pg * p.Hk + h) * p.P + off;
}

// Rows of the tile's keys. PG16 (P % 16 == 0): each 16-key half of the tile lies in one
// page, found with a scalar block-table load; key k's row is half_row[k / 16] + k % 16.
// Otherwise a per-key lookup (vector loads).
template <bool PG16>
struct TileRows {
    long long half_row[2];
    const PrefillParams *p;
    const int32_t *bt;
    int h, kt, kend;
    __device__ __forceinline__ TileRows(const PrefillParams &pp, const int32_t *btp, int hh, int ktt, int ke)
        : p(&pp), bt(btp), h(hh), kt(ktt), kend(ke) {
        if (PG16) {
#pragma unroll
            for (int x = 0; x < 2; x++) {
                const int pos = min(kt * KT + 16 * x, kend - 1);
                const int idx = pp.pshift >= 0 ? pos >> pp.pshift : pos / pp.P;
                const int off = pp.pshift >= 0 ? pos & (pp.P - 1) : pos % pp.P;
                const int pg = page_of_s(btp, idx, pp.num_pages);
                half_row[x] = ((long long)pg * pp.Hk + hh) * pp.P + (off & ~15);
            }
        }
    }
    __device__ __forceinline__ long long row(int key) const {
        if (PG16) {
            const int pos = kt * KT + key, last = kend - 1;
            const int k = pos <= last ? key : last - kt * KT;   // clamp into the step's keys
            return (k < 16 ? half_row[0] : half_row[1]) + (k & 15);
        }
        return key_row(*p, bt, h, kt * KT + key, kend);
    }
};

template <int D, bool INT8, bool PG16>
__device__ __forceinline__ void load_tile(Stage<D, INT8> &st, const PrefillParams &p,
                                          const int32_t *bt, int h, int kt, int kend, int gtid) {
    const size_t half_q = (size_t)p.num_pages * p.Hk * p.P * D;
    const size_t half_s = (size_t)p.num_pages * p.Hk * p.P;
    constexpr int CPR = D / 8;
    const TileRows<PG16> tr(p, bt, h, kt, kend);
#pragma unroll
    for (int u = 0; u < Stage<D, INT8>::KPT; u++) {
        const int c = gtid + 256 * u, key = c / CPR, ch = c % CPR;
        if (c < Stage<D, INT8>::KCH) {
            const long long row = tr.row(key);
            if (!INT8) {
                st.k[u] = *reinterpret_cast<const uint4 *>(p.kp + row * D + ch * 8);
            } else {
                const uint2 raw = *reinterpret_cast<const uint2 *>(p.lq + row * D + ch * 8);
                st.k[u] = make_uint4(raw.x, raw.y, 0, 0);
            }
        }
    }
    // V: unit = (key pair, chunk); KT/2 * CPR units (256 for D = 128).
    const int kp2 = gtid / CPR, ch = gtid % CPR;
    if (kp2 < KT / 2) {
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const long long row = tr.row(2 * kp2 + e);
            if (!INT8) {
                st.v[e] = *reinterpret_cast<const uint4 *>(p.vp + row * D + ch * 8);
            } else {
                const uint2 raw = *reinterpret_cast<const uint2 *>(p.lq + half_q + row * D + ch * 8);
                st.v[e] = make_uint4(raw.x, raw.y, 0, 0);
            }
        }
    }
    if (INT8 && gtid < 2 * KT) {
        const long long row = tr.row(gtid % KT);
        st.s = gtid < KT ? p.ls[row] : p.ls[half_s + row];
    }
}

template <int D, bool INT8>
__device__ __forceinline__ void store_tile(const Stage<D, INT8> &st, Smem<D> &sm, int buf, int gtid) {
    constexpr int CPR = D / 8;
#pragma unroll
    for (int u = 0; u < Stage<D, INT8>::KPT; u++) {
        const int c = gtid + 256 * u, key = c / CPR, ch = c % CPR;
        if (c < Stage<D, INT8>::KCH) {
            const uint4 val = INT8 ? i8x8_to_bf16x8(make_uint2(st.k[u].x, st.k[u].y)) : st.k[u];
            *reinterpret_cast<uint4 *>(&sm.k[buf][key * Smem<D>::KROW + ch * 8]) = val;
        }
    }
    const int kp2 = gtid / CPR, ch = gtid % CPR;
    if (kp2 < KT / 2) {
        uint4 a = st.v[0], b = st.v[1];
        if (INT8) {
            a = i8x8_to_bf16x8(make_uint2(a.x, a.y));
            b = i8x8_to_bf16x8(make_uint2(b.x, b.y));
        }
        const uint32_t wa[4] = {a.x, a.y, a.z, a.w}, wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int dd = 0; dd < 8; dd++) {
            const uint32_t word = __builtin_amdgcn_perm(wb[dd / 2], wa[dd / 2], (dd & 1) ? 0x07060302u : 0x05040100u);
            *reinterpret_cast<uint32_t *>(&sm.vt[buf][(ch * 8 + dd) * Smem<D>::VROW + 2 * kp2]) = word;
        }
    }
    if (INT8 && gtid < 2 * KT) {
        if (gtid < KT) sm.sk[buf][gtid] = st.s;
        else sm.sv[buf][gtid - KT] = st.s;
    }
}

// NG key groups of 4 waves each. Every group holds all 64 packed rows (16 per wave) and
// walks the key tiles kt = grp, grp + NG, ... with its own LDS double buffer and a
// two-deep register prefetch, so NG tiles (and up to 2 NG more in flight) are processed at
// once; the groups' online-softmax states merge through LDS at the end.
template <int D, bool INT8, int NG, bool PG16>
__global__ void __launch_bounds__(256 * NG) prefill_kernel(PrefillParams p) {
    constexpr int NKB = D / 32;
    constexpr int NDT = D / 16;
    constexpr int SMEM = sizeof(Smem<D>) * NG;
    constexpr int MERGE = 64 * (D + 2) * 4;
    __shared__ __attribute__((aligned(16))) char smem_raw[SMEM > MERGE ? SMEM : MERGE];
    Smem<D> *smg = reinterpret_cast<Smem<D> *>(smem_raw);
    float (*mrg)[D + 2] = reinterpret_cast<float (*)[D + 2]>(smem_raw);

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
    const int grp = w >> 2, wl = w & 3, gtid = threadIdx.x & 255;
    const int r16 = lane & 15, kg = lane >> 4;
    // Grid (Hk, qtiles, B): consecutive work-groups (spread round-robin over the 8 XCDs)
    // belong to different KV heads, so each head's K/V stays in one XCD's L2.
    const int h = blockIdx.x;
    const int qt = p.qtiles - 1 - (int)blockIdx.y;   // heaviest tiles first
    const int b = blockIdx.z;
    const int tok0 = p.qsl ? p.qsl[b] : b * p.nmax;
    const int nb = p.qsl ? p.qsl[b + 1] - tok0 : p.nmax;
    const int t_first = qt * p.TQ;
    if (t_first >= nb) return;
    const int start = p.positions[tok0], len = start + nb;
    const int t_last = min(t_first + p.TQ, nb) - 1;
    const int kend = p.causal ? start + t_last + 1 : len;
    const int nkt = (kend + KT - 1) / KT;
    const int steps = (nkt + NG - 1) / NG;                 // same for every group
    const int32_t *bt = p.bt + (size_t)b * p.bt_stride;
    Smem<D> &sm = smg[grp];
    // Keys up to mask_from are visible to every row of this tile.
    const int mask_from = p.causal ? start + t_first : len - 1;

    // This lane's query row (B operand of S^T = K Q^T).
    const int r = wl * 16 + r16, tl = r / p.G, g = r - tl * p.G, t = t_first + tl;
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
                u32x4 wv;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    wv[e] = pack_bf16x2(__uint_as_float(raw[e] << 16) * p.smooth[d0 + 2 * e],
                                        __uint_as_float(raw[e] & 0xffff0000u) * p.smooth[d0 + 2 * e + 1]);
                qreg[i] = as_bf16x8(wv);
            }
        }
    }

    f32x4 o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) o[dt] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m = NEG_BIG, l = 0.0f;

    auto compute = [&](int kt, int buf) {
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
        const bool need_mask = kt * KT + KT - 1 > mask_from;
        float x[8];
        float mt = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int key = kb * 16 + kg * 4 + e;
                float v = sc[kb][e];
                if (INT8) v *= sm.sk[buf][key];
                v *= p.scale_log2;
                if (need_mask) {
                    const int kpos = kt * KT + key;
                    v = (kpos <= qpos && kpos < kend) ? v : -INFINITY;
                }
                x[kb * 4 + e] = v;
                mt = fmaxf(mt, v);
            }
        if (__any(mt > m + RESCALE_LOG2)) {
            mt = fmaxf(mt, __shfl_xor(mt, 16));
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float mn = fmaxf(m, mt);
            const float alpha = fast_exp2(m - mn);
            m = mn;
            l *= alpha;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) o[dt] *= alpha;
        }
        float ps = 0.0f, pe[8];
#pragma unroll
        for (int k8 = 0; k8 < 8; k8++) {
            pe[k8] = fast_exp2(x[k8] - m);
            ps += pe[k8];
            if (INT8) pe[k8] *= sm.sv[buf][(k8 / 4) * 16 + kg * 4 + (k8 & 3)];
        }
        const bf16x8 pb = as_bf16x8((u32x4){pack_bf16x2(pe[0], pe[1]), pack_bf16x2(pe[2], pe[3]),
                                            pack_bf16x2(pe[4], pe[5]), pack_bf16x2(pe[6], pe[7])});
        l += ps;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            const uint16_t *vrow = &sm.vt[buf][(dt * 16 + r16) * Smem<D>::VROW];
            const u32x2 lo = *reinterpret_cast<const u32x2 *>(vrow + kg * 4);
            const u32x2 hi = *reinterpret_cast<const u32x2 *>(vrow + 16 + kg * 4);
            const bf16x8 a = as_bf16x8((u32x4){lo[0], lo[1], hi[0], hi[1]});
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, o[dt], 0, 0, 0);
        }
    };

    // Step i of this group handles tile grp + NG i. Register stages s0/s1 alternate: at
    // step i, tile i + 1 is already in flight and tile i + 2 is issued.
    // Loads are issued unconditionally (a step past the group's last tile re-reads its
    // last tile, never used) so the number of loads in flight is static and the waits
    // before each LDS store only cover the tile being stored.
    Stage<D, INT8> s0, s1;
    auto tile_of = [&](int i) { return grp + NG * i; };
    auto ld = [&](Stage<D, INT8> &stg, int i) {
        load_tile<D, INT8, PG16>(stg, p, bt, h, min(tile_of(i), nkt - 1), kend, gtid);
    };
    ld(s0, 0);
    ld(s1, 1);
    if (tile_of(0) < nkt) store_tile<D, INT8>(s0, sm, 0, gtid);
    __syncthreads();
    for (int i = 0; i < steps; i += 2) {
        // even step: compute buf 0, prefetch into s0, stage s1 -> buf 1
        ld(s0, i + 2);
        if (tile_of(i) < nkt) compute(tile_of(i), 0);
        if (tile_of(i + 1) < nkt) store_tile<D, INT8>(s1, sm, 1, gtid);
        __syncthreads();
        if (i + 1 >= steps) break;
        // odd step: compute buf 1, prefetch into s1, stage s0 -> buf 0
        ld(s1, i + 3);
        if (tile_of(i + 1) < nkt) compute(tile_of(i + 1), 1);
        if (tile_of(i + 2) < nkt) store_tile<D, INT8>(s0, sm, 0, gtid);
        __syncthreads();
    }

    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (NG > 1) {
        // Merge the groups' states (same rows, disjoint keys) through LDS, group by group.
        for (int src = 0; src < NG; src++) {
            if (grp == src) {
                float mo = NEG_BIG, lo = 0.0f;
                if (src > 0) {
                    mo = mrg[r][D];
                    lo = mrg[r][D + 1];
                }
                const float mn = fmaxf(mo, m);
                const float wo = src > 0 ? fast_exp2(mo - mn) : 0.0f;
                const float wm = fast_exp2(m - mn);
#pragma unroll
                for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int d = dt * 16 + kg * 4 + e;
                        const float prev = src > 0 ? mrg[r][d] : 0.0f;
                        o[dt][e] = prev * wo + o[dt][e] * wm;
                        mrg[r][d] = o[dt][e];
                    }
                l = lo * wo + l * wm;
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                if (kg == 0) {
                    mrg[r][D] = mn;
                    mrg[r][D + 1] = l;
                }
            }
            __syncthreads();
        }
        if (grp != NG - 1) return;   // the last group holds the merged state in registers
    }
    if (!row_ok) return;
    const float inv = 1.0f / l;
    uint16_t *orow = p.out + ((size_t)(tok0 + t) * p.Hq + h * p.G + g) * D;
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) {
        const int d = dt * 16 + kg * 4;
        const uint32_t w0 = pack_bf16x2(o[dt][0] * inv, o[dt][1] * inv);
        const uint32_t w1 = pack_bf16x2(o[dt][2] * inv, o[dt][3] * inv);
        *reinterpret_cast<u32x2 *>(orow + d) = (u32x2){w0, w1};
    }
}

template <int D, bool INT8, bool PG16>
void launch_prefill_g(const PrefillParams &p, int ng, dim3 grid, hipStream_t s) {
    switch (ng) {
        case 1: prefill_kernel<D, INT8, 1, PG16><<<grid, 256, 0, s>>>(p); break;
        case 2: prefill_kernel<D, INT8, 2, PG16><<<grid, 512, 0, s>>>(p); break;
        default: prefill_kernel<D, INT8, 4, PG16><<<grid, 1024, 0, s>>>(p); break;
    }
}

template <int D, bool INT8>
void launch_prefill_d(const PrefillParams &p, int ng, dim3 grid, hipStream_t s) {
    if (p.P % 16 == 0) launch_prefill_g<D, INT8, true>(p, ng, grid, s);
    else launch_prefill_g<D, INT8, false>(p, ng, grid, s);
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
    p.pshift = (c->page_size & (c->page_size - 1)) == 0 ? __builtin_ctz(c->page_size) : -1;
    p.Hk = c->kv_heads;
    p.Hq = a->q_heads;
    p.G = a->q_heads / c->kv_heads;
    p.TQ = 64 / p.G;
    p.nmax = a->max_query_len;
    p.qtiles = (a->max_query_len + p.TQ - 1) / p.TQ;
    p.causal = a->causal;
    p.scale_log2 = a->scale * LOG2E;
    // Key groups per work-group: enough waves to hide the tile loads' latency when the
    // grid alone cannot (TI_PREFILL_GROUPS overrides, tuning only).
    static const int forced = [] {
        const char *e = getenv("TI_PREFILL_GROUPS");
        return e ? atoi(e) : 0;
    }();
    const long long wgs = (long long)p.qtiles * c->kv_heads * a->num_seqs;
    int ng = wgs >= 1024 ? 1 : (wgs >= 512 ? 2 : 4);
    if (forced == 1 || forced == 2 || forced == 4) ng = forced;
    dim3 grid(c->kv_heads, p.qtiles, a->num_seqs);
    const bool int8 = c->kind == TI_KV_INT8;
    if (c->head_dim == 128) {
        if (int8) launch_prefill_d<128, true>(p, ng, grid, s);
        else launch_prefill_d<128, false>(p, ng, grid, s);
    } else {
        if (int8) launch_prefill_d<64, true>(p, ng, grid, s);
        else launch_prefill_d<64, false>(p, ng, grid, s);
    }
    return hipGetLastError() == hipSuccess ? TI_OK : TI_ERR_LAUNCH;
}
