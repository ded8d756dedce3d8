// Split-KV paged decode / verify attention on bf16 MFMA (gfx950), dense bf16 or INT8 cache.
//
// Reference: attention_decode_kernel / decode_body / attention_combine_kernel
// (src/ops/tile/attention.jl:185-245) and its INT8 variant (:68-95, :194-202).
//
// Work decomposition. The G = Hq/Hk query heads that share a KV head, times the n query
// tokens of the step, are packed into M = G*n query rows (row r = g + G t, as the
// reference's packed tile). One work-group (4 waves) handles one (sequence, KV head,
// split); a split is a contiguous range of 16-key tiles of the sequence, and the waves of
// the group take every 4th tile of it, each with its own online-softmax state. The grid
// depends only on host shapes (B, Hk, splits), never on the context length, so a captured
// graph stays valid as sequences grow; splits that get no keys write a neutral partial.
//
// Per 16-key tile and wave (lane l; r = l % 16 is the query row within a 16-row block,
// k = l / 16 its key/element group):
//   S^T = K Q^T      v_mfma_f32_16x16x32_bf16, A = K rows loaded straight from HBM
//                    (lane: key l%16, 8 head-dim elements per 32-wide block, 16 B loads);
//                    C lands as lane (row r, keys 4k..4k+3).
//   online softmax   exp2 domain (scale * log2 e), per lane for its own row; the row max
//                    over the tile's 16 keys is two xor shuffles (lanes r, r+16, r+32, r+48).
//   O^T += V^T P^T   v_mfma_f32_16x16x16_bf16, B = P^T comes straight from the S^T
//                    registers (same lane layout), A = V^T read from a per-wave LDS tile
//                    that holds V transposed (written from coalesced 16 B row loads).
//                    O^T's lane layout keeps each lane on its own row, so the rescale by
//                    alpha needs no shuffles.
// INT8 keys and values are exact in bf16; a key's scale multiplies its scores and a
// value's scale its probability (src/ops/quant.jl:56-72); queries are multiplied by the
// keys' smoothing and rounded to bf16 (attention.jl:90-95).
//
// At the end the four waves merge their (m, l, O) through LDS and the group writes one
// Float32 partial (acc[D], m, l) per packed row; the combine kernel merges the splits:
// w_s = exp2(m_s - max m), o = sum acc_s w_s / sum l_s w_s.
#include "common.hpp"

using namespace ti;

namespace {

struct DecodeParams {
    const uint16_t *q;
    uint16_t *out;
    const uint16_t *kp, *vp;
    const int8_t *lq;
    const float *ls, *smooth;
    const int32_t *positions, *qsl, *bt;
    float *part;
    int bt_stride, num_pages, P, Hk, Hq, G, nmax, M, splits, causal;
    float scale_log2;
};

typedef short s16x4 __attribute__((ext_vector_type(4)));

// Transposed V tile in LDS: [D][16 keys] bf16, rows padded to 40 B (conflict-free reads).
constexpr int VT_ROW = 20;  // uint16 per padded row

__device__ __forceinline__ void lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// 8 int8 -> 8 bf16 words (exact).
__device__ __forceinline__ u32x4 i8x8_to_bf16(uint2 v) {
    u32x4 r;
    uint32_t a, b, c, d;
    i8x4_to_bf16(v.x, a, b);
    i8x4_to_bf16(v.y, c, d);
    r[0] = a; r[1] = b; r[2] = c; r[3] = d;
    return r;
}

template <int D, int ROWB, bool INT8>
__global__ void __launch_bounds__(256) decode_kernel(DecodeParams p) {
    constexpr int NKB = D / 32;          // 32-wide head-dim blocks (QK MFMAs per tile)
    constexpr int NDT = D / 16;          // 16-wide head-dim tiles (PV MFMAs per tile)
    constexpr int CPR = D / 8;           // 8-element chunks per V row
    constexpr int KPL = 16 * CPR / 64;   // keys per lane in the V load (4 for D=128)
    constexpr int MP = ROWB * 16;        // padded rows

    __shared__ __attribute__((aligned(16))) uint16_t vt[4][D * VT_ROW];
    __shared__ float mrg[MP][D + 2];

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int r16 = lane & 15, kg = lane >> 4;
    const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tok0 = p.qsl ? p.qsl[b] : b * p.nmax;
    const int nb = p.qsl ? p.qsl[b + 1] - tok0 : p.nmax;
    if (nb <= 0) return;
    const int start = p.positions[tok0], len = start + nb;
    const int ntiles = (len + 15) >> 4;
    const int per = (ntiles + p.splits - 1) / p.splits;
    const int j0 = s * per, j1 = min(j0 + per, ntiles);
    const int32_t *bt = p.bt + (size_t)b * p.bt_stride;
    const size_t half_q = (size_t)p.num_pages * p.Hk * p.P * D;
    const size_t half_s = (size_t)p.num_pages * p.Hk * p.P;

    // Query operands (B of S^T = K Q^T): row rb*16 + r16, elements i*32 + kg*8 .. +8.
    bf16x8 qreg[ROWB][NKB];
    int qpos[ROWB];
#pragma unroll
    for (int rb = 0; rb < ROWB; rb++) {
        const int r = rb * 16 + r16, t = r / p.G, g = r - t * p.G;
        const bool ok = r < p.M && t < nb;
        qpos[rb] = p.causal && ok ? start + t : len - 1;
        const uint16_t *qr = p.q + ((size_t)(tok0 + t) * p.Hq + h * p.G + g) * D;
#pragma unroll
        for (int i = 0; i < NKB; i++) {
            const int d0 = i * 32 + kg * 8;
            if (!ok) {
                qreg[rb][i] = as_bf16x8((u32x4){0u, 0u, 0u, 0u});
            } else if (!INT8) {
                qreg[rb][i] = as_bf16x8(*reinterpret_cast<const u32x4 *>(qr + d0));
            } else {
                const u32x4 raw = *reinterpret_cast<const u32x4 *>(qr + d0);
                u32x4 wv;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    wv[e] = pack_bf16x2(__uint_as_float(raw[e] << 16) * p.smooth[d0 + 2 * e],
                                        __uint_as_float(raw[e] & 0xffff0000u) * p.smooth[d0 + 2 * e + 1]);
                qreg[rb][i] = as_bf16x8(wv);
            }
        }
    }

    f32x4 o[ROWB][NDT];
    float m[ROWB], l[ROWB];
#pragma unroll
    for (int rb = 0; rb < ROWB; rb++) {
        m[rb] = NEG_BIG;
        l[rb] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) o[rb][dt] = (f32x4){0.f, 0.f, 0.f, 0.f};
    }

    uint16_t *myvt = vt[w];
    const int vc = lane % CPR, vg = lane / CPR;   // V load: chunk, key group

    for (int j = j0 + w; j < j1; j += 4) {
        // ---- loads: K rows (lane key r16) and V rows (lane keys vg*KPL + e) ----
        const int kpos = j * 16 + r16;
        long long krow = -1;
        if (kpos < len) {
            const int pg = page_of(bt, kpos / p.P, p.num_pages);
            krow = ((long long)pg * p.Hk + h) * p.P + kpos % p.P;
        }
        bf16x8 kreg[NKB];
        float sk = 0.0f, sv = 0.0f;
        if (!INT8) {
#pragma unroll
            for (int i = 0; i < NKB; i++)
                kreg[i] = as_bf16x8(krow >= 0 ? *reinterpret_cast<const u32x4 *>(p.kp + krow * D + i * 32 + kg * 8)
                                              : (u32x4){0u, 0u, 0u, 0u});
        } else {
#pragma unroll
            for (int i = 0; i < NKB; i++) {
                const uint2 raw = krow >= 0 ? *reinterpret_cast<const uint2 *>(p.lq + krow * D + i * 32 + kg * 8)
                                            : make_uint2(0, 0);
                kreg[i] = as_bf16x8(i8x8_to_bf16(raw));
            }
            if (krow >= 0) {
                sk = p.ls[krow];
                sv = p.ls[half_s + krow];
            }
        }
        // V rows -> transposed LDS tile vt[d][key].
        {
            uint32_t packed[8][KPL / 2];
            uint16_t vals[KPL][8];
#pragma unroll
            for (int e = 0; e < KPL; e++) {
                const int key = vg * KPL + e, vpos = j * 16 + key;
                if (vpos < len) {
                    const int pg = page_of(bt, vpos / p.P, p.num_pages);
                    const long long vrow = ((long long)pg * p.Hk + h) * p.P + vpos % p.P;
                    if (!INT8) {
                        const uint4 raw = *reinterpret_cast<const uint4 *>(p.vp + vrow * D + vc * 8);
                        const uint32_t wds[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                        for (int q2 = 0; q2 < 4; q2++) {
                            vals[e][2 * q2] = (uint16_t)(wds[q2] & 0xffff);
                            vals[e][2 * q2 + 1] = (uint16_t)(wds[q2] >> 16);
                        }
                    } else {
                        const uint2 raw = *reinterpret_cast<const uint2 *>(p.lq + half_q + vrow * D + vc * 8);
                        const u32x4 cv = i8x8_to_bf16(raw);
#pragma unroll
                        for (int q2 = 0; q2 < 4; q2++) {
                            vals[e][2 * q2] = (uint16_t)(cv[q2] & 0xffff);
                            vals[e][2 * q2 + 1] = (uint16_t)(cv[q2] >> 16);
                        }
                    }
                } else {
#pragma unroll
                    for (int q2 = 0; q2 < 8; q2++) vals[e][q2] = 0;
                }
            }
#pragma unroll
            for (int dd = 0; dd < 8; dd++)
#pragma unroll
                for (int e2 = 0; e2 < KPL / 2; e2++)
                    packed[dd][e2] = (uint32_t)vals[2 * e2][dd] | ((uint32_t)vals[2 * e2 + 1][dd] << 16);
            lds_fence();   // previous tile's reads of myvt are done before overwriting
#pragma unroll
            for (int dd = 0; dd < 8; dd++) {
                uint16_t *dst = myvt + (vc * 8 + dd) * VT_ROW + vg * KPL;
                if (KPL == 4)
                    *reinterpret_cast<u32x2 *>(dst) = (u32x2){packed[dd][0], packed[dd][KPL / 2 - 1]};
                else
                    *reinterpret_cast<uint32_t *>(dst) = packed[dd][0];
            }
        }

        // ---- S^T = K Q^T ----
        f32x4 sc[ROWB];
#pragma unroll
        for (int rb = 0; rb < ROWB; rb++) {
            sc[rb] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < NKB; i++)
                sc[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kreg[i], qreg[rb][i], sc[rb], 0, 0, 0);
        }
        // Key scales of this lane's 4 keys (kg*4 + e), from the lanes that loaded them.
        float skk[4], svk[4];
        if (INT8) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                skk[e] = __shfl(sk, kg * 4 + e);
                svk[e] = __shfl(sv, kg * 4 + e);
            }
        }

        // ---- online softmax + P^T operands ----
        s16x4 pop[ROWB];
        float alpha[ROWB];
#pragma unroll
        for (int rb = 0; rb < ROWB; rb++) {
            float x[4];
            float mt = -INFINITY;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int kp = j * 16 + kg * 4 + e;
                float v = sc[rb][e];
                if (INT8) v *= skk[e];
                v *= p.scale_log2;
                x[e] = (kp <= qpos[rb] && kp < len) ? v : -INFINITY;
                mt = fmaxf(mt, x[e]);
            }
            mt = fmaxf(mt, __shfl_xor(mt, 16));
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float mn = fmaxf(m[rb], mt);
            alpha[rb] = fast_exp2(m[rb] - mn);
            m[rb] = mn;
            float ps = 0.0f, pe[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                pe[e] = fast_exp2(x[e] - mn);
                ps += pe[e];
                if (INT8) pe[e] *= svk[e];
            }
            l[rb] = l[rb] * alpha[rb] + ps;
            pop[rb] = __builtin_bit_cast(s16x4, (u32x2){pack_bf16x2(pe[0], pe[1]), pack_bf16x2(pe[2], pe[3])});
        }

        // ---- O^T = alpha O^T + V^T P^T ----
        lds_fence();   // this tile's V^T is in LDS
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            const s16x4 a = __builtin_bit_cast(s16x4, *reinterpret_cast<const u32x2 *>(myvt + (dt * 16 + r16) * VT_ROW + kg * 4));
#pragma unroll
            for (int rb = 0; rb < ROWB; rb++) {
                o[rb][dt] *= alpha[rb];
                o[rb][dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, pop[rb], o[rb][dt], 0, 0, 0);
            }
        }
    }

    // ---- merge the four waves' states through LDS (sequentially) ----
#pragma unroll
    for (int rb = 0; rb < ROWB; rb++) {
        l[rb] += __shfl_xor(l[rb], 16);
        l[rb] += __shfl_xor(l[rb], 32);
    }
    for (int src = 0; src < 4; src++) {
        if (w == src) {
#pragma unroll
            for (int rb = 0; rb < ROWB; rb++) {
                const int r = rb * 16 + r16;
                float mo = NEG_BIG, lo = 0.0f;
                if (src > 0) {
                    mo = mrg[r][D];
                    lo = mrg[r][D + 1];
                }
                const float mn = fmaxf(mo, m[rb]);
                const float wo = src > 0 ? fast_exp2(mo - mn) : 0.0f;
                const float wm = fast_exp2(m[rb] - mn);
#pragma unroll
                for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int d = dt * 16 + kg * 4 + e;
                        const float prev = src > 0 ? mrg[r][d] : 0.0f;
                        mrg[r][d] = prev * wo + o[rb][dt][e] * wm;
                    }
                lds_fence();
                if (kg == 0) {
                    mrg[r][D] = mn;
                    mrg[r][D + 1] = lo * wo + l[rb] * wm;
                }
            }
        }
        __syncthreads();
    }

    // ---- write the partial of this split: part[unit][r][D + 2] for rows r < M ----
    const size_t unit = ((size_t)b * p.Hk + h) * p.splits + s;
    float *dst = p.part + unit * (size_t)p.M * (D + 2);
    for (int idx = threadIdx.x; idx < p.M * (D + 2); idx += 256) {
        const int r = idx / (D + 2), c = idx - r * (D + 2);
        dst[idx] = mrg[r][c];
    }
}

// Merge the splits of one packed row: grid (M, Hk, B), one wave.
template <int D>
__global__ void __launch_bounds__(64) combine_kernel(DecodeParams p) {
    const int r = blockIdx.x, h = blockIdx.y, b = blockIdx.z, lane = threadIdx.x;
    const int tok0 = p.qsl ? p.qsl[b] : b * p.nmax;
    const int nb = p.qsl ? p.qsl[b + 1] - tok0 : p.nmax;
    const int t = r / p.G, g = r - t * p.G;
    if (t >= nb) return;
    const size_t unit0 = ((size_t)b * p.Hk + h) * p.splits;
    const size_t stride = (size_t)p.M * (D + 2);
    const float *base = p.part + unit0 * stride + (size_t)r * (D + 2);
    __shared__ float ws[256];
    float mmax = NEG_BIG;
    for (int sp = lane; sp < p.splits; sp += 64) mmax = fmaxf(mmax, base[sp * stride + D]);
    mmax = wave_max(mmax);
    float lsum = 0.0f;
    for (int sp = lane; sp < p.splits; sp += 64) {
        const float wgt = fast_exp2(base[sp * stride + D] - mmax);
        ws[sp] = wgt;
        lsum += base[sp * stride + D + 1] * wgt;
    }
    lsum = wave_sum(lsum);
    __syncthreads();
    constexpr int PER = D / 64;
    float acc[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) acc[k] = 0.0f;
    for (int sp = 0; sp < p.splits; sp++) {
        const float wgt = ws[sp];
#pragma unroll
        for (int k = 0; k < PER; k++) acc[k] += base[sp * stride + lane + 64 * k] * wgt;
    }
    uint16_t *o = p.out + ((size_t)(tok0 + t) * p.Hq + h * p.G + g) * D;
#pragma unroll
    for (int k = 0; k < PER; k++) o[lane + 64 * k] = f2bf(acc[k] / lsum);
}

template <int D, bool INT8>
void launch_decode_d(const DecodeParams &p, int rowb, dim3 grid, hipStream_t s) {
    switch (rowb) {
        case 1: decode_kernel<D, 1, INT8><<<grid, 256, 0, s>>>(p); break;
        case 2: decode_kernel<D, 2, INT8><<<grid, 256, 0, s>>>(p); break;
        case 3: decode_kernel<D, 3, INT8><<<grid, 256, 0, s>>>(p); break;
        default: decode_kernel<D, 4, INT8><<<grid, 256, 0, s>>>(p); break;
    }
}

}  // namespace

// Splits per (sequence, KV head): enough work-groups to fill 256 CUs several times over,
// a power of two, depending only on host shapes (never on context length).
ti_decode_plan ti_plan_decode(const ti_attention_args *a, const ti_kv_cache *c) {
    ti_decode_plan pl;
    const int G = a->q_heads / c->kv_heads;
    pl.rows = G * a->max_query_len;
    const long long pairs = (long long)a->num_seqs * c->kv_heads;
    const long long target = 2048;
    int sp = 1;
    while (sp < 128 && pairs * sp < target) sp <<= 1;
    pl.splits = sp;
    pl.bytes = (size_t)pairs * sp * pl.rows * (c->head_dim + 2) * sizeof(float);
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
    p.bt_stride = a->block_table_stride;
    p.num_pages = c->num_pages;
    p.P = c->page_size;
    p.Hk = c->kv_heads;
    p.Hq = a->q_heads;
    p.G = a->q_heads / c->kv_heads;
    p.nmax = a->max_query_len;
    p.M = pl.rows;
    p.splits = pl.splits;
    p.causal = a->causal;
    p.scale_log2 = a->scale * LOG2E;
    const int rowb = (pl.rows + 15) / 16;
    dim3 grid(pl.splits, c->kv_heads, a->num_seqs);
    const bool int8 = c->kind == TI_KV_INT8;
    if (c->head_dim == 128) {
        if (int8) launch_decode_d<128, true>(p, rowb, grid, s);
        else launch_decode_d<128, false>(p, rowb, grid, s);
    } else {
        if (int8) launch_decode_d<64, true>(p, rowb, grid, s);
        else launch_decode_d<64, false>(p, rowb, grid, s);
    }
    if (hipGetLastError() != hipSuccess) return TI_ERR_LAUNCH;
    dim3 cgrid(pl.rows, c->kv_heads, a->num_seqs);
    if (c->head_dim == 128) combine_kernel<128><<<cgrid, 64, 0, s>>>(p);
    else combine_kernel<64><<<cgrid, 64, 0, s>>>(p);
    return hipGetLastError() == hipSuccess ? TI_OK : TI_ERR_LAUNCH;
}
