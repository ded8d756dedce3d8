// Split-KV paged decode / verify attention on bf16 MFMA (gfx950), dense bf16 or INT8 cache.
//
// Reference: attention_decode_kernel / decode_body / attention_combine_kernel
// (src/ops/tile/attention.jl:185-245) and its INT8 variant (:68-95, :194-202).
//
// Work decomposition. The G = Hq/Hk query heads that share a KV head, times the n query
// tokens of the step, are packed into M = G*n query rows (row r = g + G t, as the
// reference's packed tile). One work-group (NW = 4 or 8 waves) handles one (sequence, KV
// head, split); a split is a contiguous range of 16-key tiles of the sequence, and the
// waves of the group take every NW-th tile of it, each with its own online-softmax state
// (RS = 2: pairs of waves take the same tiles, each holding half of the rows). The grid
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
//                    registers (same lane layout), A = V^T built by ds_read_b64_tr_b16
//                    from a per-wave row-major V tile in LDS (written with 16-B stores
//                    straight from the coalesced row loads).
//                    O^T's lane layout keeps each lane on its own row, so the rescale by
//                    alpha needs no shuffles.
// INT8 (src/ops/quant.jl:56-72; attention.jl:68-95): a key's scale multiplies its scores
// and a value's scale its probability; queries are multiplied by the keys' smoothing and
// rounded to bf16 (attention.jl:90-95). Both products run on fp16 MFMAs whose int8
// operands cost one byte permute per two values: with u = b ^ 0x80 (= b + 128), the fp16
// bit pattern 0x6400 | u is exactly 1152 + b. The biases come off in fp32: each score
// loses 1152 sum(q), each output row 1152 sum(p) (sum(p) from one more MFMA against a
// tile of ones). A query row enters fp16 as its bf16 values times 2^e (its largest
// magnitude scaled into [2^14, 2^15): exact, but for elements below 2^-28 of the largest),
// and the scores are multiplied back by 2^-e; the probabilities (p <= 1: the running
// max is exact for INT8) times the values' scales enter fp16 rounded to nearest.
//
// At the end the four waves merge their (m, l, O) through LDS and the group writes one
// Float32 partial (acc[D], m, l) per packed row; the combine kernel merges the splits:
// w_s = exp2(m_s - max m), o = sum acc_s w_s / sum l_s w_s.
#pragma once

#include "common.hpp"

using namespace ti;

namespace ti_decode {

typedef short s16x4 __attribute__((ext_vector_type(4)));

struct DecodeParams {
    const uint16_t *q;
    uint16_t *out;
    const uint16_t *kp, *vp;
    const int8_t *lq;
    const float *ls, *smooth;
    const int32_t *positions, *qsl, *bt;
    float *part;
    int *meta;   // flat mode: per sequence {first work-group, pieces}, written by the decode kernel
    int bt_stride, num_pages, P, pshift, Hk, Hq, G, nmax, M, splits, causal;
    int B, flat;   // flat: work-groups per KV head shared by all sequences (0: `splits` each)
    int min_tiles;   // > 0: splits of at least this many 16-key tiles (f32_active_splits)
    float scale_log2;
};

// Flat mode: the W = p.flat work-groups of a KV head are shared out over the B sequences
// in proportion to their 16-key tiles: sequence i gets 1 + (its share of the other W - B),
// the shares cut from the running tile total, so pieces of every sequence are about equally
// long and a long sequence no longer sets the end of the launch. Work-group x belongs to the
// sequence whose range [lo, lo + n) holds x. Computed by every wave from the sequences'
// positions (one lane per sequence, B <= 64) with a wave prefix sum: no extra round trip
// beyond the positions load that every work-group makes anyway. Results are wave-uniform.
struct FlatPiece {
    int b, lo, n, tok0, nb, start;
};
__device__ inline FlatPiece flat_piece(const DecodeParams &p, int x, int lane) {
    int tok0 = 0, nb = 0, st = 0, nt = 0;
    if (lane < p.B) {
        tok0 = p.qsl ? p.qsl[lane] : lane * p.nmax;
        nb = p.qsl ? min(p.qsl[lane + 1] - tok0, p.nmax) : p.nmax;
        if (nb > 0) {
            st = max(p.positions[tok0], 0);
            nt = (st + nb + 15) >> 4;
        }
    }
    int incl = nt;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int v = __shfl_up(incl, d);
        if (lane >= d) incl += v;
    }
    const long long total = __shfl(incl, 63);
    const long long extra = p.flat - p.B;
    const int lo = lane + (total ? (int)((incl - nt) * extra / total) : 0);
    const int hi = lane + 1 + (total ? (int)(incl * extra / total) : 0);
    const unsigned long long m = __ballot(lane < p.B && lo <= x);
    const int b = 63 - __builtin_clzll(m);   // lo grows with the lane; lane 0's lo is 0 <= x
    FlatPiece f;
    f.b = b;
    f.lo = __builtin_amdgcn_readlane(lo, b);
    f.n = __builtin_amdgcn_readlane(hi, b) - f.lo;
    f.tok0 = __builtin_amdgcn_readlane(tok0, b);
    f.nb = __builtin_amdgcn_readlane(nb, b);
    f.start = __builtin_amdgcn_readlane(st, b);
    return f;
}

// Per-wave V tile in LDS: [16 keys][D + 16] bf16, row-major. The row stride (an odd
// multiple of 32 B) puts the 8 rows x 32 B that 32 lanes of a transposing read touch on
// 64 distinct banks; 16 lanes storing one key's row write 256 contiguous bytes.
template <int D>
constexpr int vtile_row() { return D + 16; }
constexpr float RESCALE_LOG2 = 8.0f;

__device__ __forceinline__ void lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// ds_read_b64_tr_b16: within each 16-lane group, lane j receives element (j % 4) of the
// 4 bf16 that lanes j/4, j/4 + 4, j/4 + 8 and j/4 + 12 address.
__device__ __forceinline__ s16x4 lds_tr16(const uint16_t *p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4 *)(__attribute__((address_space(3))) uint16_t *)p);
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// The fp16 bias of the int8 operands: 0x6400 | (b ^ 0x80) is 1152 + b exactly.
constexpr float I8_BIAS = 1152.0f;

// 8 int8 (two words) -> 8 fp16 of 1152 + b: one xor per word, one byte permute per pair
// (bytes 0x64 from the first source, the biased bytes from the second).
__device__ __forceinline__ u32x4 i8x8_to_f16b(uint32_t x, uint32_t y) {
    const uint32_t tx = x ^ 0x80808080u, ty = y ^ 0x80808080u;
    return (u32x4){__builtin_amdgcn_perm(0x64646464u, tx, 0x04010400u),
                   __builtin_amdgcn_perm(0x64646464u, tx, 0x04030402u),
                   __builtin_amdgcn_perm(0x64646464u, ty, 0x04010400u),
                   __builtin_amdgcn_perm(0x64646464u, ty, 0x04030402u)};
}

// S^T += K Q^T on one 32-wide head-dim block: bf16, or fp16 for INT8 caches.
template <bool INT8>
__device__ __forceinline__ f32x4 qk_mfma(u32x4 k, u32x4 q, f32x4 c) {
    if constexpr (INT8)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, k), __builtin_bit_cast(f16x8, q),
                                                      c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(k), as_bf16x8(q), c, 0, 0, 0);
}

// O^T += V^T P^T on one 16-wide head-dim tile: bf16, or fp16 for INT8 caches.
template <bool INT8>
__device__ __forceinline__ f32x4 pv_mfma(s16x4 v, s16x4 pt, f32x4 c) {
    if constexpr (INT8)
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, v), __builtin_bit_cast(f16x4, pt),
                                                     c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v, pt, c, 0, 0, 0);
}

// One 16-key tile's raw loads, held in registers from issue to use (software pipeline).
template <int D, bool INT8>
struct TileRegs {
    static constexpr int NKB = D / 32;
    static constexpr int KPL = 16 * (D / 8) / 64;
    u32x4 k[NKB];          // dense: 8 bf16 per 32-wide block;   INT8: .xy = 8 int8
    u32x4 v[KPL];          // dense: 8 bf16 of key vg*KPL + e;   INT8: .xy = 8 int8
    float sk, sv;          // INT8 scales of this lane's K key
};

// Pool row of key position pos of KV head h. PG16: the 16-key tile lies in one page
// (P a power of two >= 16), so the caller passes the page's first row; otherwise a per-key lookup
// with the position clamped into the sequence (rows past len are never used unmasked).
struct RowMap {
    const int32_t *bt;
    int P, pshift, Hk, h, num_pages, len, bt_stride;
    __device__ __forceinline__ int page_index(int pos) const {
        return pshift >= 0 ? (pos >> pshift) : pos / P;
    }
    __device__ __forceinline__ int page_offset(int pos) const {
        return pshift >= 0 ? (pos & (P - 1)) : pos % P;
    }
    __device__ __forceinline__ long long row(int pos) const {
        pos = min(pos, len - 1);
        const int pg = page_of(bt, page_index(pos), bt_stride, num_pages);
        return ((long long)pg * Hk + h) * P + page_offset(pos);
    }
    // pos wave-uniform, P a power of two: scalar block-table load, shifts only
    __device__ __forceinline__ long long row_s(int pos) const {
        pos = min(pos, len - 1);
        const int pg = page_of_s(bt, pos >> pshift, bt_stride, num_pages);
        return ((long long)pg * Hk + h) * P + (pos & (P - 1));
    }
};

template <int D, bool INT8, bool PG16>
__device__ __forceinline__ void load_tile(TileRegs<D, INT8> &t, const DecodeParams &p,
                                          const RowMap &rm, int j, int r16, int kg, int vg,
                                          int vc, size_t half_q, size_t half_s) {
    constexpr int NKB = TileRegs<D, INT8>::NKB, KPL = TileRegs<D, INT8>::KPL;
    if (PG16) {
        // One page per tile: a wave-uniform 64-bit base plus small per-lane 32-bit offsets
        // (scalar-base addressing, no 64-bit vector math). Keys past len read the last
        // valid key's row, whose finite values meet p = 0 (never stale memory that could
        // hold NaN).
        const long long r0 = rm.row_s(j * 16);
        const int last = rm.len - 1 - j * 16;
        const uint32_t kr = (uint32_t)min(r16, last);
        uint32_t vr[KPL];
#pragma unroll
        for (int e = 0; e < KPL; e++) vr[e] = (uint32_t)min(vg * KPL + e, last);
        // Values are streamed with non-temporal loads: each value row is read once per
        // split, and keeping them out of the caches measured 8-10% faster on bf16 pages and
        // 4% on INT8 pages. Keys keep normal loads (non-temporal keys measured 26% slower on
        // INT8 pages).
        if (!INT8) {
            const uint16_t *kb = p.kp + r0 * D, *vb = p.vp + r0 * D;
#pragma unroll
            for (int i = 0; i < NKB; i++)
                t.k[i] = *reinterpret_cast<const u32x4 *>(kb + (kr * D + i * 32 + kg * 8));
#pragma unroll
            for (int e = 0; e < KPL; e++)
                t.v[e] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(vb + (vr[e] * D + vc * 8)));
        } else {
            const int8_t *kb = p.lq + r0 * D, *vb = p.lq + half_q + r0 * D;
            // keys in 16-B pieces (64 contiguous bytes per row across a lane group, against
            // 32 with 8-B pieces: 1 % faster); score MFMA 2 u + c takes bytes 64 u + 16 kg +
            // 8 c, and the queries' head dimension is gathered in the same order
#pragma unroll
            for (int u = 0; u < NKB / 2; u++) {
                const u32x4 r = *reinterpret_cast<const u32x4 *>(kb + (kr * D + u * 64 + kg * 16));
                t.k[2 * u] = (u32x4){r[0], r[1], 0u, 0u};
                t.k[2 * u + 1] = (u32x4){r[2], r[3], 0u, 0u};
            }
#pragma unroll
            for (int e = 0; e < KPL; e++) {
                const u32x2 r = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(vb + (vr[e] * D + vc * 8)));
                t.v[e] = (u32x4){r[0], r[1], 0u, 0u};
            }
            const float *sb = p.ls + r0;
            t.sk = sb[kr];
            t.sv = sb[half_s + kr];
        }
        return;
    }
    long long krow, vrow[KPL];
    krow = rm.row(j * 16 + r16);
#pragma unroll
    for (int e = 0; e < KPL; e++) vrow[e] = rm.row(j * 16 + vg * KPL + e);
    if (!INT8) {
#pragma unroll
        for (int i = 0; i < NKB; i++)
            t.k[i] = *reinterpret_cast<const u32x4 *>(p.kp + krow * D + i * 32 + kg * 8);
#pragma unroll
        for (int e = 0; e < KPL; e++)
            t.v[e] = *reinterpret_cast<const u32x4 *>(p.vp + vrow[e] * D + vc * 8);
    } else {
#pragma unroll
        for (int u = 0; u < NKB / 2; u++) {
            const u32x4 r = *reinterpret_cast<const u32x4 *>(p.lq + krow * D + u * 64 + kg * 16);
            t.k[2 * u] = (u32x4){r[0], r[1], 0u, 0u};
            t.k[2 * u + 1] = (u32x4){r[2], r[3], 0u, 0u};
        }
#pragma unroll
        for (int e = 0; e < KPL; e++) {
            const uint2 r = *reinterpret_cast<const uint2 *>(p.lq + half_q + vrow[e] * D + vc * 8);
            t.v[e] = (u32x4){r.x, r.y, 0u, 0u};
        }
        t.sk = p.ls[krow];
        t.sv = p.ls[half_s + krow];
    }
}

template <int D, int ROWB, bool INT8, bool PG16, int NW, int RS>
__global__ void __launch_bounds__(NW * 64) decode_kernel(DecodeParams p) {
    constexpr int NKB = D / 32;          // 32-wide head-dim blocks (QK MFMAs per tile)
    constexpr int NDT = D / 16;          // 16-wide head-dim tiles (PV MFMAs per tile)
    constexpr int CPR = D / 8;           // 8-element chunks per V row
    constexpr int KPL = 16 * CPR / 64;   // keys per lane in the V load (4 for D=128)
    constexpr int MP = ROWB * 16;        // padded rows per wave
    constexpr int NKW = NW / RS;         // waves splitting the keys (RS row slices each)

    // Per-wave transposed V tiles during the key loop; afterwards the same LDS holds each
    // wave's (O, m, l) slab for the merge (rows of D + 4 floats, 16-B aligned).
    constexpr int MROW = D + 4;
    constexpr int VROW = vtile_row<D>();
    constexpr int VT_BYTES = NW * 16 * VROW * 2;
    constexpr int SLAB_BYTES = NW * MP * MROW * 4;
    __shared__ __attribute__((aligned(16))) char smem_raw[VT_BYTES > SLAB_BYTES ? VT_BYTES : SLAB_BYTES];
    uint16_t (*vt)[16 * VROW] = reinterpret_cast<uint16_t (*)[16 * VROW]>(smem_raw);
    float *mslab = reinterpret_cast<float *>(smem_raw);

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
    const int r16 = lane & 15, kg = lane >> 4;
    // RS = 2: waves pair up on the same keys, wave w holding rows MP*(w%2) .. + MP.
    const int rslice = RS == 2 ? (w & 1) : 0, kw = RS == 2 ? (w >> 1) : w;
    const int row0 = rslice * MP;
    const int h = blockIdx.y;
    int s, b, nsp, tok0, nb, start;
    size_t unit;   // this work-group's partial slot
    if (p.flat) {
        const FlatPiece f = flat_piece(p, blockIdx.x, lane);
        b = f.b;
        s = blockIdx.x - f.lo;
        nsp = f.n;
        tok0 = f.tok0;
        nb = f.nb;
        start = f.start;
        unit = (size_t)h * p.flat + blockIdx.x;
        if (h == 0 && s == 0 && threadIdx.x == 0) *reinterpret_cast<int2 *>(p.meta + 2 * b) = make_int2(f.lo, f.n);
        if (nb <= 0) return;
    } else {
        s = blockIdx.x;
        b = blockIdx.z;
        nsp = p.splits;
        tok0 = p.qsl ? p.qsl[b] : b * p.nmax;
        nb = p.qsl ? min(p.qsl[b + 1] - tok0, p.nmax) : p.nmax;   // at most max_query_len
        if (nb <= 0) return;
        start = max(p.positions[tok0], 0);   // a negative position reads as 0
        unit = ((size_t)b * p.Hk + h) * p.splits + s;
    }
    const int len = start + nb;
    const int ntiles = (len + 15) >> 4;
    const int per = (ntiles + nsp - 1) / nsp;
    const int j0 = s * per, j1 = min(j0 + per, ntiles);
    const size_t half_q = (size_t)p.num_pages * p.Hk * p.P * D;
    const size_t half_s = (size_t)p.num_pages * p.Hk * p.P;
    const RowMap rm{p.bt + (size_t)b * p.bt_stride, p.P, p.pshift, p.Hk, h, p.num_pages, len, p.bt_stride};
    // Keys up to mask_from are visible to every row; later tiles need the mask.
    const int mask_from = p.causal ? start : len - 1;

    // Query operands (B of S^T = K Q^T): row rb*16 + r16, elements i*32 + kg*8 .. +8.
    // INT8: fp16 of the bf16-rounded q * smooth times 2^e (see the header); qcorr is the
    // row's 1152 sum(q 2^e) that comes off its scores, qsl the score multiplier
    // scale * log2(e) * 2^-e.
    u32x4 qreg[ROWB][NKB];
    int qpos[ROWB];
    float qcorr[ROWB], qsl[ROWB];
#pragma unroll
    for (int rb = 0; rb < ROWB; rb++) {
        const int r = row0 + rb * 16 + r16, t = r / p.G, g = r - t * p.G;
        const bool ok = r < p.M && t < nb;
        qpos[rb] = p.causal && ok ? start + t : len - 1;
        const uint16_t *qr = p.q + ((size_t)(tok0 + t) * p.Hq + h * p.G + g) * D;
        if constexpr (!INT8) {
#pragma unroll
            for (int i = 0; i < NKB; i++)
                qreg[rb][i] = ok ? *reinterpret_cast<const u32x4 *>(qr + i * 32 + kg * 8) : (u32x4){0u, 0u, 0u, 0u};
        } else {
            float qf[NKB][8], amax = 0.0f;
#pragma unroll
            for (int i = 0; i < NKB; i++) {
                const int d0 = (i >> 1) * 64 + kg * 16 + (i & 1) * 8;   // the keys' 16-B loads' order
                const u32x4 raw = ok ? *reinterpret_cast<const u32x4 *>(qr + d0) : (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    // bf16(q * smooth) (attention.jl:90-95), kept as float
                    qf[i][2 * e] = bf2f(f2bf(__uint_as_float(raw[e] << 16) * p.smooth[d0 + 2 * e]));
                    qf[i][2 * e + 1] = bf2f(f2bf(__uint_as_float(raw[e] & 0xffff0000u) * p.smooth[d0 + 2 * e + 1]));
                    amax = fmaxf(amax, fmaxf(fabsf(qf[i][2 * e]), fabsf(qf[i][2 * e + 1])));
                }
            }
            amax = fmaxf(amax, __shfl_xor(amax, 16));
            amax = fmaxf(amax, __shfl_xor(amax, 32));
            // amax * 2^e in [2^14, 2^15): frexp gives amax = f 2^x with f in [0.5, 1)
            const int e2 = amax > 0.0f ? 15 - __builtin_amdgcn_frexp_expf(amax) : 0;
            float qs = 0.0f;
#pragma unroll
            for (int i = 0; i < NKB; i++) {
                u32x4 wv;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const f16x2 hv = __builtin_convertvector(
                        ((f32x2){__builtin_ldexpf(qf[i][2 * e], e2), __builtin_ldexpf(qf[i][2 * e + 1], e2)}), f16x2);
                    qs += (float)hv[0] + (float)hv[1];
                    wv[e] = __builtin_bit_cast(uint32_t, hv);
                }
                qreg[rb][i] = wv;
            }
            qs += __shfl_xor(qs, 16);
            qs += __shfl_xor(qs, 32);
            qcorr[rb] = I8_BIAS * qs;
            qsl[rb] = __builtin_ldexpf(p.scale_log2, -e2);
        }
    }

    f32x4 o[ROWB][NDT];
    f32x4 psum[ROWB];   // INT8: sum of the fp16 probabilities (every element: the row's)
    float m[ROWB], l[ROWB];
#pragma unroll
    for (int rb = 0; rb < ROWB; rb++) {
        m[rb] = NEG_BIG;
        l[rb] = 0.0f;
        psum[rb] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) o[rb][dt] = (f32x4){0.f, 0.f, 0.f, 0.f};
    }

    uint16_t *myvt = vt[w];
    const int vc = lane % CPR, vg = lane / CPR;   // V load: chunk, key group

    auto compute = [&](const TileRegs<D, INT8> &t, int j) {
        // ---- V rows -> row-major LDS tile (INT8: biased fp16, exact) ----
        u32x4 vrows[KPL];
#pragma unroll
        for (int e = 0; e < KPL; e++) vrows[e] = INT8 ? i8x8_to_f16b(t.v[e][0], t.v[e][1]) : t.v[e];
        lds_fence();   // the previous tile's reads of myvt are done before overwriting
#pragma unroll
        for (int e = 0; e < KPL; e++)
            *reinterpret_cast<u32x4 *>(myvt + (vg * KPL + e) * VROW + vc * 8) = vrows[e];
        // ---- S^T = K Q^T ----
        u32x4 kreg[NKB];
#pragma unroll
        for (int i = 0; i < NKB; i++) kreg[i] = INT8 ? i8x8_to_f16b(t.k[i][0], t.k[i][1]) : t.k[i];
        f32x4 sc[ROWB];
#pragma unroll
        for (int rb = 0; rb < ROWB; rb++) {
            sc[rb] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < NKB; i++) sc[rb] = qk_mfma<INT8>(kreg[i], qreg[rb][i], sc[rb]);
        }
        // Scales of this lane's 4 score keys (kg*4 + e), from the lanes that loaded them.
        float skk[4], svk[4];
        if (INT8) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                skk[e] = __shfl(t.sk, kg * 4 + e);
                svk[e] = __shfl(t.sv, kg * 4 + e);
            }
        }
        // ---- online softmax + P^T operands ----
        // Lazy rescaling: m is a reference max that only moves when a tile's max exceeds
        // it by more than RESCALE_LOG2 (then p <= 2^RESCALE_LOG2, safe in bf16 and fp32);
        // l and O always use the same reference, so the result is exact. INT8 moves m
        // with every larger max (p <= 1, so p times a value scale stays within fp16).
        const bool need_mask = j * 16 + 15 > mask_from;
        s16x4 pop[ROWB];
        float x[ROWB][4], mt[ROWB];
        bool grow = false;
#pragma unroll
        for (int rb = 0; rb < ROWB; rb++) {
            mt[rb] = -INFINITY;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float v = sc[rb][e];
                if (INT8) v = (v - qcorr[rb]) * skk[e] * qsl[rb];
                else v *= p.scale_log2;
                if (need_mask) {
                    const int kp = j * 16 + kg * 4 + e;
                    v = (kp <= qpos[rb] && kp < len) ? v : -INFINITY;
                }
                x[rb][e] = v;
                mt[rb] = fmaxf(mt[rb], v);
            }
            grow |= mt[rb] > m[rb] + (INT8 ? 0.0f : RESCALE_LOG2);
        }
        if (__any(grow)) {
#pragma unroll
            for (int rb = 0; rb < ROWB; rb++) {
                float t2 = fmaxf(mt[rb], __shfl_xor(mt[rb], 16));
                t2 = fmaxf(t2, __shfl_xor(t2, 32));
                const float mn = fmaxf(m[rb], t2);
                const float alpha = fast_exp2(m[rb] - mn);
                m[rb] = mn;
                l[rb] *= alpha;
                if (INT8) psum[rb] *= alpha;
#pragma unroll
                for (int dt = 0; dt < NDT; dt++) o[rb][dt] *= alpha;
            }
        }
#pragma unroll
        for (int rb = 0; rb < ROWB; rb++) {
            float ps = 0.0f, pe[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                pe[e] = fast_exp2(x[rb][e] - m[rb]);
                ps += pe[e];
                if (INT8) pe[e] *= svk[e];
            }
            l[rb] += ps;
            if (INT8) {
                const f16x2 h0 = __builtin_convertvector(((f32x2){pe[0], pe[1]}), f16x2);
                const f16x2 h1 = __builtin_convertvector(((f32x2){pe[2], pe[3]}), f16x2);
                pop[rb] = __builtin_bit_cast(s16x4, (u32x2){__builtin_bit_cast(uint32_t, h0),
                                                            __builtin_bit_cast(uint32_t, h1)});
                // the row's sum of these fp16 probabilities, for the values' bias
                const s16x4 ones = __builtin_bit_cast(s16x4, (u32x2){0x3c003c00u, 0x3c003c00u});
                psum[rb] = pv_mfma<true>(ones, pop[rb], psum[rb]);
            } else {
                pop[rb] = __builtin_bit_cast(s16x4, (u32x2){pack_bf16x2(pe[0], pe[1]), pack_bf16x2(pe[2], pe[3])});
            }
        }
        // ---- O^T += V^T P^T ----
        lds_fence();   // this tile's V^T is in LDS
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            const s16x4 a = lds_tr16(myvt + (4 * kg + (r16 >> 2)) * VROW + dt * 16 + 4 * (r16 & 3));
#pragma unroll
            for (int rb = 0; rb < ROWB; rb++) o[rb][dt] = pv_mfma<INT8>(a, pop[rb], o[rb][dt]);
        }
    };

    // Two register sets, ping-ponged: the next group of TPI tiles is loading while the
    // current one computes. INT8 tiles are half the bytes, so INT8 waves take more tiles
    // per step: three for 16-row waves (configs[3], Llama-3-8B B = 8 x 32768, same process:
    // 96.5-98.6 us with two, 94.2-94.7 with three, 100-102 with four, 104-106 with one),
    // two for 32-row waves, whose accumulators leave less room. The prefetch is issued
    // unconditionally (past the last tile it re-reads that tile, unused) so the count of
    // loads in flight is static and each wait covers only the tiles in use.
    constexpr int TPI = INT8 ? (ROWB == 1 ? 3 : 2) : 1;
    constexpr int STRIDE = NKW * TPI;
    TileRegs<D, INT8> ta[TPI], tb[TPI];
    auto ld = [&](TileRegs<D, INT8> (&t)[TPI], int jj) {
#pragma unroll
        for (int e = 0; e < TPI; e++)
            load_tile<D, INT8, PG16>(t[e], p, rm, min(jj + e, j1 - 1), r16, kg, vg, vc, half_q, half_s);
    };
    auto run = [&](const TileRegs<D, INT8> (&t)[TPI], int jj) {
#pragma unroll
        for (int e = 0; e < TPI; e++)
            if (jj + e < j1) compute(t[e], jj + e);
    };
    int j = j0 + TPI * kw;
    if (j < j1) {
        ld(ta, j);
        while (true) {
            ld(tb, j + STRIDE);
            run(ta, j);
            j += STRIDE;
            if (j >= j1) break;
            ld(ta, j + STRIDE);
            run(tb, j);
            j += STRIDE;
            if (j >= j1) break;
        }
    }

    // INT8: the values' bias, 1152 times each row's sum of fp16 probabilities
    if constexpr (INT8) {
#pragma unroll
        for (int rb = 0; rb < ROWB; rb++)
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) o[rb][dt] -= I8_BIAS * psum[rb];
    }

    // ---- merge the waves' states (same rows, disjoint keys) through LDS slabs ----
#pragma unroll
    for (int rb = 0; rb < ROWB; rb++) {
        l[rb] += __shfl_xor(l[rb], 16);
        l[rb] += __shfl_xor(l[rb], 32);
    }
    __syncthreads();   // every wave is done with its V tile
#pragma unroll
    for (int rb = 0; rb < ROWB; rb++) {
        float *my = mslab + ((size_t)w * MP + rb * 16 + r16) * MROW;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
            *reinterpret_cast<f32x4 *>(my + dt * 16 + kg * 4) = o[rb][dt];
        if (kg == 0) {
            my[D] = m[rb];
            my[D + 1] = l[rb];
        }
    }
    __syncthreads();
    for (int item = threadIdx.x; item < p.M * (D / 4); item += NW * 64) {
        const int r = item / (D / 4), d4 = (item % (D / 4)) * 4;
        const int rs = RS == 2 ? r / MP : 0, rr = r - rs * MP;   // row slice, row in slab
        float mx = NEG_BIG;
#pragma unroll
        for (int wi = 0; wi < NKW; wi++) mx = fmaxf(mx, mslab[((size_t)(wi * RS + rs) * MP + rr) * MROW + D]);
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        float lsum = 0.0f;
#pragma unroll
        for (int wi = 0; wi < NKW; wi++) {
            const float *src = mslab + ((size_t)(wi * RS + rs) * MP + rr) * MROW;
            const float wgt = fast_exp2(src[D] - mx);
            lsum += src[D + 1] * wgt;
            acc += *reinterpret_cast<const f32x4 *>(src + d4) * wgt;
        }
        if (nsp == 1) {
            // One split: this group saw every key; normalize and write the output rows.
            const int t = r / p.G, g = r - t * p.G;
            if (t < nb) {
                const float inv = 1.0f / lsum;
                uint16_t *o16 = p.out + ((size_t)(tok0 + t) * p.Hq + h * p.G + g) * D + d4;
                *reinterpret_cast<u32x2 *>(o16) = (u32x2){pack_bf16x2(acc[0] * inv, acc[1] * inv),
                                                          pack_bf16x2(acc[2] * inv, acc[3] * inv)};
            }
        } else {
            // The split's partial: part[unit][r][D + 2] = (acc, m, l).
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

}  // namespace ti_decode

