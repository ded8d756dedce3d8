// Paged causal / chunked / non-causal prefill attention on bf16 MFMA (gfx950), dense bf16
// or INT8 cache.
//
// Reference: attention_prefill_kernel / prefill_body (src/ops/tile/attention.jl:130-177)
// and attention_prefill_int8_kernel (:139-147). Query t of the step sits at position
// start + t (start = positions of the sequence's first query, read on the device) and sees
// keys 0 .. start + t; with causal = 0 it sees all start + n keys (attention.jl:155-157).
// Chunked prefill over a cached prefix is the same kernel with start > 0.
//
// Work decomposition. A work-group is NG key groups of WPG waves. Each wave owns 32
// packed query rows of one (sequence, KV head) — the G query heads of the KV head times
// consecutive positions, row r = g + G t as in the decode kernel — so every K/V tile
// loaded into LDS serves all G heads. The key groups split the q-tile's key tiles and
// merge through LDS at the end; with key splits across work-groups (small grids), each
// work-group covers a contiguous range of key tiles and writes Float32 partials that the
// combine kernel merges. Query tiles are issued heaviest first (the last positions see
// the most keys). Keys stream through LDS in 32-key tiles, double-buffered: global loads
// of later tiles are in flight while the waves compute the current one.
//
// Per wave (32 rows) and 32-key tile:
//   S^T = K Q^T        D/16 v_mfma_f32_32x32x16_bf16 (K rows from LDS as the A operand)
//   online softmax     exp2 domain, lane-local per row + one xor shuffle for the max
//   O^T += V^T P^T     2 D/32 v_mfma_f32_32x32x16_bf16; P^T is the S^T registers rounded
//                      to bf16, V^T is read from the row-major V tile by transposing
//                      LDS reads (ds_read_b64_tr_b16).
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
    float *part;                       // split partials [B][Hk][splits][M][D + 2]
    int bt_stride, num_pages, P, pshift, Hk, Hq, G, gshift, TQ, nmax, qtiles, causal, splits, M;
    float scale_log2;
};

constexpr int KT = 32;                 // keys per LDS tile
constexpr bool PAIR_BY_DEFAULT = true; // AUTO / PREFILL take paired q-tiles where they apply
constexpr bool R16_BY_DEFAULT = true;  // paired q-tiles on 16-row waves (prefill16_kernel)
constexpr float RESCALE_LOG2 = 8.0f;   // lazy-rescale threshold (see the decode kernel)

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

// One key group's LDS: K and V tiles row-major, double-buffered. Row strides (in bf16)
// D + 8 for K (16-B reads by 16 consecutive lanes of 16 keys hit 64 distinct banks) and
// D + 32 for V: a transposing read by 32 lanes covers 4 rows x 64 B, and rows 16 banks
// apart make those 256 B bank-disjoint.
template <int D>
struct Smem {
    static constexpr int KROW = D + 8;
    static constexpr int VROW = D + 32;
    uint16_t k[2][KT * KROW];
    uint16_t v[2][KT * VROW];
    float sk[2][KT], sv[2][KT];
};

// Direct-load variant (bf16 dense cache, D = 128, pages of 2^k >= 16 tokens): one key
// group's K and V tiles, double-buffered, filled by global -> LDS loads
// (global_load_lds_dwordx4: no staging registers, no LDS store instructions). Rows are
// unpadded, since each load instruction writes 1 KB (4 rows) contiguously; the 16-byte
// chunks of a row are XOR-swizzled by the key instead (K: slot = chunk ^ (key % 16), V:
// slot = chunk ^ 4 (key % 4)), so 16-key K reads and 4-row transposing V reads fall on
// distinct banks.
struct DlSmem {
    uint16_t k[2][KT * 128];
    uint16_t v[2][KT * 128];
};

// vmcnt(0): this wave's direct global -> LDS loads have landed. Issued explicitly before
// the barrier that publishes a tile: the compiler's own waits for direct loads do not
// cover reads of the buffer by other waves.
__device__ __forceinline__ void wait_direct_loads() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// Pool row of key position pos (clamped into the step's keys: rows past kend hold finite
// cache data whose probabilities are masked to 0).
__device__ __forceinline__ long long key_row(const PrefillParams &p, const int32_t *bt, int h,
                                             int pos, int kend) {
    pos = min(pos, kend - 1);
    const int idx = p.pshift >= 0 ? pos >> p.pshift : pos / p.P;
    const int off = p.pshift >= 0 ? pos & (p.P - 1) : pos % p.P;
    const int pg = page_of(bt, idx, p.bt_stride, p.num_pages);
    return ((long long)pg * p.Hk + h) * p.P + off;
}

// Rows of a tile's keys. PG16 (P a power of two >= 16): each 16-key half of the tile lies
// in one page, found with a scalar block-table load and shifts (no division); key k's row
// is half_row[k / 16] + k % 16. Otherwise a per-key lookup (vector loads).
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
                const int idx = pos >> pp.pshift, off = pos & (pp.P - 1);   // PG16: P is 2^pshift
                const int pg = page_of_s(btp, idx, pp.bt_stride, pp.num_pages);
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

// One tile's K and V (and INT8 scales) in registers between the global load and the LDS
// store, for one thread of a GT-thread key group: chunk c = gtid + GT u of the tile's
// KT x (D/8) 16-byte chunks (INT8: 8-byte chunks).
template <int D, bool INT8, int GT>
struct Stage {
    static constexpr int CH = KT * D / 8;
    static constexpr int PER = (CH + GT - 1) / GT;
    u32x4 k[PER], v[PER];
    float s;
};

// Page ids (0-based, clamped into the pool) of the two 16-key halves of tile kt, read with
// scalar loads; fetched one tile ahead of use so their latency hides behind compute.
struct TilePages {
    int pg[2];
};

// The block-table entries (1-based page ids, unclamped) of tile kt's two 16-key halves, as
// scalar loads: their consumer clamps them (clamp_page), so the wait for these loads can sit
// where the pages are used, a step later, instead of right after the loads.
__device__ __forceinline__ TilePages raw_pages(const PrefillParams &p, const int32_t *bt, int kt) {
    TilePages tp;
#pragma unroll
    for (int x = 0; x < 2; x++) {
        const int idx = min((kt * KT + 16 * x) >> p.pshift, p.bt_stride - 1);   // PG16: P = 2^pshift; kt >= 0
        tp.pg[x] = sload(bt, idx);
    }
    return tp;
}

__device__ __forceinline__ TilePages tile_pages(const PrefillParams &p, const int32_t *bt, int kt) {
    TilePages tp;
#pragma unroll
    for (int x = 0; x < 2; x++) {
        const int pos = kt * KT + 16 * x;
        tp.pg[x] = page_of_s(bt, pos >> p.pshift, p.bt_stride, p.num_pages);   // PG16: P = 2^pshift
    }
    return tp;
}

template <int D, bool INT8, bool PG16, int GT>
__device__ __forceinline__ void load_tile(Stage<D, INT8, GT> &st, const PrefillParams &p,
                                          const int32_t *bt, int h, int kt, int kend, int gtid,
                                          const TilePages &tp) {
    const size_t half_q = (size_t)p.num_pages * p.Hk * p.P * D;
    const size_t half_s = (size_t)p.num_pages * p.Hk * p.P;
    constexpr int CPR = D / 8;
    constexpr int KPU = GT / CPR;              // keys covered by one chunk round (GT % CPR == 0)
    if (PG16) {
        // Each 16-key half of the tile lies in one page: the page's row base is scalar and
        // chunk u of this thread sits at a loop-invariant offset from it. Keys past kend
        // read stale-but-allocated rows of the same page (their scores are masked and their
        // values zeroed when the tile is stored).
        long long base[2];
#pragma unroll
        for (int x = 0; x < 2; x++) {
            const int pos = kt * KT + 16 * x;
            const int off = pos & (p.P - 1);
            base[x] = (((long long)tp.pg[x] * p.Hk + h) * p.P + off) * D;
        }
#pragma unroll
        for (int u = 0; u < Stage<D, INT8, GT>::PER; u++) {
            const int key = gtid / CPR + KPU * u, ch = gtid % CPR;
            const long long e0 = base[key >> 4] + (key & 15) * D + ch * 8;   // key >> 4 folds per u
            if (!INT8) {
                st.k[u] = *reinterpret_cast<const u32x4 *>(p.kp + e0);
                st.v[u] = *reinterpret_cast<const u32x4 *>(p.vp + e0);
            } else {
                const uint2 a = *reinterpret_cast<const uint2 *>(p.lq + e0);
                const uint2 b = *reinterpret_cast<const uint2 *>(p.lq + half_q + e0);
                st.k[u] = (u32x4){a.x, a.y, 0u, 0u};
                st.v[u] = (u32x4){b.x, b.y, 0u, 0u};
            }
        }
        if (INT8 && gtid < 2 * KT) {
            const int key = gtid % KT;
            const long long row = base[key >> 4] / D + (key & 15);
            st.s = gtid < KT ? p.ls[row] : p.ls[half_s + row];
        }
        return;
    }
    const TileRows<PG16> tr(p, bt, h, kt, kend);
#pragma unroll
    for (int u = 0; u < Stage<D, INT8, GT>::PER; u++) {
        const int c = gtid + GT * u, key = c / CPR, ch = c % CPR;
        if (c < Stage<D, INT8, GT>::CH) {
            const long long row = tr.row(key);
            if (!INT8) {
                st.k[u] = *reinterpret_cast<const u32x4 *>(p.kp + row * D + ch * 8);
                st.v[u] = *reinterpret_cast<const u32x4 *>(p.vp + row * D + ch * 8);
            } else {
                const uint2 a = *reinterpret_cast<const uint2 *>(p.lq + row * D + ch * 8);
                const uint2 b = *reinterpret_cast<const uint2 *>(p.lq + half_q + row * D + ch * 8);
                st.k[u] = (u32x4){a.x, a.y, 0u, 0u};
                st.v[u] = (u32x4){b.x, b.y, 0u, 0u};
            }
        }
    }
    if (INT8 && gtid < 2 * KT) {
        const long long row = tr.row(gtid % KT);
        st.s = gtid < KT ? p.ls[row] : p.ls[half_s + row];
    }
}

__device__ __forceinline__ u32x4 i8x8_to_bf16x8(uint32_t x, uint32_t y) {
    u32x4 r;
    uint32_t a, b, c, d;
    i8x4_to_bf16(x, a, b);
    i8x4_to_bf16(y, c, d);
    r[0] = a; r[1] = b; r[2] = c; r[3] = d;
    return r;
}

template <int D, bool INT8, int GT>
__device__ __forceinline__ void store_tile(const Stage<D, INT8, GT> &st, Smem<D> &sm, int buf, int gtid,
                                           int valid_keys) {
    constexpr int CPR = D / 8;
    const bool partial = valid_keys < KT;      // wave-uniform: only the last tile
#pragma unroll
    for (int u = 0; u < Stage<D, INT8, GT>::PER; u++) {
        const int c = gtid + GT * u, key = c / CPR, ch = c % CPR;
        if (c < Stage<D, INT8, GT>::CH) {
            const u32x4 kv = INT8 ? i8x8_to_bf16x8(st.k[u][0], st.k[u][1]) : st.k[u];
            const u32x4 vv = INT8 ? i8x8_to_bf16x8(st.v[u][0], st.v[u][1]) : st.v[u];
            *reinterpret_cast<u32x4 *>(&sm.k[buf][key * Smem<D>::KROW + ch * 8]) = kv;
            if (partial) {
                // Only the last tile has keys past the step's end (their values meet p = 0 and
                // must be finite); the empty asm keeps this a real branch, so full tiles skip
                // the selects.
                asm volatile("");
                const uint32_t keep = key < valid_keys ? ~0u : 0u;
                *reinterpret_cast<u32x4 *>(&sm.v[buf][key * Smem<D>::VROW + ch * 8]) = vv & keep;
            } else {
                *reinterpret_cast<u32x4 *>(&sm.v[buf][key * Smem<D>::VROW + ch * 8]) = vv;
            }
        }
    }
    if (INT8 && gtid < 2 * KT) {
        if (gtid < KT) sm.sk[buf][gtid] = st.s;
        else sm.sv[buf][gtid - KT] = st.s;
    }
}

__device__ __forceinline__ u32x2 lds_tr16(const uint16_t *p) {
    const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4 *)(__attribute__((address_space(3))) uint16_t *)p);
    return __builtin_bit_cast(u32x2, v);
}

// A work-group = NG key groups of WPG waves. Each wave owns 32 packed query rows
// (row = g + G t, the G heads of one KV head times consecutive positions), so a group
// covers 32 WPG rows; every group holds the same rows and walks the key tiles
// kt = grp, grp + NG, ... through its own double-buffered LDS tiles with a two-deep
// register prefetch; the groups' states merge through LDS at the end.
//
// Per wave and 32-key tile (lane l: row l % 32, k-group kg = l / 32):
//   S^T = K Q^T     D/16 v_mfma_f32_32x32x16_bf16; A = K rows from LDS (16 B per lane),
//                   B = Q^T in registers. Lane holds 16 scores of its row, keys
//                   8 (e/4) + 4 kg + e%4.
//   softmax         exp2 domain, lane-local, one xor-32 shuffle for the row max; lazy rescale.
//   O^T += V^T P^T  2 x D/32 v_mfma_f32_32x32x16_bf16; B = P^T is the score registers
//                   (keys 0-15, then 16-31), A = V^T built by ds_read_b64_tr_b16 from the
//                   row-major V tile (two 8-B transposing reads per operand).
//
// PAIR (causal, unsplit, direct loads, two waves per group): the two waves of a key group
// own two different 32-row q-tiles instead of one 64-row q-tile: a heavy one from the end
// of the step (wave 0 of the group) and a light one from its start (wave 1), q-tiles
// qtiles - 1 - y and y of work-group y, so every work-group carries the same causal work
// (the light tile's keys are the first tiles of the heavy one's: they share the LDS
// tiles). Waves 0-3 are the groups' heavy waves, 4-7 the light ones, one of each per SIMD;
// a light wave past its keys only issues its share of the tile loads.
template <int D, bool INT8, bool PG16, int WPG, int NG, bool DL, bool PAIR = false>
__global__ void __launch_bounds__(64 * WPG * NG) prefill_kernel(PrefillParams p) {
    static_assert(!DL || (!INT8 && PG16 && D == 128 && (WPG == 2 || WPG == 4)), "direct loads: bf16, D 128, 2^k pages");
    static_assert(!PAIR || (DL && WPG == 2 && NG == 4), "paired q-tiles: direct loads, 2 x 4 waves");
    constexpr int NQB = D / 16;          // QK MFMAs (16 head-dim elements each)
    constexpr int NDB = D / 32;          // 32-row output blocks of O^T
    constexpr int GT = 64 * WPG;         // threads per key group
    // direct loads: waves per 16-key page half, load instructions per wave and half
    constexpr int HW = WPG / 2 > 0 ? WPG / 2 : 1, NQ = 8 / WPG;
    constexpr int SMEM = DL ? (int)sizeof(DlSmem) * NG : (int)sizeof(Smem<D>) * NG;
    constexpr int RPG = 32 * WPG;        // packed rows per group
    constexpr int MROW = D + 4;          // merge slab row: O[D], m, l, pad (16-B aligned)
    constexpr int MERGE = NG > 1 ? NG * RPG * MROW * 4 : 0;
    __shared__ __attribute__((aligned(16))) char smem_raw[SMEM > MERGE ? SMEM : MERGE];
    Smem<D> *smg = reinterpret_cast<Smem<D> *>(smem_raw);
    float *mslab = reinterpret_cast<float *>(smem_raw);

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
    const int grp = PAIR ? w % NG : w / WPG, wl = PAIR ? w / NG : w % WPG, gtid = threadIdx.x % GT;
    const int r32 = lane & 31, kg = lane >> 5;
    // Grid (Hk, qtiles, B): consecutive work-groups (spread round-robin over the 8 XCDs)
    // belong to different KV heads, so each head's K/V stays in one XCD's L2.
    const int h = blockIdx.x;
    // PAIR: qt is the heavy q-tile (it bounds the work-group's keys), qtw this wave's.
    const int qt = PAIR ? p.qtiles - 1 - (int)blockIdx.y : p.qtiles - 1 - (int)blockIdx.y / p.splits;   // heaviest tiles first
    const int qt_light = PAIR ? (int)blockIdx.y : qt;
    const int qtw = PAIR && wl == 1 ? qt_light : qt;
    const int split = PAIR ? 0 : (int)blockIdx.y % p.splits;
    const int b = blockIdx.z;
    const int tok0 = p.qsl ? sload(p.qsl, b) : b * p.nmax;
    const int nb = p.qsl ? min(sload(p.qsl, b + 1) - tok0, p.nmax) : p.nmax;   // at most max_query_len
    const int t_first = qt * p.TQ;
    if (qt_light * p.TQ >= nb) return;
    const int t_first_w = qtw * p.TQ;
    const int32_t *bt = p.bt + (size_t)b * p.bt_stride;
    // Loads that do not depend on the step's positions go out first, so their latency
    // overlaps the positions load: the queries and, when keys are not split, the page ids
    // of the group's first tile (tile grp; re-fetched below in the rare case that the
    // q-tile has fewer key tiles than groups).
    // This lane's query row (B operand of S^T = K Q^T): elements i*16 + kg*8 .. +8.
    const int r = wl * 32 + r32;                    // the row's place in the group's slab
    const int rw = PAIR ? r32 : r, tl = rw / p.G, g = rw - tl * p.G, t = t_first_w + tl;
    // PAIR with an odd count of q-tiles: the middle one pairs with itself (its light wave idles)
    const bool row_ok = tl < p.TQ && t < nb && !(PAIR && wl == 1 && qt_light == qt);
    bf16x8 qreg[NQB];
    {
        const uint16_t *qr = p.q + ((size_t)(tok0 + (row_ok ? t : 0)) * p.Hq + h * p.G + g) * D;
#pragma unroll
        for (int i = 0; i < NQB; i++) {
            const int d0 = i * 16 + kg * 8;
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

    TilePages spec{};
    if constexpr (DL) {
        if (p.splits == 1) spec = raw_pages(p, bt, grp);
    }
    const int start = max(sload(p.positions, nb > 0 ? tok0 : 0), 0), len = start + nb;   // a negative position reads as 0
    const int qpos = p.causal && row_ok ? start + t : len - 1;
    const int t_last = min(t_first + p.TQ, nb) - 1;
    const int kend = p.causal ? start + t_last + 1 : len;
    // this wave's own keys (PAIR: the light wave's end before the work-group's)
    const int kend_w = PAIR && p.causal ? start + min(t_first_w + p.TQ, nb) : kend;
    const int kt_hi_w = (kend_w + KT - 1) / KT;
    const int nkt = (kend + KT - 1) / KT;
    // This work-group's split: key tiles [kt_lo, kt_hi) of the q-tile's nkt.
    const int per = (nkt + p.splits - 1) / p.splits;
    const int kt_lo = min(split * per, nkt), kt_hi = min(kt_lo + per, nkt);
    const int steps = (kt_hi - kt_lo + NG - 1) / NG;       // same for every group
    const size_t unit = ((size_t)b * p.Hk + h) * p.splits + split;
    Smem<D> &sm = smg[grp];
    DlSmem &dsm = reinterpret_cast<DlSmem *>(smem_raw)[grp];
    const int mask_from = p.causal ? start + t_first_w : len - 1;
    if (steps == 0) {
        // A split with no keys (short sequence): neutral partials (m = -big, l = 0, acc = 0)
        // that the combine weights to zero.
        constexpr int RPGW = 32 * WPG;
        for (int idx = threadIdx.x; idx < RPGW * (D + 2); idx += 64 * WPG * NG) {
            const int rr = idx / (D + 2), c = idx - rr * (D + 2);
            const int ttl = rr / p.G, gg = rr - ttl * p.G, tt = t_first + ttl;
            if (ttl < p.TQ && tt < nb)
                p.part[(unit * p.M + (size_t)tt * p.G + gg) * (D + 2) + c] = c == D ? NEG_BIG : 0.0f;
        }
        return;
    }

    f32x16 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; db++)
#pragma unroll
        for (int e = 0; e < 16; e++) o[db][e] = 0.0f;
    float m = NEG_BIG, l = 0.0f;

    // transposing-read address parts of this lane: 16-lane group c = lane / 16
    const int c16 = lane >> 4, s16 = lane & 15;
    const int tr_row = 4 * (c16 >> 1) + (s16 >> 2), tr_col = 16 * (c16 & 1) + 4 * (s16 & 3);

    auto compute = [&](int kt, int buf, auto &&issue_loads) {
        if constexpr (!DL) issue_loads();
        if constexpr (PAIR) {
            // a light wave past its keys: its share of the next tile's loads only
            if (kt >= kt_hi_w) {
                issue_loads();
                return;
            }
        }
        // One accumulation chain: dependent v_mfma_f32_32x32x16_bf16 issue back to back
        // (31 cycles each, measured), and a second chain would cost 16 VALU adds.
        f32x16 sc;
#pragma unroll
        for (int e = 0; e < 16; e++) sc[e] = 0.0f;
        // All K reads go out before the first score MFMA (one LDS latency per tile instead
        // of one per MFMA pair); the next tile's global loads are spread between the MFMAs
        // so the CU's load path drains while the matrix cores run.
        u32x4 ka[NQB];
        u32x4 va[NDB][2];   // direct loads: this tile's V^T operands, read before the next loads
        if constexpr (DL) {
            // Every LDS read of this tile goes out before the next tile's loads into the
            // other buffer, so no read of this step waits for those loads. K: chunk 2 i + kg
            // of key r32 sits in slot (2 i + kg) ^ (r32 % 16); V: rows tr_row + 16 hh (+ 8)
            // all have row % 4 = tr_row % 4, one swizzle per lane.
            const uint16_t *krow = &dsm.k[buf][r32 * D];
#pragma unroll
            for (int i = 0; i < NQB; i++)
                ka[i] = *reinterpret_cast<const u32x4 *>(krow + (((2 * i + kg) ^ (r32 & 15)) * 8));
            const uint16_t *vb = &dsm.v[buf][tr_row * D + (tr_col & 7)];
            const int sw = 4 * (tr_row & 3), c0 = tr_col >> 3;
#pragma unroll
            for (int db = 0; db < NDB; db++)
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    const int col = ((c0 + 4 * db) ^ sw) * 8;
                    const u32x2 lo = lds_tr16(vb + (16 * hh) * D + col);
                    const u32x2 hi = lds_tr16(vb + (16 * hh + 8) * D + col);
                    va[db][hh] = (u32x4){lo[0], lo[1], hi[0], hi[1]};
                }
            issue_loads();
        } else {
            const uint16_t *krow = &sm.k[buf][r32 * Smem<D>::KROW + kg * 8];
#pragma unroll
            for (int i = 0; i < NQB; i++) ka[i] = *reinterpret_cast<const u32x4 *>(krow + i * 16);
        }
#pragma unroll
        for (int i = 0; i < NQB; i++)
            sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(ka[i]), qreg[i], sc, 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x0100, DL ? NQB + 4 * NDB : NQB, 0);   // all K (and V) reads
#pragma unroll
        for (int i = 0; i < NQB; i++) {
            __builtin_amdgcn_sched_group_barrier(0x0020, 1, 0);   // one global load
            __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);   // one MFMA
        }
        // Online softmax in the exp2 domain: p = exp2(s * scale - m) with m the running
        // (scaled) reference max; the tile max is taken on raw scores (scale > 0).
        // A tile past this group's keys (its last step) runs the score stage on whatever
        // the buffer holds, fully masked, so the next loads and the score MFMAs share one
        // scheduling region; its PV stage is skipped.
        const bool valid = kt < (PAIR ? kt_hi_w : kt_hi);
        const bool need_mask = !valid || kt * KT + KT - 1 > mask_from;
        // INT8: the scales of this lane's 16 score keys, 8 q + 4 kg + (0..3) for q = 0..3,
        // as four 16-B reads per array
        f32x4 skq[4], svq[4];
        if constexpr (INT8) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                skq[q] = *reinterpret_cast<const f32x4 *>(&sm.sk[buf][8 * q + 4 * kg]);
                svq[q] = *reinterpret_cast<const f32x4 *>(&sm.sv[buf][8 * q + 4 * kg]);
            }
        }
        float x[16];
        float mt = -INFINITY;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int key = 8 * (e >> 2) + 4 * kg + (e & 3);
            float v = sc[e];
            if constexpr (INT8) v *= skq[e >> 2][e & 3];
            if (need_mask) {
                const int kpos = kt * KT + key;
                v = (valid && kpos <= qpos && kpos < kend_w) ? v : -INFINITY;
            }
            x[e] = v;
            mt = fmaxf(mt, v);
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
            if constexpr (INT8) pe[e] *= svq[e >> 2][e & 3];
        }
        l += ps;
        bf16x8 pb[2];
#pragma unroll
        for (int hh = 0; hh < 2; hh++)
            pb[hh] = as_bf16x8((u32x4){pack_bf16x2(pe[8 * hh + 0], pe[8 * hh + 1]), pack_bf16x2(pe[8 * hh + 2], pe[8 * hh + 3]),
                                       pack_bf16x2(pe[8 * hh + 4], pe[8 * hh + 5]), pack_bf16x2(pe[8 * hh + 6], pe[8 * hh + 7])});
        if (!valid) return;
        if constexpr (DL) {
#pragma unroll
            for (int db = 0; db < NDB; db++)
#pragma unroll
                for (int hh = 0; hh < 2; hh++)
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(va[db][hh]), pb[hh], o[db], 0, 0, 0);
        } else {
            const uint16_t *vb = &sm.v[buf][tr_row * Smem<D>::VROW + tr_col];
#pragma unroll
            for (int db = 0; db < NDB; db++)
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    const u32x2 lo = lds_tr16(vb + (16 * hh) * Smem<D>::VROW + 32 * db);
                    const u32x2 hi = lds_tr16(vb + (16 * hh + 8) * Smem<D>::VROW + 32 * db);
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8((u32x4){lo[0], lo[1], hi[0], hi[1]}),
                                                                   pb[hh], o[db], 0, 0, 0);
                }
        }
    };

    auto tile_of = [&](int i) { return kt_lo + grp + NG * i; };
    if constexpr (DL) {
        // A tile's page half x (keys 16 x .. 16 x + 15) is 4 load instructions for K and 4
        // for V; instruction q4 writes 1 KB = keys 4 q4 + lane / 16, slot lane % 16 of the
        // half. Wave wl of the group issues NQ = 8 / WPG of them: half wl / (WPG / 2),
        // instructions NQ (wl % (WPG / 2)) .. + NQ. Step i: wait for this wave's loads of
        // tile i, barrier (every wave's loads of tile i have landed and every wave is done
        // with the other buffer), issue tile i + 1 into the other buffer, compute tile i.
        const int dx = wl / HW, q0 = NQ * (wl % HW);
        const int ksub = lane >> 4, slot = lane & 15;
        // byte offsets of this lane's chunk in each of the wave's instructions of a full
        // half (loop-invariant; indexed by the unrolled u only, so they stay in registers;
        // sized for the most instructions per wave, 4: the host compilation pass drops
        // the kernel's launch stub when a lambda captures an array whose bound depends on
        // a template parameter)
        uint32_t koff[4], voff[4];
#pragma unroll
        for (int u = 0; u < NQ; u++) {
            const int key = 4 * (q0 + u) + ksub;
            koff[u] = (uint32_t)(key * D + ((slot ^ key) * 8)) * 2u;
            voff[u] = (uint32_t)(key * D + ((slot ^ (4 * ksub)) * 8)) * 2u;
        }
        // Value rows load with cache-policy bits 3 (sc0 sc1), keys with the default policy:
        // measured 12% faster on decode-like verify steps (few queries per sequence, every
        // row read once) and unchanged on long prompts, whose q-tiles re-read the rows.
        // element offsets: page pg, row r of KV head h at pg * pstride + hoff + r * D (the
        // page ids arrive raw from the block table and are clamped here)
        const uint32_t pstride = (uint32_t)p.Hk * p.P * D, hoff = (uint32_t)h * p.P * D;
        auto page_base = [&](int raw, int pos) -> uint64_t {
            return (uint64_t)(uint32_t)clamp_page(raw, p.num_pages) * pstride + hoff + (uint32_t)((pos & (p.P - 1)) * D);
        };
        auto dl_load = [&](int kt, int buf, const TilePages &tp) {
            typedef __attribute__((address_space(3))) void *lds_ptr;
            const int pos0 = kt * KT, last = kend - 1 - pos0;   // >= 0 for every tile loaded
            uint16_t *kd = &dsm.k[buf][dx * 2048], *vd = &dsm.v[buf][dx * 2048];
            if (last >= KT - 1) {
                // every key of the tile is a step key: a scalar base and fixed offsets
                // (selects, not indexing: a dynamically indexed array would be placed in LDS,
                // whose accesses then wait for every pending direct load)
                const uint64_t base = page_base(dx ? tp.pg[1] : tp.pg[0], pos0 + 16 * dx);
                const char *kb = reinterpret_cast<const char *>(p.kp + base);
                const char *vb = reinterpret_cast<const char *>(p.vp + base);
#pragma unroll
                for (int u = 0; u < NQ; u++) {
                    const int q4 = q0 + u;
                    __builtin_amdgcn_global_load_lds(kb + koff[u], (lds_ptr)(kd + q4 * 512), 16, 0, 0);
                    __builtin_amdgcn_global_load_lds(vb + voff[u], (lds_ptr)(vd + q4 * 512), 16, 0, 3);
                }
            } else {
                // the step's last tile: keys past its end read the last key's row (finite
                // data under p = 0); a slot keeps the swizzle of the key it stands for
                const uint64_t base0 = page_base(tp.pg[0], pos0), base1 = page_base(tp.pg[1], pos0 + 16);
#pragma unroll
                for (int u = 0; u < NQ; u++) {
                    const int q4 = q0 + u;
                    const int key = 16 * dx + 4 * q4 + ksub, kk = min(key, last);
                    const uint64_t row = (kk >> 4 ? base1 : base0) + (uint32_t)((kk & 15) * D);
                    const int kc = slot ^ (key & 15), vc = slot ^ (4 * (key & 3));
                    __builtin_amdgcn_global_load_lds(p.kp + row + kc * 8, (lds_ptr)(kd + q4 * 512), 16, 0, 0);
                    __builtin_amdgcn_global_load_lds(p.vp + row + vc * 8, (lds_ptr)(vd + q4 * 512), 16, 0, 3);
                }
            }
        };
        // raw page ids of the next tile to load, fetched one load ahead (the first tile's
        // with the queries, before the positions, when keys are not split); a step looks up
        // the tile after next at its end, so the scalar loads' wait falls on the closing
        // barrier instead of on the step's LDS reads
        const int ft = min(tile_of(0), kt_hi - 1);
        TilePages pn = p.splits == 1 && ft == grp ? spec : raw_pages(p, bt, ft);
        auto issue = [&](int i, int buf) {
            if (i < steps) dl_load(min(tile_of(i), kt_hi - 1), buf, pn);
        };
        auto next_pages = [&](int i) {
            if (i < steps) pn = raw_pages(p, bt, min(tile_of(i), kt_hi - 1));
        };
        issue(0, 0);
        next_pages(1);
        for (int i = 0; i < steps; i += 2) {
            wait_direct_loads();
            __syncthreads();
            compute(tile_of(i), 0, [&] { issue(i + 1, 1); });
            next_pages(i + 2);
            if (i + 1 >= steps) break;
            wait_direct_loads();
            __syncthreads();
            compute(tile_of(i + 1), 1, [&] { issue(i + 2, 0); });
            next_pages(i + 3);
        }
        __syncthreads();   // every wave is done with the tiles before the merge reuses the LDS
    } else {
        // Loads are issued unconditionally (a step past the group's last tile re-reads its
        // last tile, never used) so the number of loads in flight is static and the waits
        // before each LDS store only cover the tile being stored.
        Stage<D, INT8, GT> s0, s1;
        // Page ids of the next tile to load, fetched one load ahead.
        TilePages pnext = PG16 ? tile_pages(p, bt, min(tile_of(0), kt_hi - 1)) : TilePages{};
        auto ld = [&](Stage<D, INT8, GT> &stg, int i) {
            load_tile<D, INT8, PG16, GT>(stg, p, bt, h, min(tile_of(i), kt_hi - 1), kend, gtid, pnext);
            if (PG16) pnext = tile_pages(p, bt, min(tile_of(i + 1), kt_hi - 1));
        };
        ld(s0, 0);
        ld(s1, 1);
        if (tile_of(0) < kt_hi) store_tile<D, INT8, GT>(s0, sm, 0, gtid, kend - tile_of(0) * KT);
        __syncthreads();
        for (int i = 0; i < steps; i += 2) {
            compute(tile_of(i), 0, [&] { ld(s0, i + 2); });
            if (tile_of(i + 1) < kt_hi) store_tile<D, INT8, GT>(s1, sm, 1, gtid, kend - tile_of(i + 1) * KT);
            __syncthreads();
            if (i + 1 >= steps) break;
            compute(tile_of(i + 1), 1, [&] { ld(s1, i + 3); });
            if (tile_of(i + 2) < kt_hi) store_tile<D, INT8, GT>(s0, sm, 0, gtid, kend - tile_of(i + 2) * KT);
            __syncthreads();
        }
    }
    l += __shfl_xor(l, 32);
    if (NG > 1) {
        // Merge the groups' states (same rows, disjoint keys): every group writes its
        // (O, m, l) to its own LDS slab, then all threads combine (row, 4 elements) items.
        float *my = mslab + (size_t)grp * RPG * MROW + r * MROW;
#pragma unroll
        for (int db = 0; db < NDB; db++)
#pragma unroll
            for (int e4 = 0; e4 < 4; e4++)
                *reinterpret_cast<f32x4 *>(my + 32 * db + 8 * e4 + 4 * kg) =
                    (f32x4){o[db][4 * e4], o[db][4 * e4 + 1], o[db][4 * e4 + 2], o[db][4 * e4 + 3]};
        if (kg == 0) {
            my[D] = m;
            my[D + 1] = l;
        }
        __syncthreads();
        // Each thread combines IT (row, 4-element) items; all slab reads are issued
        // before any arithmetic so their LDS latencies overlap.
        constexpr int NT = 64 * WPG * NG, IT = RPG * (D / 4) / NT;
        static_assert(IT * NT == RPG * (D / 4), "merge items must divide evenly");
        float2 ml[IT][NG];
        f32x4 dv[IT][NG];
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int item = threadIdx.x + it * NT, rr = item / (D / 4), d4 = (item % (D / 4)) * 4;
#pragma unroll
            for (int gi = 0; gi < NG; gi++) {
                const float *src = mslab + ((size_t)gi * RPG + rr) * MROW;
                ml[it][gi] = *reinterpret_cast<const float2 *>(src + D);
                dv[it][gi] = *reinterpret_cast<const f32x4 *>(src + d4);
            }
        }
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int item = threadIdx.x + it * NT, rr = item / (D / 4), d4 = (item % (D / 4)) * 4;
            // PAIR: slab rows 0-31 are the heavy q-tile's, 32-63 the light one's
            const int wr = PAIR ? rr / 32 : 0, rl = PAIR ? rr % 32 : rr;
            const int ttl = rl / p.G, gg = rl - ttl * p.G, tt = (PAIR && wr ? qt_light : qt) * p.TQ + ttl;
            if (PAIR && wr == 1 && qt_light == qt) continue;
            float mx = NEG_BIG;
#pragma unroll
            for (int gi = 0; gi < NG; gi++) mx = fmaxf(mx, ml[it][gi].x);
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            float lsum = 0.0f;
#pragma unroll
            for (int gi = 0; gi < NG; gi++) {
                const float wgt = fast_exp2(ml[it][gi].x - mx);
                lsum += ml[it][gi].y * wgt;
                acc += dv[it][gi] * wgt;
            }
            if (ttl >= p.TQ || tt >= nb) continue;
            if (p.splits > 1) {
                // The split's partial for packed row tt * G + gg: (acc, m, l).
                float *dst = p.part + (unit * p.M + (size_t)tt * p.G + gg) * (D + 2);
                *reinterpret_cast<f32x4 *>(dst + d4) = acc;
                if (d4 == 0) *reinterpret_cast<float2 *>(dst + D) = make_float2(mx, lsum);
                continue;
            }
            const float inv = 1.0f / lsum;
            uint16_t *orow = p.out + ((size_t)(tok0 + tt) * p.Hq + h * p.G + gg) * D + d4;
            *reinterpret_cast<u32x2 *>(orow) = (u32x2){pack_bf16x2(acc[0] * inv, acc[1] * inv),
                                                       pack_bf16x2(acc[2] * inv, acc[3] * inv)};
        }
        return;
    }
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

// One 16-byte-per-lane direct global -> LDS load (global_load_lds_dwordx4 through the
// compiler's builtin, which sets M0 itself), from a wave-uniform base plus a per-lane byte
// offset (NT: cache-policy bits 3, sc0 nt). The LDS address must be wave-uniform. The caller
// waits with an explicit vmcnt and a barrier before any wave reads the tile; the compiler
// adds a vmcnt(0) of its own before the transposing V reads that follow a step's loads
// (it cannot tell the two buffers apart), which costs 0.1-1.0 us per call against issuing
// the same loads from inline assembly (measured: 512 tokens 9.99 -> 10.27 us, chunked 512 on
// 1024 19.07 -> 19.82, 1024 tokens 23.6 -> 24.6), the price of leaving M0 to the compiler.
typedef __attribute__((address_space(3))) void *lds_ptr_t;
template <bool NT>
__device__ __forceinline__ void lds_dma16(const void *base, uint32_t voff, uint32_t lds) {
    // the base and the LDS address are wave-uniform: pin them in scalar registers
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    // (readfirstlane returns int: each half goes through uint32_t, never sign-extended)
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
    const char *sbase = reinterpret_cast<const char *>((hi << 32) | lo);
    const uint32_t lds_addr = (uint32_t)__builtin_amdgcn_readfirstlane(lds);
    __builtin_amdgcn_global_load_lds(sbase + voff, (lds_ptr_t)(size_t)lds_addr, 16, 0, NT ? 3 : 0);
}
// The same from a per-lane 64-bit address (the step's last tile, whose rows are clamped per key).
template <bool NT>
__device__ __forceinline__ void lds_dma16_v(const void *gptr, uint32_t lds) {
    const uint32_t lds_addr = (uint32_t)__builtin_amdgcn_readfirstlane(lds);
    __builtin_amdgcn_global_load_lds(gptr, (lds_ptr_t)(size_t)lds_addr, 16, 0, NT ? 3 : 0);
}

// Paired q-tiles on 16-row waves (bf16 activations, D = 128, pages of 2^k >= 16 tokens,
// causal, no key splits; dense bf16 cache, or INT8 with INT8 = true). The work of the paired
// kernel above — work-group y holds the
// heavy q-tile qtiles - 1 - y and the light q-tile y, four key groups walk the key tiles
// through their own double-buffered LDS tiles and merge at the end — with each q-tile's 32
// rows split over two waves of 16 rows: 16 waves of at most 128 VGPRs, four per SIMD.
// Wave w is wave wl = w / 4 of key group w % 4 (wl 0, 1: heavy rows 0-15, 16-31; 2, 3:
// light rows), so a SIMD holds one group's four waves: two heavy waves with independent
// dependency chains on the same tiles, whose MFMAs and softmax interleave.
// Per wave (lane l: row r16 = l % 16 of the wave, k-group kg = l / 16) and 32-key tile:
//   S^T = K Q^T     2 x D/32 v_mfma_f32_16x16x32_bf16 (keys 0-15, 16-31); A = K rows from
//                   LDS (16 B per lane), B = Q^T in registers; the lane holds its row's
//                   scores of keys 4 kg + e and 16 + 4 kg + e, e < 4.
//   softmax         exp2 domain, 8 scores per lane, two xor shuffles for the row max.
//   O^T += V^T P^T  D/16 v_mfma_f32_16x16x32_bf16; B = P^T is the score registers (k-index
//                   8 kg + j: key 4 kg + j, then 16 + 4 kg + j - 4), A = V^T from two 8-B
//                   transposing reads (rows 4 kg .. + 3 and 16 + 4 kg .. + 3).
// A step issues the next tile's loads first (dense: direct loads into the other buffer;
// INT8: loads into registers, converted to bf16 and stored into the
// other buffer after the step's compute), then reads this tile's keys, runs the score MFMAs
// and the softmax, and only then reads the values, so key and value operands never occupy
// registers together. The pair's 64 query rows come through LDS (one direct load per lane),
// read once into registers after the first tile lands.
template <bool INT8>
__global__ void __launch_bounds__(1024) prefill16_kernel(PrefillParams p) {
    constexpr int D = 128, NG = 4, NQB = D / 32, NDB = D / 16;
    constexpr int HW = 2, NQ = 2;        // direct loads: waves per 16-key page half, instructions per wave
    constexpr int RPG = 64, MROW = D + 4;
    // a key group's tiles (bf16, swizzled rows) and, for an INT8 cache, their scales
    struct Bufs {
        uint16_t k[2][KT * 128];
        uint16_t v[2][KT * 128];
        float sk[2][INT8 ? KT : 1], sv[2][INT8 ? KT : 1];
    };
    constexpr int QOFF = (int)sizeof(Bufs) * NG;   // the pair's 64 query rows (16 KB)
    constexpr int SMEM = QOFF + RPG * D * 2, MERGE = NG * RPG * MROW * 4;
    __shared__ __attribute__((aligned(16))) char smem_raw[SMEM > MERGE ? SMEM : MERGE];
    float *mslab = reinterpret_cast<float *>(smem_raw);

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = w % NG, wl = w / NG;
    const bool light = wl >= 2;
    const int r16 = lane & 15, kg = lane >> 4;
    const int h = blockIdx.x;
    const int qt = p.qtiles - 1 - (int)blockIdx.y, qt_light = blockIdx.y;
    const int qtw = light ? qt_light : qt;
    const int b = blockIdx.z;
    // the pointer arguments the prologue dereferences, loaded in the kernel arguments' first
    // batch of scalar loads (left to itself the compiler loads some only after the query
    // counts, a second dependent round trip before the first tile's loads)
    asm volatile("" ::"s"(p.q), "s"(p.kp), "s"(p.vp), "s"(p.bt), "s"(p.positions), "s"(p.qsl));
    const int32_t *bt = p.bt + (size_t)b * p.bt_stride;
    // The first tile's page ids do not depend on the step's positions: their scalar loads go
    // out first, in the same batch as the query-count and position loads.
    const TilePages spec = raw_pages(p, bt, grp);
    const int tok0 = p.qsl ? sload(p.qsl, b) : b * p.nmax;
    const int nb = p.qsl ? min(sload(p.qsl, b + 1) - tok0, p.nmax) : p.nmax;
    const int start = max(sload(p.positions, nb > 0 ? tok0 : 0), 0), len = start + nb;
    const int t_first = qt * p.TQ;
    // No early exit for a pair past the sequence's queries (a shorter sequence of a ragged
    // batch): a branch here would let the compiler sink the scalar loads above past it, behind
    // the query rows' address arithmetic. Such a pair has no row to compute (row_ok is false
    // everywhere, its key steps are at most those of its first positions) and writes nothing.
    const int t_first_w = qtw * p.TQ;
    // This lane's row: row rr of its q-tile (B operand of S^T: elements 32 i + 8 kg .. + 8).
    // (G divides 32 here, a power of two: rows split into position and head by shifts)
    const int rr = 16 * (wl & 1) + r16, tl = rr >> p.gshift, t = t_first_w + tl;
    const bool row_ok = tl < p.TQ && t < nb && !(light && qt_light == qt);
    // The pair's 64 query rows (heavy 0-31, light 32-63) go to LDS with one direct load per
    // lane (row threadIdx / 16, 16-B slot threadIdx % 16 holding chunk slot ^ (row % 16));
    // each wave reads its operands back once, after the first barrier.
    {
        const int qrow = threadIdx.x >> 4, qslot = threadIdx.x & 15, rl = qrow & 31;
        const int tq = ((qrow >> 5) ? qt_light : qt) * p.TQ + (rl >> p.gshift), gq = rl & (p.G - 1);
        const bool ok = (rl >> p.gshift) < p.TQ && tq < nb;
        const uint16_t *src = p.q + ((size_t)(ok ? tok0 + tq : 0) * p.Hq + h * p.G + gq) * D + (qslot ^ (qrow & 15)) * 8;
        lds_dma16_v<false>(src, (uint32_t)(uintptr_t)(smem_raw + QOFF) + w * 1024);
    }
    Bufs &dsm = reinterpret_cast<Bufs *>(smem_raw)[grp];
    // direct loads: wave wl issues instructions q0, q0 + 1 of page half dx (instruction q4
    // writes keys 4 q4 + lane / 16 of the half, 16-B slot lane % 16)
    const int dx = wl / HW, q0 = NQ * (wl % HW);
    const int ksub = lane >> 4, slot = lane & 15;
    uint32_t koff[NQ], voff[NQ];
#pragma unroll
    for (int u = 0; u < NQ; u++) {
        const int key = 4 * (q0 + u) + ksub;
        koff[u] = (uint32_t)(key * D + ((slot ^ key) * 8)) * 2u;
        voff[u] = (uint32_t)(key * D + ((slot ^ (4 * (key & 3)) ^ (2 * ((key >> 2) & 1))) * 8)) * 2u;
    }
    // element offsets: page pg, row r of KV head h at pg * pstride + hoff + r * D
    const uint32_t pstride = (uint32_t)p.Hk * p.P * D, hoff = (uint32_t)h * p.P * D;
    auto page_base = [&](int raw, int pos) -> uint64_t {
        return (uint64_t)(uint32_t)clamp_page(raw, p.num_pages) * pstride + hoff + (uint32_t)((pos & (p.P - 1)) * D);
    };
    // a tile whose 32 keys are all visible: one page half per wave, scalar row bases
    auto dl_full = [&](int kt, int buf, const TilePages &tp) {
        const uint32_t kd = (uint32_t)(uintptr_t)&dsm.k[buf][dx * 2048];
        const uint32_t vd = (uint32_t)(uintptr_t)&dsm.v[buf][dx * 2048];
        const uint64_t base = page_base(dx ? tp.pg[1] : tp.pg[0], kt * KT + 16 * dx);
        const uint16_t *kb = p.kp + base, *vb = p.vp + base;
#pragma unroll
        for (int u = 0; u < NQ; u++) {
            lds_dma16<false>(kb, koff[u], kd + (q0 + u) * 1024);
            lds_dma16<true>(vb, voff[u], vd + (q0 + u) * 1024);
        }
    };
    // Tile grp is whole for any start when the q-tile's last position alone reaches past it
    // (the step's keys end at start + t_last + 1 >= t_last + 1): its loads then go out before
    // the positions load returns.
    const bool first_full = !INT8 && min(t_first + p.TQ, nb) - 1 - grp * KT >= KT - 1;
    if (first_full) dl_full(grp, 0, spec);
    u32x4 qreg[NQB];
    const int qpos = p.causal && row_ok ? start + t : len - 1;
    const int t_last = min(t_first + p.TQ, nb) - 1;
    const int kend = p.causal ? start + t_last + 1 : len;
    const int kend_w = light && p.causal ? start + min(t_first_w + p.TQ, nb) : kend;
    const int kt_hi_w = (kend_w + KT - 1) / KT;
    const int nkt = (kend + KT - 1) / KT;
    const int steps = (nkt + NG - 1) / NG;
    const int mask_from = p.causal ? start + t_first_w : len - 1;

    f32x4 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; db++) o[db] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m = NEG_BIG, l = 0.0f;
    // transposing V reads: 16-lane group kg reads rows 4 kg + r16 / 4 (and + 16), columns
    // 4 (r16 % 4) .. + 3 of each 16-column block. Value rows are swizzled by their key:
    // 16-B chunk c sits in slot c ^ 4 (key % 4) ^ 2 ((key / 4) % 2), so the four rows of one
    // lane group fall in distinct 32-B windows and groups kg, kg + 1 (rows 4 apart) in the
    // other half of the banks (bank-conflict cycles 1.33 M -> 4 K per chunked-prefill launch).
    const int vrow = 4 * kg + (r16 >> 2), vsw = 4 * (r16 >> 2) ^ 2 * (kg & 1);
    const int vc_lo = (r16 & 3) >> 1, vc_off = 4 * (r16 & 1);

    auto dl_load = [&](int kt, int buf, const TilePages &tp) {
        const int pos0 = kt * KT, last = kend - 1 - pos0;   // >= 0 for every tile loaded
        const uint32_t kd = (uint32_t)(uintptr_t)&dsm.k[buf][dx * 2048];
        const uint32_t vd = (uint32_t)(uintptr_t)&dsm.v[buf][dx * 2048];
        if (last >= KT - 1) {
            dl_full(kt, buf, tp);
        } else {
            const uint64_t base0 = page_base(tp.pg[0], pos0), base1 = page_base(tp.pg[1], pos0 + 16);
#pragma unroll
            for (int u = 0; u < NQ; u++) {
                const int q4 = q0 + u;
                const int key = 16 * dx + 4 * q4 + ksub, kk = min(key, last);
                const uint64_t row = (kk >> 4 ? base1 : base0) + (uint32_t)((kk & 15) * D);
                const int kc = slot ^ (key & 15), vc = slot ^ (4 * (key & 3)) ^ (2 * ((key >> 2) & 1));
                lds_dma16_v<false>(p.kp + row + kc * 8, kd + q4 * 1024);
                lds_dma16_v<true>(p.vp + row + vc * 8, vd + q4 * 1024);
            }
        }
    };

    // INT8 cache: tiles staged through registers. Lane gl of the group's 256 holds 16 bytes
    // of key gl / 8 (elements 16 (gl % 8) ..) for K and for V, and lanes 0-63 one scale;
    // stored as bf16 (exact) into the same swizzled rows as the direct loads. Keys past the
    // step's end read the last key's row (finite values and scales, masked to p = 0).
    const int gl = 64 * wl + lane, key_l = gl >> 3, part = gl & 7;
    const size_t half_q = (size_t)p.num_pages * p.Hk * p.P * D;
    const size_t half_s = (size_t)p.num_pages * p.Hk * p.P;
    u32x4 stk = {0u, 0u, 0u, 0u}, stv = {0u, 0u, 0u, 0u};
    float sts = 0.0f;
    auto i8_row = [&](int kt, int key, const TilePages &tp) -> long long {
        const int pos0 = kt * KT, kk = min(key, kend - 1 - pos0);
        const int pg = clamp_page(kk >> 4 ? tp.pg[1] : tp.pg[0], p.num_pages);
        return ((long long)pg * p.Hk + h) * p.P + ((pos0 + (kk & 16)) & (p.P - 1)) + (kk & 15);
    };
    auto i8_load = [&](int kt, const TilePages &tp) {
        const long long row = i8_row(kt, key_l, tp);
        stk = *reinterpret_cast<const u32x4 *>(p.lq + row * D + 16 * part);
        stv = *reinterpret_cast<const u32x4 *>(p.lq + half_q + row * D + 16 * part);
        if (gl < 2 * KT) {
            const long long srow = i8_row(kt, gl & (KT - 1), tp);
            sts = p.ls[(gl < KT ? 0 : half_s) + srow];
        }
    };
    auto i8_store = [&](int buf) {
#pragma unroll
        for (int c2 = 0; c2 < 2; c2++) {
            const int c = 2 * part + c2;
            uint32_t a0, a1, a2, a3;
            i8x4_to_bf16(stk[2 * c2], a0, a1);
            i8x4_to_bf16(stk[2 * c2 + 1], a2, a3);
            *reinterpret_cast<u32x4 *>(&dsm.k[buf][key_l * D + ((c ^ (key_l & 15)) * 8)]) = (u32x4){a0, a1, a2, a3};
            i8x4_to_bf16(stv[2 * c2], a0, a1);
            i8x4_to_bf16(stv[2 * c2 + 1], a2, a3);
            const int vs = c ^ (4 * (key_l & 3)) ^ (2 * ((key_l >> 2) & 1));
            *reinterpret_cast<u32x4 *>(&dsm.v[buf][key_l * D + vs * 8]) = (u32x4){a0, a1, a2, a3};
        }
        if (gl < KT) dsm.sk[buf][gl] = sts;
        else if (gl < 2 * KT) dsm.sv[buf][gl - KT] = sts;
    };

    auto compute = [&](int kt, int buf, auto &&issue_loads) {
        issue_loads();
        if (kt >= kt_hi_w) return;   // past this wave's keys (a light wave, or the group's last step)
        const uint16_t *kt_lds = &dsm.k[buf][0];
        f32x4 sc[2];
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
            u32x4 ka[NQB];
            const uint16_t *krow = kt_lds + (16 * kb + r16) * D;
#pragma unroll
            for (int i = 0; i < NQB; i++) ka[i] = *reinterpret_cast<const u32x4 *>(krow + (((4 * i + kg) ^ r16) * 8));
            sc[kb] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < NQB; i++)
                sc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ka[i]), as_bf16x8(qreg[i]), sc[kb], 0, 0, 0);
        }
        const bool need_mask = kt * KT + KT - 1 > mask_from;
        // INT8: the scales of this lane's 8 score keys, 4 kg + e and 16 + 4 kg + e
        f32x4 skq[2];
        if constexpr (INT8) {
            skq[0] = *reinterpret_cast<const f32x4 *>(&dsm.sk[buf][4 * kg]);
            skq[1] = *reinterpret_cast<const f32x4 *>(&dsm.sk[buf][16 + 4 * kg]);
        }
        float x[8], mt = -INFINITY;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            x[e] = sc[e >> 2][e & 3];
            if constexpr (INT8) x[e] *= skq[e >> 2][e & 3];
        }
        if (need_mask) {   // wave-uniform: only tiles that reach past a row's first visible limit
            const int lim = min(qpos, kend_w - 1) - (kt * KT + 4 * kg);   // last visible key, tile-relative
#pragma unroll
            for (int e = 0; e < 8; e++) x[e] = 16 * (e >> 2) + (e & 3) <= lim ? x[e] : -INFINITY;
        }
#pragma unroll
        for (int e = 0; e < 8; e++) mt = fmaxf(mt, x[e]);
        mt *= p.scale_log2;
        if (__any(mt > m + RESCALE_LOG2)) {
            mt = fmaxf(mt, __shfl_xor(mt, 16));
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float mn = fmaxf(m, mt);
            const float alpha = fast_exp2(m - mn);
            m = mn;
            l *= alpha;
#pragma unroll
            for (int db = 0; db < NDB; db++) o[db] *= alpha;
        }
        float pe[8], ps = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            pe[e] = fast_exp2(__builtin_fmaf(x[e], p.scale_log2, -m));
            ps += pe[e];
        }
        l += ps;
        if constexpr (INT8) {
            // a value's scale multiplies its probability before the bf16 rounding
            const f32x4 sva = *reinterpret_cast<const f32x4 *>(&dsm.sv[buf][4 * kg]);
            const f32x4 svb = *reinterpret_cast<const f32x4 *>(&dsm.sv[buf][16 + 4 * kg]);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                pe[e] *= sva[e];
                pe[4 + e] *= svb[e];
            }
        }
        const u32x4 pb = {pack_bf16x2(pe[0], pe[1]), pack_bf16x2(pe[2], pe[3]), pack_bf16x2(pe[4], pe[5]),
                          pack_bf16x2(pe[6], pe[7])};
        const uint16_t *vt = &dsm.v[buf][0];
#pragma unroll
        for (int db = 0; db < NDB; db++) {
            const int col = ((2 * db + vc_lo) ^ vsw) * 8 + vc_off;
            const u32x2 lo = lds_tr16(vt + vrow * D + col);
            const u32x2 hi = lds_tr16(vt + (vrow + 16) * D + col);
            o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8((u32x4){lo[0], lo[1], hi[0], hi[1]}),
                                                            as_bf16x8(pb), o[db], 0, 0, 0);
        }
    };

    auto tile_of = [&](int i) { return grp + NG * i; };
    const int ft = min(tile_of(0), nkt - 1);
    TilePages pn = ft == grp ? spec : raw_pages(p, bt, ft);
    // A step issues the next tile's loads first and looks up the page ids of the tile after
    // at its end (next_pages), so the scalar loads' wait falls on the step's closing barrier
    // instead of on its LDS reads (both are counted by lgkmcnt).
    auto issue = [&](int i, int buf) {
        if (i < steps) dl_load(min(tile_of(i), nkt - 1), buf, pn);
    };
    auto next_pages = [&](int i) {
        if (i < steps) pn = raw_pages(p, bt, min(tile_of(i), nkt - 1));
    };
    if constexpr (!INT8) {
        if (!first_full) issue(0, 0);
        next_pages(1);
    } else {
        i8_load(min(tile_of(0), nkt - 1), pn);
        pn = raw_pages(p, bt, min(tile_of(1), nkt - 1));
        i8_store(0);
    }
    wait_direct_loads();   // the queries' direct loads (and tile 0's)
    __syncthreads();
    {
        const int qr = 32 * (wl >> 1) + rr;   // this lane's row in the query block
        const uint16_t *qb = reinterpret_cast<const uint16_t *>(smem_raw + QOFF) + qr * D;
#pragma unroll
        for (int i = 0; i < NQB; i++) {
            const u32x4 raw = *reinterpret_cast<const u32x4 *>(qb + (((4 * i + kg) ^ (qr & 15)) * 8));
            if constexpr (INT8) {
                // bf16(q * smooth) (attention.jl:90-95)
                const int d0 = 32 * i + 8 * kg;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    qreg[i][e] = pack_bf16x2(__uint_as_float(raw[e] << 16) * p.smooth[d0 + 2 * e],
                                             __uint_as_float(raw[e] & 0xffff0000u) * p.smooth[d0 + 2 * e + 1]);
            } else {
                qreg[i] = raw;
            }
            if (!row_ok) qreg[i] = (u32x4){0u, 0u, 0u, 0u};
        }
    }
    if constexpr (!INT8) {
        for (int i = 0; i < steps; i += 2) {
            if (i > 0) {
                wait_direct_loads();
                __syncthreads();
            }
            compute(tile_of(i), 0, [&] { issue(i + 1, 1); });
            next_pages(i + 2);
            if (i + 1 >= steps) break;
            wait_direct_loads();
            __syncthreads();
            compute(tile_of(i + 1), 1, [&] { issue(i + 2, 0); });
            next_pages(i + 3);
        }
    } else {
        for (int i = 0; i < steps; i++) {
            if (i > 0) __syncthreads();
            const bool more = i + 1 < steps;
            compute(tile_of(i), i & 1, [&] {
                if (more) {
                    i8_load(min(tile_of(i + 1), nkt - 1), pn);
                    pn = raw_pages(p, bt, min(tile_of(i + 2), nkt - 1));
                }
            });
            if (more) i8_store((i + 1) & 1);
        }
    }
    __syncthreads();   // every wave is done with the tiles before the merge reuses the LDS

    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    // Merge the groups' states: slab rows 0-31 hold the heavy q-tile's rows, 32-63 the light one's.
    {
        float *my = mslab + ((size_t)grp * RPG + 32 * (wl >> 1) + rr) * MROW;
#pragma unroll
        for (int db = 0; db < NDB; db++) *reinterpret_cast<f32x4 *>(my + 16 * db + 4 * kg) = o[db];
        if (kg == 0) {
            my[D] = m;
            my[D + 1] = l;
        }
    }
    __syncthreads();
    constexpr int NT = 1024, IT = RPG * (D / 4) / NT;
    float2 ml[IT][NG];
    f32x4 dv[IT][NG];
#pragma unroll
    for (int it = 0; it < IT; it++) {
        const int item = threadIdx.x + it * NT, sr = item / (D / 4), d4 = (item % (D / 4)) * 4;
#pragma unroll
        for (int gi = 0; gi < NG; gi++) {
            const float *src = mslab + ((size_t)gi * RPG + sr) * MROW;
            ml[it][gi] = *reinterpret_cast<const float2 *>(src + D);
            dv[it][gi] = *reinterpret_cast<const f32x4 *>(src + d4);
        }
    }
#pragma unroll
    for (int it = 0; it < IT; it++) {
        const int item = threadIdx.x + it * NT, sr = item / (D / 4), d4 = (item % (D / 4)) * 4;
        const int wr = sr / 32, rl = sr % 32;
        const int ttl = rl >> p.gshift, gg = rl & (p.G - 1), tt = (wr ? qt_light : qt) * p.TQ + ttl;
        if (wr == 1 && qt_light == qt) continue;
        float mx = NEG_BIG;
#pragma unroll
        for (int gi = 0; gi < NG; gi++) mx = fmaxf(mx, ml[it][gi].x);
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        float lsum = 0.0f;
#pragma unroll
        for (int gi = 0; gi < NG; gi++) {
            const float wgt = fast_exp2(ml[it][gi].x - mx);
            lsum += ml[it][gi].y * wgt;
            acc += dv[it][gi] * wgt;
        }
        if (ttl >= p.TQ || tt >= nb) continue;
        const float inv = 1.0f / lsum;
        uint16_t *orow = p.out + ((size_t)(tok0 + tt) * p.Hq + h * p.G + gg) * D + d4;
        *reinterpret_cast<u32x2 *>(orow) = (u32x2){pack_bf16x2(acc[0] * inv, acc[1] * inv),
                                                   pack_bf16x2(acc[2] * inv, acc[3] * inv)};
    }
}

template <int D, bool INT8, bool PG16, bool DL>
void launch_prefill_w2(const PrefillParams &p, int ng, dim3 grid, hipStream_t s, bool pair = false) {
    if constexpr (DL) {
        if (pair) return (void)(prefill_kernel<D, INT8, PG16, 2, 4, true, true><<<grid, 512, 0, s>>>(p));
    }
    switch (ng) {
        case 1: prefill_kernel<D, INT8, PG16, 2, 1, DL><<<grid, 128, 0, s>>>(p); break;
        case 2: prefill_kernel<D, INT8, PG16, 2, 2, DL><<<grid, 256, 0, s>>>(p); break;
        default: prefill_kernel<D, INT8, PG16, 2, 4, DL><<<grid, 512, 0, s>>>(p); break;
    }
}

template <int D, bool INT8, bool PG16, bool DL>
void launch_prefill_w4(const PrefillParams &p, int ng, dim3 grid, hipStream_t s) {
    switch (ng) {
        case 1: prefill_kernel<D, INT8, PG16, 4, 1, DL><<<grid, 256, 0, s>>>(p); break;
        default: prefill_kernel<D, INT8, PG16, 4, 2, DL><<<grid, 512, 0, s>>>(p); break;
    }
}

template <int D, bool INT8, bool PG16>
void launch_prefill_g(const PrefillParams &p, int wpg, int ng, bool dl, dim3 grid, hipStream_t s, bool pair) {
    if (wpg == 2) {
        if constexpr (!INT8 && PG16 && D == 128) {
            if (dl) return launch_prefill_w2<D, INT8, PG16, true>(p, ng, grid, s, pair);
        }
        launch_prefill_w2<D, INT8, PG16, false>(p, ng, grid, s);
    } else {
        if constexpr (!INT8 && PG16 && D == 128) {
            if (dl) return launch_prefill_w4<D, INT8, PG16, true>(p, ng, grid, s);
        }
        launch_prefill_w4<D, INT8, PG16, false>(p, ng, grid, s);
    }
}

template <int D, bool INT8>
void launch_prefill_d(const PrefillParams &p, int wpg, int ng, bool dl, dim3 grid, hipStream_t s, bool pair) {
    if (p.P % 16 == 0 && p.pshift >= 0) launch_prefill_g<D, INT8, true>(p, wpg, ng, dl, grid, s, pair);
    else launch_prefill_g<D, INT8, false>(p, wpg, ng, dl, grid, s, false);
}

}  // namespace

// Shape of a prefill launch: WPG waves (32 packed rows each) per key group, NG key groups
// per work-group, and key splits across work-groups, chosen so small prefills and verify
// steps still spread over the 256 CUs. Depends only on host shapes (the block-table
// width bounds the keys), never on positions, so a captured graph stays valid.
ti_prefill_plan ti_plan_prefill(const ti_attention_args *a, const ti_kv_cache *c, bool bound_keys) {
    ti_prefill_plan pl;
    const int G = a->q_heads / c->kv_heads;
    const long long pairs = (long long)c->kv_heads * a->num_seqs;
    const long long key_tiles = ((long long)a->block_table_stride * c->page_size + 31) / 32;
    // The 8-wave ping-pong kernel (256 packed rows per work-group, one per CU) is taken
    // when its work-groups fill the 256 CUs at least twice without key splits: measured
    // 906 vs 745 TFLOP/s at a 4096-token causal prefill (512 work-groups), but slower
    // at 2048 tokens (256) and below, where the four-wave kernel's smaller q-tiles and
    // in-work-group key groups keep more CUs busy. TI_PATH_PREFILL_PINGPONG pins it
    // wherever the shapes allow; the other pinned variants never take it.
    const long long pp_wgs = (long long)((a->max_query_len + 256 / G - 1) / (256 / G)) * pairs;
    const bool pp_ok = ti_prefill_pp_eligible(a, c);
    pl.pp = pp_ok && (a->path == TI_PATH_PREFILL_PINGPONG ||
                      ((a->path == TI_PATH_PREFILL || a->path == TI_PATH_AUTO) && pp_wgs >= 512));
    pl.dl = 0;
    pl.pair = 0;
    pl.r16 = 0;
    if (pl.pp) {
        // Key splits (pinned runs on small grids) while work-groups are fewer than the
        // CUs and every split keeps at least 8 key tiles of the longest context the
        // block tables can hold.
        pl.wpg = 8;
        pl.ng = 1;
        pl.TQ = 256 / G;
        pl.qtiles = (a->max_query_len + pl.TQ - 1) / pl.TQ;
        const long long wgs = (long long)pl.qtiles * pairs;
        pl.splits = 1;
        while (pl.splits < 16 && wgs * pl.splits < 256 && (!bound_keys || key_tiles / (2 * pl.splits) >= 8))
            pl.splits *= 2;
        pl.rows = G * a->max_query_len;
        pl.bytes = pl.splits == 1 ? 0 : (size_t)pairs * pl.splits * pl.rows * (c->head_dim + 2) * sizeof(float);
        return pl;
    }
    pl.wpg = (long long)((a->max_query_len + 128 / G - 1) / (128 / G)) * pairs >= 256 ? 4 : 2;
    if (32 * pl.wpg < G) pl.wpg = 4;
    pl.TQ = 32 * pl.wpg / G;
    pl.qtiles = (a->max_query_len + pl.TQ - 1) / pl.TQ;
    const long long wgs = (long long)pl.qtiles * pairs;
    pl.ng = wgs >= 1024 ? 1 : (wgs >= 512 ? 2 : 4);
    if (pl.wpg == 4 && pl.ng > 2) pl.ng = 2;   // 16 waves of this kernel do not fit one CU's registers
    // Split the keys while work-groups are fewer than the CUs and every split keeps at
    // least 4 steps per key group of the longest context the block tables can hold.
    pl.splits = 1;
    while (pl.splits < 16 && wgs * pl.splits < 256 &&
           (!bound_keys || key_tiles / (2 * pl.splits) >= 4LL * pl.ng))
        pl.splits *= 2;
    // Direct global -> LDS tile loads (bf16 dense cache, head_dim 128, pages of 2^k >= 16
    // tokens) for two-wave key groups, the small grids: measured 13.8 -> 12.4 us at a
    // 512-token prefill and 25.6 -> 23.3 us chunked, bit-identical; for four-wave groups
    // (1024-3072 tokens) no change, so those keep the register-staged loads.
    const bool dl_ok = c->kind == TI_KV_DENSE && a->dtype == TI_BF16 && c->head_dim == 128 &&
                       c->page_size >= 16 && (c->page_size & (c->page_size - 1)) == 0;
    pl.dl = dl_ok && (a->path == TI_PATH_PREFILL_DIRECT || a->path == TI_PATH_PREFILL_PAIRED ||
                      a->path == TI_PATH_PREFILL_PAIRED16 ||
                      (a->path != TI_PATH_PREFILL_STAGED && pl.wpg == 2));
    // Paired q-tiles (a heavy and a light 32-row q-tile per work-group, equal causal work
    // per work-group) for causal steps without key splits on the direct-load shapes; G
    // must divide 32 (whole positions per 32-row q-tile). On 16-row waves
    // (prefill16_kernel) while the pairs make at most 512 work-groups: measured against the
    // plan's four-wave kernel (same process) 11.4 -> 10.4 us at 512 tokens, 22.0 -> 19.7 us
    // for 512 on a 1024-token prefix, 27.2 -> 24.6 us at 1024 tokens, 46.3 -> 42.9 us for
    // 1024 on 1024, even at 768 tokens (384 work-groups), but 37.0 -> 43.3 us at 1536 tokens
    // (768) and twice as slow from 2048 tokens. The 32-row paired kernel (pinned with
    // TI_PATH_PREFILL_PAIRED) needs the plan's two-wave, four-group shape.
    // (INT8 caches pair on the 16-row kernel only, its tiles staged through registers)
    const bool i8_ok = c->kind == TI_KV_INT8 && a->dtype == TI_BF16 && c->head_dim == 128 &&
                       c->page_size >= 16 && (c->page_size & (c->page_size - 1)) == 0;
    const bool pair_ok = (dl_ok || i8_ok) && a->causal && pl.splits == 1 && 32 % G == 0;
    // (32 % G == 0 in pair_ok: G <= 32, so 32 / G >= 1)
    const long long pair_wgs = pair_ok ? pairs * (((a->max_query_len + 32 / G - 1) / (32 / G) + 1) / 2) : 0;
    const bool auto_path = a->path == TI_PATH_PREFILL || a->path == TI_PATH_AUTO;
    pl.r16 = pair_ok && (a->path == TI_PATH_PREFILL_PAIRED16 || (auto_path && R16_BY_DEFAULT && pair_wgs <= 512));
    pl.pair = pl.r16 || (pair_ok && dl_ok && pl.dl && pl.wpg == 2 && pl.ng == 4 &&
                         (a->path == TI_PATH_PREFILL_PAIRED || (auto_path && PAIR_BY_DEFAULT)));
    if (pl.pair) {
        pl.TQ = 32 / G;
        pl.qtiles = (a->max_query_len + pl.TQ - 1) / pl.TQ;
    }
    pl.rows = G * a->max_query_len;
    pl.bytes = pl.splits == 1 ? 0 : (size_t)pairs * pl.splits * pl.rows * (c->head_dim + 2) * sizeof(float);
    return pl;
}

int ti_launch_prefill(const ti_attention_args *a, const ti_kv_cache *c, const ti_prefill_plan &pl,
                      hipStream_t s) {
    if (pl.pp) return ti_launch_prefill_pp(a, c, pl, s);
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
    p.gshift = (p.G & (p.G - 1)) == 0 ? __builtin_ctz(p.G) : -1;   // used by the paired 16-row kernel only
    p.nmax = a->max_query_len;
    p.causal = a->causal;
    p.scale_log2 = a->scale * LOG2E;
    p.part = (float *)a->workspace;
    p.splits = pl.splits;
    p.M = pl.rows;
    p.TQ = pl.TQ;
    p.qtiles = pl.qtiles;
    const int wpg = pl.wpg, ng = pl.ng;
    dim3 grid(c->kv_heads, pl.pair ? (p.qtiles + 1) / 2 : p.qtiles * pl.splits, a->num_seqs);
    if (pl.r16) {
        if (c->kind == TI_KV_INT8) prefill16_kernel<true><<<grid, 1024, 0, s>>>(p);
        else prefill16_kernel<false><<<grid, 1024, 0, s>>>(p);
        return hipGetLastError() == hipSuccess ? TI_OK : TI_ERR_LAUNCH;
    }
    const bool int8 = c->kind == TI_KV_INT8;
    const bool dl = pl.dl;
    if (c->head_dim == 128) {
        if (int8) launch_prefill_d<128, true>(p, wpg, ng, dl, grid, s, false);
        else launch_prefill_d<128, false>(p, wpg, ng, dl, grid, s, pl.pair);
    } else {
        if (int8) launch_prefill_d<64, true>(p, wpg, ng, dl, grid, s, false);
        else launch_prefill_d<64, false>(p, wpg, ng, dl, grid, s, false);
    }
    if (hipGetLastError() != hipSuccess) return TI_ERR_LAUNCH;
    return pl.splits > 1 ? ti_launch_combine(a, c, pl.rows, pl.splits, s) : TI_OK;
}
