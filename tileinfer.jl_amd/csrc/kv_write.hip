// KV-cache writes, rotary embedding and the fused attention-input op.
//
// All three are HBM-bound element-wise kernels whose results must be bit-identical to the
// reference's: every product and sum is rounded separately, so contraction into FMA is
// disabled for the whole file.
#pragma clang fp contract(off)

#include "common.hpp"

using namespace ti;

namespace {

// Pool row (0-based, in units of D elements) of (1-based slot, KV head h) in a
// [pages][H][P][D] pool: offset + P h + P H page (src/ops/reference.jl:61-70,
// src/ops/tile/elementwise.jl:122-128). Returns -1 for a slot outside the pool.
__device__ __forceinline__ long long slot_row(int32_t slot, int h, int P, int H, int pages) {
    long long s = (long long)slot - 1;
    if (s < 0 || s >= (long long)P * pages) return -1;
    return (s % P) + (long long)P * h + (long long)P * H * (s / P);
}

// ---- rope (src/ops/tile/elementwise.jl:10-27; reference src/ops/reference.jl:32-39) ----
// y1 = rnd(rnd(x1 c1) + rnd(-x2 s1)), y2 = rnd(rnd(x2 c2) + rnd(x1 s2)), rnd = round to T.
template <typename T>
__global__ void __launch_bounds__(256) rope_kernel(T *__restrict__ y, const T *__restrict__ x,
                                                   const T *__restrict__ cos_t,
                                                   const T *__restrict__ sin_t, int table_len,
                                                   const int32_t *__restrict__ positions,
                                                   int heads, int D) {
    using E = Elt<T>;
    const int t = blockIdx.x, half = D / 2;   // tokens on x: no 65535 limit
    const int idx = blockIdx.y * blockDim.x + threadIdx.x;
    if (idx >= heads * half) return;
    const int p = positions[t];
    if (p < 0 || p >= table_len) return;
    const int h = idx / half, i = idx % half;
    const size_t base = ((size_t)t * heads + h) * D, tab = (size_t)p * D;
    const float a = E::ld(x, base + i), b = E::ld(x, base + i + half);
    const float c1 = E::ld(cos_t, tab + i), c2 = E::ld(cos_t, tab + i + half);
    const float s1 = E::ld(sin_t, tab + i), s2 = E::ld(sin_t, tab + i + half);
    E::st(y, base + i, E::rnd(E::rnd(a * c1) + E::rnd(-b * s1)));
    E::st(y, base + i + half, E::rnd(E::rnd(b * c2) + E::rnd(a * s2)));
}

// ---- dense store_kv (src/ops/tile/elementwise.jl:119-131): bit copies, 16 B per lane ----
// Grid (n, H), one wave per (token, head): K and V rows of D elements.
template <typename T>
__global__ void __launch_bounds__(64) store_kv_kernel(T *__restrict__ kp, T *__restrict__ vp,
                                                      const T *__restrict__ k,
                                                      const T *__restrict__ v,
                                                      const int32_t *__restrict__ slots, int D,
                                                      int P, int H, int pages) {
    const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const long long row = slot_row(slots[t], h, P, H, pages);
    if (row < 0) return;
    const size_t src = ((size_t)t * H + h) * D, dst = (size_t)row * D;
    const int bytes = D * (int)sizeof(T);
    if ((bytes & 15) == 0) {
        const uint4 *ks = reinterpret_cast<const uint4 *>(k + src);
        const uint4 *vs = reinterpret_cast<const uint4 *>(v + src);
        uint4 *kd = reinterpret_cast<uint4 *>(kp + dst);
        uint4 *vd = reinterpret_cast<uint4 *>(vp + dst);
        for (int i = lane; i < bytes / 16; i += WAVE) {
            kd[i] = ks[i];
            vd[i] = vs[i];
        }
    } else {
        for (int i = lane; i < D; i += WAVE) {
            kp[dst + i] = k[src + i];
            vp[dst + i] = v[src + i];
        }
    }
}

// Quantize one vector held as up to 8 values per lane (element i = lane + 64 j) into q at
// row `row` and its scale, as quantize_columns (src/ops/quant.jl:141-145) and store_int8!
// (src/ops/tile/elementwise.jl:154-161): absmax = max|x|; inv = absmax > 0 ? 127/absmax : 0;
// q = Int8(floor(x inv + 1/2)); s = absmax / 127. All lanes of the wave must call it.
__device__ __forceinline__ void quantize_store(const float (&x)[8], int D, int8_t *__restrict__ q,
                                               float *__restrict__ scale, size_t row) {
    const int lane = threadIdx.x;
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++)
        if (lane + WAVE * j < D) m = fmaxf(m, fabsf(x[j]));
    const float absmax = wave_max(m);
    const float inv = absmax > 0.0f ? __fdiv_rn(127.0f, absmax) : 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int i = lane + WAVE * j;
        if (i < D) q[row * D + i] = (int8_t)floorf(__fadd_rn(__fmul_rn(x[j], inv), 0.5f));
    }
    if (lane == 0) scale[row] = __fdiv_rn(absmax, 127.0f);
}

// ---- INT8 store_kv (src/ops/tile/elementwise.jl:163-178; src/ops/quant.jl:147-159) ----
// Keys are divided by the smoothing factors first; values are not.
template <typename T>
__global__ void __launch_bounds__(64) store_kv_int8_kernel(int8_t *__restrict__ lq,
                                                           float *__restrict__ ls,
                                                           const float *__restrict__ smooth,
                                                           const T *__restrict__ k,
                                                           const T *__restrict__ v,
                                                           const int32_t *__restrict__ slots,
                                                           int D, int P, int H, int pages) {
    using E = Elt<T>;
    const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const long long row = slot_row(slots[t], h, P, H, pages);
    if (row < 0) return;  // uniform across the wave
    const size_t src = ((size_t)t * H + h) * D;
    const size_t half_q = (size_t)pages * H * P * D, half_s = (size_t)pages * H * P;
    float x[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int i = lane + WAVE * j;
        x[j] = i < D ? __fdiv_rn(E::ld(k, src + i), smooth[i]) : 0.0f;
    }
    quantize_store(x, D, lq, ls, (size_t)row);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int i = lane + WAVE * j;
        x[j] = i < D ? E::ld(v, src + i) : 0.0f;
    }
    quantize_store(x, D, lq + half_q, ls + half_s, (size_t)row);
}

// ---- rmsnorm (src/ops/tile/norm.jl:5-38; reference src/ops/interface.jl:118-122) ----
// y = rnd(rnd(x inv_rms) w), inv_rms = 1 / sqrt(sum x^2 / H + eps) in Float32; one wave
// per row of H elements. Rows of up to 128 elements (even H) are reduced with the fused
// attention-input kernel's pairing (lane i holds elements i and i + H/2), so a per-head
// norm here is bit-identical to the one inside that kernel.
template <typename T>
__global__ void __launch_bounds__(64) rmsnorm_kernel(T *__restrict__ y, const T *__restrict__ x,
                                                      const T *__restrict__ w, int H, float eps) {
    using E = Elt<T>;
    const size_t base = (size_t)blockIdx.x * H;
    const int lane = threadIdx.x;
    if (H <= 128 && (H & 1) == 0) {
        const int half = H / 2;
        const bool on = lane < half;
        const float a = on ? E::ld(x, base + lane) : 0.0f;
        const float b = on ? E::ld(x, base + lane + half) : 0.0f;
        const float ss = wave_sum(a * a + b * b);
        const float inv_rms = __frcp_rn(__fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)H), eps)));
        if (on) {
            E::st(y, base + lane, E::rnd(E::rnd(a * inv_rms) * E::ld(w, lane)));
            E::st(y, base + lane + half, E::rnd(E::rnd(b * inv_rms) * E::ld(w, lane + half)));
        }
        return;
    }
    float acc = 0.0f;
    for (int i = lane; i < H; i += WAVE) {
        const float v = E::ld(x, base + i);
        acc = acc + v * v;
    }
    const float ss = wave_sum(acc);
    const float inv_rms = __frcp_rn(__fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)H), eps)));
    for (int i = lane; i < H; i += WAVE)
        E::st(y, base + i, E::rnd(E::rnd(E::ld(x, base + i) * inv_rms) * E::ld(w, i)));
}

// ---- fused attention inputs (src/ops/tile/fused.jl:15-92) ----
// Grid (n, nq + nkv), one wave per (token, head). Lane i < D/2 owns the rotary pair
// (i, i + D/2). Heads j < nq are queries -> q_out; the others are KV head h = j - nq:
// the key (normed, rotated) and the value go to the cache at slots[t].
template <typename T, bool NORM, bool INT8>
__global__ void __launch_bounds__(64) attention_inputs_kernel(
    T *__restrict__ q_out, T *__restrict__ kp, T *__restrict__ vp, int8_t *__restrict__ lq,
    float *__restrict__ ls, const float *__restrict__ smooth, const T *__restrict__ qkv,
    const T *__restrict__ q_norm, const T *__restrict__ k_norm, const T *__restrict__ cos_sin,
    int table_len, const int32_t *__restrict__ positions, const int32_t *__restrict__ slots,
    int nq, int nkv, int D, int P, int pages, float eps) {
    using E = Elt<T>;
    const int t = blockIdx.x, j = blockIdx.y, lane = threadIdx.x, half = D / 2;
    const bool is_q = j < nq;
    const int h = j - nq;
    const int pos = positions[t];
    if (pos < 0 || pos >= table_len) return;
    long long row = 0;
    if (!is_q) {
        row = slot_row(slots[t], h, P, nkv, pages);
        if (row < 0) return;
    }
    const size_t col = ((size_t)t * (nq + 2 * nkv) + j) * D;
    const bool on = lane < half;
    float a = on ? E::ld(qkv, col + lane) : 0.0f;
    float b = on ? E::ld(qkv, col + lane + half) : 0.0f;
    if (NORM) {
        // rmsnorm in Float32, rounding as rmsnorm_kernel: rnd(rnd(x inv_rms) w).
        const float ss = wave_sum(a * a + b * b);
        const float inv_rms = __frcp_rn(__fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), eps)));
        const T *w = is_q ? q_norm : k_norm;
        if (on) {
            a = E::rnd(E::rnd(a * inv_rms) * E::ld(w, lane));
            b = E::rnd(E::rnd(b * inv_rms) * E::ld(w, lane + half));
        }
    }
    const size_t cs = (size_t)pos * 2 * D;
    float y1 = 0.0f, y2 = 0.0f;
    if (on) {
        const float c1 = E::ld(cos_sin, cs + lane), c2 = E::ld(cos_sin, cs + lane + half);
        const float s1 = E::ld(cos_sin, cs + D + lane), s2 = E::ld(cos_sin, cs + D + lane + half);
        y1 = E::rnd(E::rnd(a * c1) + E::rnd(-b * s1));
        y2 = E::rnd(E::rnd(b * c2) + E::rnd(a * s2));
    }
    if (is_q) {
        if (on) {
            const size_t o = ((size_t)t * nq + j) * D;
            E::st(q_out, o + lane, y1);
            E::st(q_out, o + lane + half, y2);
        }
        return;
    }
    const size_t vcol = ((size_t)t * (nq + 2 * nkv) + nq + nkv + h) * D;
    if (!INT8) {
        const size_t dst = (size_t)row * D;
        if (on) {
            E::st(kp, dst + lane, y1);
            E::st(kp, dst + lane + half, y2);
        }
        for (int i = lane; i < D; i += WAVE) vp[dst + i] = qkv[vcol + i];
    } else {
        const size_t half_q = (size_t)pages * nkv * P * D, half_s = (size_t)pages * nkv * P;
        // Element i = lane + 64 jj of the vector for quantize_store: pair halves map to
        // lane (first half) and lane + half; for D = 128 that is j = 0 and j = 1 of lane.
        float x[8];
#pragma unroll
        for (int jj = 0; jj < 8; jj++) x[jj] = 0.0f;
        // Gather the rotated key into the element-major layout through LDS.
        __shared__ float kv_tmp[512];
        if (on) {
            kv_tmp[lane] = __fdiv_rn(y1, smooth[lane]);
            kv_tmp[lane + half] = __fdiv_rn(y2, smooth[lane + half]);
        }
        __syncthreads();
#pragma unroll
        for (int jj = 0; jj < 8; jj++) {
            const int i = lane + WAVE * jj;
            if (i < D) x[jj] = kv_tmp[i];
        }
        quantize_store(x, D, lq, ls, (size_t)row);
#pragma unroll
        for (int jj = 0; jj < 8; jj++) {
            const int i = lane + WAVE * jj;
            x[jj] = i < D ? E::ld(qkv, vcol + i) : 0.0f;
        }
        quantize_store(x, D, lq + half_q, ls + half_s, (size_t)row);
    }
}

// quantize_store for one vector held by an LPH-lane group, 8 elements per lane: elements
// x[0..3] go to bytes o1 .. o1 + 3 of the row, x[4..7] to o2 .. o2 + 3 (as 32-bit words).
template <int LPH>
__device__ __forceinline__ void quantize_group(const float (&x)[8], int8_t *__restrict__ qrow, int o1,
                                               int o2, float *__restrict__ scale, int u) {
    float m = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) m = fmaxf(m, fabsf(x[e]));
#pragma unroll
    for (int o = LPH / 2; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    const float inv = m > 0.0f ? __fdiv_rn(127.0f, m) : 0.0f;
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const int qv = (int)floorf(__fadd_rn(__fmul_rn(x[e], inv), 0.5f));
        w[e >> 2] |= (uint32_t)(uint8_t)(int8_t)qv << (8 * (e & 3));
    }
    *reinterpret_cast<uint32_t *>(qrow + o1) = w[0];
    *reinterpret_cast<uint32_t *>(qrow + o2) = w[1];
    if (u == 0) *scale = __fdiv_rn(m, 127.0f);
}

// Vectorized form of attention_inputs_kernel for head_dim 128 or 64: D / 8 lanes per head
// (16 or 8), lane u owning elements 4u .. 4u + 3 of each half (8-byte bf16 / 16-byte Float32
// loads), 2048 / D heads per 256-thread work-group: grid (n, ceil((nq + nkv) / (2048 / D))).
// Same rounding points element by element. With the q/k norm, each lane keeps the four
// per-lane partials a_i^2 + b_i^2 (i = 4u + e) that the one-wave kernel's lanes hold and
// combines them in that kernel's butterfly order (xor 32, 16, 8, 4 across lanes u ^ 8,
// u ^ 4, u ^ 2, u ^ 1, then xor 2 and 1 inside the lane), so the sum of squares, and with
// it every output, is bit-identical to the one-wave kernel and to rmsnorm_kernel.
template <typename T> struct Vec4;
template <> struct Vec4<uint16_t> {
    static __device__ __forceinline__ void ld(const uint16_t *p, float (&x)[4]) {
        const uint2 w = *reinterpret_cast<const uint2 *>(p);
        x[0] = __uint_as_float(w.x << 16);
        x[1] = __uint_as_float(w.x & 0xffff0000u);
        x[2] = __uint_as_float(w.y << 16);
        x[3] = __uint_as_float(w.y & 0xffff0000u);
    }
    static __device__ __forceinline__ void st(uint16_t *p, const float (&x)[4]) {
        const uint2 w = make_uint2((uint32_t)f2bf(x[0]) | ((uint32_t)f2bf(x[1]) << 16),
                                   (uint32_t)f2bf(x[2]) | ((uint32_t)f2bf(x[3]) << 16));
        *reinterpret_cast<uint2 *>(p) = w;
    }
};
template <> struct Vec4<float> {
    static __device__ __forceinline__ void ld(const float *p, float (&x)[4]) {
        const float4 w = *reinterpret_cast<const float4 *>(p);
        x[0] = w.x; x[1] = w.y; x[2] = w.z; x[3] = w.w;
    }
    static __device__ __forceinline__ void st(float *p, const float (&x)[4]) {
        *reinterpret_cast<float4 *>(p) = make_float4(x[0], x[1], x[2], x[3]);
    }
};

// INT8 caches: a KV head's D / 8 lanes reduce the absmax of its D (smoothed) key or value
// elements with xor shuffles and each lane stores its quantized elements as 32-bit words;
// the arithmetic is quantize_store's element by element (bit-identical).
template <typename T, bool NORM, bool INT8, int D>
__global__ void __launch_bounds__(256) attention_inputs_v_kernel(
    T *__restrict__ q_out, T *__restrict__ kp, T *__restrict__ vp, int8_t *__restrict__ lq,
    float *__restrict__ ls, const float *__restrict__ smooth, const T *__restrict__ qkv,
    const T *__restrict__ q_norm, const T *__restrict__ k_norm, const T *__restrict__ cos_sin,
    int table_len, const int32_t *__restrict__ positions, const int32_t *__restrict__ slots,
    int nq, int nkv, int P, int pages, float eps) {
    constexpr int HALF = D / 2, LPH = D / 8, HPW = 256 / LPH;   // lanes, heads per work-group
    using E = Elt<T>;
    using V = Vec4<T>;
    const int t = blockIdx.x, j = blockIdx.y * HPW + threadIdx.x / LPH, u = threadIdx.x % LPH;
    if (j >= nq + nkv) return;   // a whole 16-lane group
    const bool is_q = j < nq;
    const int h = j - nq;
    // Every load that does not depend on the position goes out first (token t < n and head
    // j are in range, so these addresses are too): one memory round trip, then the rotary
    // table rows of the position, instead of position -> slot -> qkv in sequence.
    const int pos = positions[t];
    const int32_t slot = slots[t];
    const size_t col = ((size_t)t * (nq + 2 * nkv) + j) * D;
    float a[4], b[4];
    V::ld(qkv + col + 4 * u, a);
    V::ld(qkv + col + HALF + 4 * u, b);
    constexpr int VCH = D * (int)sizeof(T) / 16;   // 16-byte chunks of a value row
    uint4 vrow[VCH / LPH];
    if (!is_q) {
        const uint4 *vs = reinterpret_cast<const uint4 *>(qkv + ((size_t)t * (nq + 2 * nkv) + nq + nkv + h) * D);
#pragma unroll
        for (int c = 0; c < VCH / LPH; c++) vrow[c] = vs[u + LPH * c];
    }
    float w1[4], w2[4];
    if (NORM) {
        const T *wn = is_q ? q_norm : k_norm;
        V::ld(wn + 4 * u, w1);
        V::ld(wn + HALF + 4 * u, w2);
    }
    if (pos < 0 || pos >= table_len) return;
    long long row = 0;
    if (!is_q) {
        row = slot_row(slot, h, P, nkv, pages);
        if (row < 0) return;
    }
    if (NORM) {
        float pp[4];
#pragma unroll
        for (int e = 0; e < 4; e++) pp[e] = a[e] * a[e] + b[e] * b[e];
#pragma unroll
        for (int o = LPH / 2; o > 0; o >>= 1)
#pragma unroll
            for (int e = 0; e < 4; e++) pp[e] = pp[e] + __shfl_xor(pp[e], o);
        const float p02 = pp[0] + pp[2], p13 = pp[1] + pp[3];
        const float ss = p02 + p13;
        const float inv_rms = __frcp_rn(__fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)D), eps)));
#pragma unroll
        for (int e = 0; e < 4; e++) {
            a[e] = E::rnd(E::rnd(a[e] * inv_rms) * w1[e]);
            b[e] = E::rnd(E::rnd(b[e] * inv_rms) * w2[e]);
        }
    }
    const T *cs = cos_sin + (size_t)pos * 2 * D;
    float c1[4], c2[4], s1[4], s2[4], y1[4], y2[4];
    V::ld(cs + 4 * u, c1);
    V::ld(cs + HALF + 4 * u, c2);
    V::ld(cs + D + 4 * u, s1);
    V::ld(cs + D + HALF + 4 * u, s2);
#pragma unroll
    for (int e = 0; e < 4; e++) {
        y1[e] = E::rnd(E::rnd(a[e] * c1[e]) + E::rnd(-b[e] * s1[e]));
        y2[e] = E::rnd(E::rnd(b[e] * c2[e]) + E::rnd(a[e] * s2[e]));
    }
    if (!INT8 || is_q) {
        T *dst = is_q ? q_out + ((size_t)t * nq + j) * D : kp + (size_t)row * D;
        V::st(dst + 4 * u, y1);
        V::st(dst + HALF + 4 * u, y2);
        if (is_q) return;
    }
    if constexpr (!INT8) {
        // the value row (loaded above): a bit copy in 16-byte chunks over the head's lanes
        uint4 *vd = reinterpret_cast<uint4 *>(vp + (size_t)row * D);
#pragma unroll
        for (int c = 0; c < VCH / LPH; c++) vd[u + LPH * c] = vrow[c];
    } else {
        const size_t half_q = (size_t)pages * nkv * P * D, half_s = (size_t)pages * nkv * P;
        // keys: the rotated elements 4u + e and 64 + 4u + e divided by their smoothing
        float x[8];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            x[e] = __fdiv_rn(y1[e], smooth[4 * u + e]);
            x[4 + e] = __fdiv_rn(y2[e], smooth[HALF + 4 * u + e]);
        }
        quantize_group<LPH>(x, lq + (size_t)row * D, 4 * u, HALF + 4 * u, ls + row, u);
        // values: this lane's 16-byte chunks of the row, elements in order
        float v[8];
        if constexpr (sizeof(T) == 2) {
            // chunk u = elements 8u .. 8u + 7
            const uint4 w = vrow[0];
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                v[2 * e] = __uint_as_float(ws[e] << 16);
                v[2 * e + 1] = __uint_as_float(ws[e] & 0xffff0000u);
            }
            quantize_group<LPH>(v, lq + half_q + (size_t)row * D, 8 * u, 8 * u + 4, ls + half_s + row, u);
        } else {
            // chunks u and u + LPH = elements 4u .. 4u + 3 and HALF + 4u .. HALF + 4u + 3
#pragma unroll
            for (int c = 0; c < 2; c++) {
                v[4 * c] = __uint_as_float(vrow[c].x);
                v[4 * c + 1] = __uint_as_float(vrow[c].y);
                v[4 * c + 2] = __uint_as_float(vrow[c].z);
                v[4 * c + 3] = __uint_as_float(vrow[c].w);
            }
            quantize_group<LPH>(v, lq + half_q + (size_t)row * D, 4 * u, HALF + 4 * u, ls + half_s + row, u);
        }
    }
}

// store_kv into INT8 pages for head_dim 128 or 64 with the fused kernel's layout: D / 8 lanes
// per KV head (lane u holds elements 4u .. 4u + 3 and D/2 + 4u .. D/2 + 4u + 3 of the key and
// of the value), 2048 / D heads per 256-thread work-group; quantize_group is quantize_store
// element by element.
template <typename T, int D>
__global__ void __launch_bounds__(256) store_kv_int8_v_kernel(int8_t *__restrict__ lq,
                                                              float *__restrict__ ls,
                                                              const float *__restrict__ smooth,
                                                              const T *__restrict__ k,
                                                              const T *__restrict__ v,
                                                              const int32_t *__restrict__ slots,
                                                              int P, int H, int pages) {
    constexpr int HALF = D / 2, LPH = D / 8, HPW = 256 / LPH;   // lanes, heads per work-group
    using V = Vec4<T>;
    const int t = blockIdx.x, h = blockIdx.y * HPW + threadIdx.x / LPH, u = threadIdx.x % LPH;
    if (h >= H) return;   // a whole 16-lane group
    const size_t src = ((size_t)t * H + h) * D;
    float ka[4], kb[4], va[4], vb[4];
    V::ld(k + src + 4 * u, ka);
    V::ld(k + src + HALF + 4 * u, kb);
    V::ld(v + src + 4 * u, va);
    V::ld(v + src + HALF + 4 * u, vb);
    const long long row = slot_row(slots[t], h, P, H, pages);
    if (row < 0) return;   // the whole group
    const size_t half_q = (size_t)pages * H * P * D, half_s = (size_t)pages * H * P;
    float x[8], y[8];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        x[e] = __fdiv_rn(ka[e], smooth[4 * u + e]);
        x[4 + e] = __fdiv_rn(kb[e], smooth[HALF + 4 * u + e]);
        y[e] = va[e];
        y[4 + e] = vb[e];
    }
    quantize_group<LPH>(x, lq + (size_t)row * D, 4 * u, HALF + 4 * u, ls + row, u);
    quantize_group<LPH>(y, lq + half_q + (size_t)row * D, 4 * u, HALF + 4 * u, ls + half_s + row, u);
}

// rope for head_dim 128 or 64 with the fused kernel's layout: D / 8 lanes per head (lane u
// holds pair elements 4u .. 4u + 3 and D/2 + 4u .. D/2 + 4u + 3), 2048 / D heads per
// 256-thread work-group; the head's elements load before the position does. Same formula and rounding
// as rope_kernel; rows at positions outside the table are left untouched.
template <typename T, int D>
__global__ void __launch_bounds__(256) rope_v_kernel(T *__restrict__ y, const T *__restrict__ x,
                                                     const T *__restrict__ cos_t,
                                                     const T *__restrict__ sin_t, int table_len,
                                                     const int32_t *__restrict__ positions,
                                                     int heads) {
    constexpr int HALF = D / 2, LPH = D / 8, HPW = 256 / LPH;   // lanes, heads per work-group
    using E = Elt<T>;
    using V = Vec4<T>;
    const int t = blockIdx.x, h = blockIdx.y * HPW + threadIdx.x / LPH, u = threadIdx.x % LPH;
    if (h >= heads) return;   // a whole 16-lane group
    const size_t base = ((size_t)t * heads + h) * D;
    float a[4], b[4];
    V::ld(x + base + 4 * u, a);
    V::ld(x + base + HALF + 4 * u, b);
    const int p = positions[t];
    if (p < 0 || p >= table_len) return;
    const size_t tab = (size_t)p * D;
    float c1[4], c2[4], s1[4], s2[4], y1[4], y2[4];
    V::ld(cos_t + tab + 4 * u, c1);
    V::ld(cos_t + tab + HALF + 4 * u, c2);
    V::ld(sin_t + tab + 4 * u, s1);
    V::ld(sin_t + tab + HALF + 4 * u, s2);
#pragma unroll
    for (int e = 0; e < 4; e++) {
        y1[e] = E::rnd(E::rnd(a[e] * c1[e]) + E::rnd(-b[e] * s1[e]));
        y2[e] = E::rnd(E::rnd(b[e] * c2[e]) + E::rnd(a[e] * s2[e]));
    }
    V::st(y + base + 4 * u, y1);
    V::st(y + base + HALF + 4 * u, y2);
}

// Dense store_kv for head_dim 128 or 64: D / 8 lanes per KV head, 2048 / D heads per
// 256-thread work-group, each lane moving its 16-byte chunks of the key and value rows (bit copies),
// loaded before the slot is.
template <typename T, int D>
__global__ void __launch_bounds__(256) store_kv_v_kernel(T *__restrict__ kp, T *__restrict__ vp,
                                                         const T *__restrict__ k,
                                                         const T *__restrict__ v,
                                                         const int32_t *__restrict__ slots, int P,
                                                         int H, int pages) {
    constexpr int LPH = D / 8, HPW = 256 / LPH, CH = D * (int)sizeof(T) / 16 / LPH;   // 16-byte chunks per lane
    const int t = blockIdx.x, h = blockIdx.y * HPW + threadIdx.x / LPH, u = threadIdx.x % LPH;
    if (h >= H) return;   // a whole 16-lane group
    const size_t src = ((size_t)t * H + h) * D;
    const uint4 *ks = reinterpret_cast<const uint4 *>(k + src);
    const uint4 *vs = reinterpret_cast<const uint4 *>(v + src);
    uint4 kc[CH], vc[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) {
        kc[c] = ks[u + LPH * c];
        vc[c] = vs[u + LPH * c];
    }
    const long long row = slot_row(slots[t], h, P, H, pages);
    if (row < 0) return;   // the whole group
    uint4 *kd = reinterpret_cast<uint4 *>(kp + (size_t)row * D);
    uint4 *vd = reinterpret_cast<uint4 *>(vp + (size_t)row * D);
#pragma unroll
    for (int c = 0; c < CH; c++) {
        kd[u + LPH * c] = kc[c];
        vd[u + LPH * c] = vc[c];
    }
}

}  // namespace

int ti_launch_rmsnorm(int dtype, void *y, const void *x, const void *w, int rows, int H, float eps,
                      hipStream_t s) {
    if (dtype == TI_BF16)
        rmsnorm_kernel<uint16_t><<<rows, 64, 0, s>>>((uint16_t *)y, (const uint16_t *)x, (const uint16_t *)w, H, eps);
    else
        rmsnorm_kernel<float><<<rows, 64, 0, s>>>((float *)y, (const float *)x, (const float *)w, H, eps);
    return hipGetLastError() == hipSuccess ? TI_OK : TI_ERR_LAUNCH;
}

int ti_launch_rope(int dtype, void *y, const void *x, const void *cos_t, const void *sin_t,
                   int table_len, const int32_t *positions, int n, int heads, int D,
                   hipStream_t s) {
    if (D == 128 || D == 64) {
        const int hpw = 2048 / D;   // heads per 256-thread work-group (D / 8 lanes per head)
        const dim3 vgrid(n, (heads + hpw - 1) / hpw);
#define TI_ROPE_V(DD)                                                                              \
    if (dtype == TI_BF16)                                                                          \
        rope_v_kernel<uint16_t, DD><<<vgrid, 256, 0, s>>>((uint16_t *)y, (const uint16_t *)x,       \
                                                          (const uint16_t *)cos_t,                  \
                                                          (const uint16_t *)sin_t, table_len,       \
                                                          positions, heads);                        \
    else                                                                                           \
        rope_v_kernel<float, DD><<<vgrid, 256, 0, s>>>((float *)y, (const float *)x,                \
                                                       (const float *)cos_t, (const float *)sin_t,  \
                                                       table_len, positions, heads);
        if (D == 128) { TI_ROPE_V(128) } else { TI_ROPE_V(64) }
#undef TI_ROPE_V
        return hipGetLastError() == hipSuccess ? TI_OK : TI_ERR_LAUNCH;
    }
    dim3 grid(n, (heads * (D / 2) + 255) / 256);
    if (dtype == TI_BF16)
        rope_kernel<uint16_t><<<grid, 256, 0, s>>>((uint16_t *)y, (const uint16_t *)x,
                                                   (const uint16_t *)cos_t, (const uint16_t *)sin_t,
                                                   table_len, positions, heads, D);
    else
        rope_kernel<float><<<grid, 256, 0, s>>>((float *)y, (const float *)x, (const float *)cos_t,
                                                (const float *)sin_t, table_len, positions, heads, D);
    return hipGetLastError() == hipSuccess ? TI_OK : TI_ERR_LAUNCH;
}

int ti_launch_store_kv(int dtype, const ti_kv_cache *c, const void *k, const void *v,
                       const int32_t *slots, int n, hipStream_t s) {
    dim3 grid(n, c->kv_heads);
    const int D = c->head_dim, P = c->page_size, H = c->kv_heads, pages = c->num_pages;
    const int hpw = 2048 / D;   // heads per 256-thread work-group (D / 8 lanes per head)
    const dim3 vgrid(n, (H + hpw - 1) / hpw);
#define TI_STORE_V(DD)                                                                             \
    if (c->kind == TI_KV_INT8) {                                                                   \
        if (dtype == TI_BF16)                                                                      \
            store_kv_int8_v_kernel<uint16_t, DD><<<vgrid, 256, 0, s>>>(                            \
                c->layer_q, c->layer_scale, c->smooth, (const uint16_t *)k, (const uint16_t *)v,    \
                slots, P, H, pages);                                                                \
        else                                                                                       \
            store_kv_int8_v_kernel<float, DD><<<vgrid, 256, 0, s>>>(                               \
                c->layer_q, c->layer_scale, c->smooth, (const float *)k, (const float *)v, slots,  \
                P, H, pages);                                                                       \
    } else if (dtype == TI_BF16) {                                                                 \
        store_kv_v_kernel<uint16_t, DD><<<vgrid, 256, 0, s>>>(                                     \
            (uint16_t *)c->k_pages, (uint16_t *)c->v_pages, (const uint16_t *)k,                    \
            (const uint16_t *)v, slots, P, H, pages);                                               \
    } else {                                                                                       \
        store_kv_v_kernel<float, DD><<<vgrid, 256, 0, s>>>((float *)c->k_pages, (float *)c->v_pages, \
                                                           (const float *)k, (const float *)v,      \
                                                           slots, P, H, pages);                     \
    }
    if (D == 128) {
        TI_STORE_V(128)
    } else if (D == 64) {
        TI_STORE_V(64)
    } else if (c->kind == TI_KV_INT8) {
        if (dtype == TI_BF16)
            store_kv_int8_kernel<uint16_t><<<grid, 64, 0, s>>>(c->layer_q, c->layer_scale, c->smooth,
                                                               (const uint16_t *)k, (const uint16_t *)v,
                                                               slots, D, P, H, pages);
        else
            store_kv_int8_kernel<float><<<grid, 64, 0, s>>>(c->layer_q, c->layer_scale, c->smooth,
                                                            (const float *)k, (const float *)v, slots,
                                                            D, P, H, pages);
    } else if (dtype == TI_BF16) {
        store_kv_kernel<uint16_t><<<grid, 64, 0, s>>>((uint16_t *)c->k_pages, (uint16_t *)c->v_pages,
                                                      (const uint16_t *)k, (const uint16_t *)v, slots,
                                                      D, P, H, pages);
    } else {
        store_kv_kernel<float><<<grid, 64, 0, s>>>((float *)c->k_pages, (float *)c->v_pages,
                                                   (const float *)k, (const float *)v, slots, D, P,
                                                   H, pages);
    }
#undef TI_STORE_V
    return hipGetLastError() == hipSuccess ? TI_OK : TI_ERR_LAUNCH;
}

template <typename T, bool NORM, bool INT8>
static void launch_inputs(void *q_out, const ti_kv_cache *c, const void *qkv, const void *q_norm,
                          const void *k_norm, const void *cos_sin, int table_len,
                          const int32_t *positions, const int32_t *slots, int n, int nq,
                          float eps, hipStream_t s) {
    if (c->head_dim == 128 || c->head_dim == 64) {
        const int hpw = 2048 / c->head_dim;   // heads per 256-thread work-group
        dim3 grid(n, (nq + c->kv_heads + hpw - 1) / hpw);
#define TI_INPUTS_V(DD)                                                                            \
    attention_inputs_v_kernel<T, NORM, INT8, DD><<<grid, 256, 0, s>>>(                             \
        (T *)q_out, (T *)c->k_pages, (T *)c->v_pages, c->layer_q, c->layer_scale, c->smooth,        \
        (const T *)qkv, (const T *)q_norm, (const T *)k_norm, (const T *)cos_sin, table_len,        \
        positions, slots, nq, c->kv_heads, c->page_size, c->num_pages, eps);
        if (c->head_dim == 128) { TI_INPUTS_V(128) } else { TI_INPUTS_V(64) }
#undef TI_INPUTS_V
        return;
    }
    dim3 grid(n, nq + c->kv_heads);
    attention_inputs_kernel<T, NORM, INT8><<<grid, 64, 0, s>>>(
        (T *)q_out, (T *)c->k_pages, (T *)c->v_pages, c->layer_q, c->layer_scale, c->smooth,
        (const T *)qkv, (const T *)q_norm, (const T *)k_norm, (const T *)cos_sin, table_len,
        positions, slots, nq, c->kv_heads, c->head_dim, c->page_size, c->num_pages, eps);
}

int ti_launch_attention_inputs(int dtype, void *q_out, const ti_kv_cache *c, const void *qkv,
                               const void *q_norm, const void *k_norm, const void *cos_sin,
                               int table_len, const int32_t *positions, const int32_t *slots,
                               int n, int q_heads, float eps, hipStream_t s) {
    const bool norm = q_norm != nullptr, int8 = c->kind == TI_KV_INT8;
#define TI_INPUTS(T, N, I)                                                                        \
    launch_inputs<T, N, I>(q_out, c, qkv, q_norm, k_norm, cos_sin, table_len, positions, slots, n, \
                           q_heads, eps, s)
    if (dtype == TI_BF16) {
        if (norm) { if (int8) TI_INPUTS(uint16_t, true, true); else TI_INPUTS(uint16_t, true, false); }
        else { if (int8) TI_INPUTS(uint16_t, false, true); else TI_INPUTS(uint16_t, false, false); }
    } else {
        if (norm) { if (int8) TI_INPUTS(float, true, true); else TI_INPUTS(float, true, false); }
        else { if (int8) TI_INPUTS(float, false, true); else TI_INPUTS(float, false, false); }
    }
#undef TI_INPUTS
    return hipGetLastError() == hipSuccess ? TI_OK : TI_ERR_LAUNCH;
}
