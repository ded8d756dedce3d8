/*
 * CPU oracle for the paged flash-attention path: a plain-C restatement of the
 * reference's Julia ops, used ONLY as the checker in tests/, by
 * __graft_entry__.smoke() and as bench.py's cpu_baseline leg. It is test
 * infrastructure, never the product: nothing in the HIP library links it.
 *
 * All arrays are C-order (the reference's column-major shapes reversed):
 *   per-head tensors q/k/v/out  [n][heads][D]
 *   dense page pools            [pages][kv_heads][P][D]
 *   INT8 layer arrays           q: [2][pages][kv_heads][P][D] int8 (keys first)
 *                               scale: [2][pages][kv_heads][P] f32, smooth: [D] f32
 *   rotary table cos_sin        [max_len][2][D] (row 2p = cos, 2p+1 = sin)
 *   block tables                int32, 1-based page ids, zero padded
 *   slots                       int32, 1-based: slot s -> page (s-1)/P, offset (s-1)%P
 * Values of element type T are carried as float; `bf16` != 0 means T = BFloat16 and
 * every op of the reference rounds its result to bf16 (round to nearest even).
 *
 * Compiled with -ffp-contract=off: the reference's broadcasts never fuse a*b+c.
 *
 * Parity pins (tests/test_oracle.py): the reference's own known-answer loops
 * (test/ops/reference.jl:29-42, :91-99, :101-119), INT8 known answers
 * (test/ops/tile.jl:76-81, src/ops/quant.jl:141-145), closed forms and invariants
 * of softmax attention (constant V, single visible key, q = 0, block-table
 * permutation, GQA head mapping) and brute force at tiny sizes.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

/* Round a float to the nearest bf16 (ties to even), returned as float.
 * BFloat16s.jl's Float32 -> BFloat16 conversion (RNE); NaN stays NaN. */
float or_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return x;          /* NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    float y;
    memcpy(&y, &u, 4);
    return y;
}

static inline float rnd(float x, int bf16) { return bf16 ? or_bf16(x) : x; }

/* rope(::RefBackend): src/ops/reference.jl:32-39 (rotate half; every op rounds to T:
 * y1 = rnd(rnd(x1 c) + rnd(-x2 s)), y2 = rnd(rnd(x2 c) + rnd(x1 s))).
 * cos/sin: [max_len][D]; positions 0-based. */
void or_rope(int bf16, float *y, const float *x, const float *cos_t, const float *sin_t,
             const int32_t *positions, int n, int heads, int D) {
    int half = D / 2;
    for (int t = 0; t < n; t++) {
        const float *c = cos_t + (size_t)positions[t] * D;
        const float *s = sin_t + (size_t)positions[t] * D;
        for (int h = 0; h < heads; h++) {
            const float *xi = x + ((size_t)t * heads + h) * D;
            float *yi = y + ((size_t)t * heads + h) * D;
            for (int i = 0; i < half; i++) {
                float a = xi[i], b = xi[i + half];
                float y1 = rnd(rnd(a * c[i], bf16) + rnd(-b * s[i], bf16), bf16);
                float y2 = rnd(rnd(b * c[i + half], bf16) + rnd(a * s[i + half], bf16), bf16);
                yi[i] = y1;
                yi[i + half] = y2;
            }
        }
    }
}

/* Flat destination row of (slot, head) in a [pages][H][P][D] pool:
 * src/ops/reference.jl:61-70 (column o + P h + P H page, 0-based). */
static inline size_t slot_row(int32_t slot, int h, int P, int H) {
    int64_t s = (int64_t)slot - 1;
    return (size_t)((s % P) + (int64_t)P * h + (int64_t)P * H * (s / P));
}

/* store_kv!(::RefBackend) dense: src/ops/reference.jl:64-74. k, v: [n][H][D]. */
void or_store_kv(float *k_pages, float *v_pages, const float *k, const float *v,
                 const int32_t *slots, int n, int D, int P, int H) {
    for (int t = 0; t < n; t++)
        for (int h = 0; h < H; h++) {
            size_t row = slot_row(slots[t], h, P, H);
            memcpy(k_pages + row * D, k + ((size_t)t * H + h) * D, sizeof(float) * D);
            memcpy(v_pages + row * D, v + ((size_t)t * H + h) * D, sizeof(float) * D);
        }
}

/* quantize_columns: src/ops/quant.jl:141-145 for one vector x[D] (Float32):
 * absmax = max|x|; inv = absmax > 0 ? 127/absmax : 0; q = Int8(floor(x inv + 1/2));
 * s = absmax / 127. */
void or_quantize_vector(const float *x, int D, int8_t *q, float *s) {
    float absmax = 0.0f;
    for (int i = 0; i < D; i++) {
        float a = fabsf(x[i]);
        if (a > absmax) absmax = a;
    }
    float inv = absmax > 0.0f ? 127.0f / absmax : 0.0f;
    for (int i = 0; i < D; i++) {
        float prod = x[i] * inv;
        float shifted = prod + 0.5f;
        q[i] = (int8_t)floorf(shifted);
    }
    *s = absmax / 127.0f;
}

/* store_kv!(::RefBackend, ::Int8Pages...): src/ops/quant.jl:147-159. Keys are divided
 * by smooth (per channel) before quantizing; values are not (their smooth is ones). */
void or_store_kv_int8(int8_t *layer_q, float *layer_scale, const float *smooth,
                      const float *k, const float *v, const int32_t *slots,
                      int n, int D, int P, int H, int pages) {
    size_t half_q = (size_t)pages * H * P * D, half_s = (size_t)pages * H * P;
    float *x = (float *)malloc(sizeof(float) * D);
    for (int t = 0; t < n; t++)
        for (int h = 0; h < H; h++) {
            size_t row = slot_row(slots[t], h, P, H);
            const float *kk = k + ((size_t)t * H + h) * D;
            for (int i = 0; i < D; i++) x[i] = kk[i] / smooth[i];
            or_quantize_vector(x, D, layer_q + row * D, layer_scale + row);
            or_quantize_vector(v + ((size_t)t * H + h) * D, D, layer_q + half_q + row * D,
                               layer_scale + half_s + row);
        }
    free(x);
}

/* rmsnorm(::RefBackend) of one head vector, as used by attention_inputs! with q/k norm:
 * src/ops/reference.jl:17-21 and the fused kernel's rounding points
 * src/ops/tile/fused.jl:20-27: y = rnd(rnd(x inv_rms) w), inv_rms in Float32.
 * The sum of squares is accumulated in double here (order-free); the HIP kernel's
 * Float32 tree sum may differ by one Float32 ulp of inv_rms. */
static void norm_vec(int bf16, float *y, const float *x, const float *w, int D, float eps) {
    double ss = 0.0;
    for (int i = 0; i < D; i++) ss += (double)x[i] * x[i];
    float mean = (float)ss / (float)D;
    float inv_rms = 1.0f / sqrtf(mean + eps);
    for (int i = 0; i < D; i++) y[i] = rnd(rnd(x[i] * inv_rms, bf16) * w[i], bf16);
}

/* One head of attention_inputs!: optional norm then rope at position pos.
 * cos_sin: [max_len][2][D]. src/ops/tile/fused.jl:15-34. */
static void norm_rope_vec(int bf16, float *y, const float *x, const float *w, int norm,
                          float eps, const float *cos_sin, int32_t pos, int D) {
    float *tmp = (float *)malloc(sizeof(float) * D);
    if (norm) norm_vec(bf16, tmp, x, w, D, eps);
    else memcpy(tmp, x, sizeof(float) * D);
    const float *c = cos_sin + (size_t)pos * 2 * D;
    const float *s = c + D;
    int half = D / 2;
    for (int i = 0; i < half; i++) {
        float a = tmp[i], b = tmp[i + half];
        y[i] = rnd(rnd(a * c[i], bf16) + rnd(-b * s[i], bf16), bf16);
        y[i + half] = rnd(rnd(b * c[i + half], bf16) + rnd(a * s[i + half], bf16), bf16);
    }
    free(tmp);
}

/* attention_inputs! (generic chain, src/ops/interface.jl:169-179; fused tile version
 * src/ops/tile/fused.jl:39-130): qkv [n][nq + 2 nkv][D] -> q [n][nq][D], and keys
 * (normed, rotated) and values into the pools at slots. int8 != 0 writes the INT8 layer
 * arrays (keys divided by smooth, src/ops/tile/fused.jl:74-92) instead of dense pools. */
void or_attention_inputs(int bf16, float *q_out, float *k_pages, float *v_pages,
                         int8_t *layer_q, float *layer_scale, const float *smooth, int int8,
                         const float *qkv, const float *q_norm, const float *k_norm, int norm,
                         const float *cos_sin, const int32_t *positions, const int32_t *slots,
                         int n, int nq, int nkv, int D, int P, int pages, float eps) {
    int all = nq + 2 * nkv;
    float *y = (float *)malloc(sizeof(float) * D);
    for (int t = 0; t < n; t++) {
        const float *base = qkv + (size_t)t * all * D;
        for (int j = 0; j < nq; j++)
            norm_rope_vec(bf16, q_out + ((size_t)t * nq + j) * D, base + (size_t)j * D, q_norm,
                          norm, eps, cos_sin, positions[t], D);
        for (int h = 0; h < nkv; h++) {
            norm_rope_vec(bf16, y, base + (size_t)(nq + h) * D, k_norm, norm, eps, cos_sin,
                          positions[t], D);
            const float *vv = base + (size_t)(nq + nkv + h) * D;
            if (!int8) {
                size_t row = slot_row(slots[t], h, P, nkv);
                memcpy(k_pages + row * D, y, sizeof(float) * D);
                memcpy(v_pages + row * D, vv, sizeof(float) * D);
            } else {
                /* as store_kv!(::RefBackend, ::Int8Pages) of one (token, head) */
                size_t half_q = (size_t)pages * nkv * P * D, half_s = (size_t)pages * nkv * P;
                size_t row = slot_row(slots[t], h, P, nkv);
                for (int i = 0; i < D; i++) y[i] = y[i] / smooth[i];
                or_quantize_vector(y, D, layer_q + row * D, layer_scale + row);
                or_quantize_vector(vv, D, layer_q + half_q + row * D, layer_scale + half_s + row);
            }
        }
    }
    free(y);
}

/* The 0-based key i of KV head g of a sequence: row in the pool through the block
 * table (src/ops/reference.jl:80-84; position p lives in page table[p / P], offset p % P,
 * src/kv/block_manager.jl:1-5). */
static inline size_t key_row(const int32_t *bt, int i, int g, int P, int H) {
    int page0 = bt[i / P] - 1;
    return ((size_t)page0 * H + g) * P + (i % P);
}

/* Dequantized key/value element, as gather_pages(::Int8Pages): src/ops/quant.jl:165-170:
 * Float32(q) * scale * smooth, each product rounded in Float32. */
static inline float deq(const int8_t *lq, const float *ls, const float *smooth, size_t row,
                        int D, int i) {
    return ((float)lq[row * D + i] * ls[row]) * smooth[i];
}

/*
 * attention(::RefBackend) for ONE sequence: src/ops/reference.jl:95-121.
 * q [n][Hq][D]; start = positions[1] (0-based position of the first query); query t sees
 * keys 0..start+t (causal) or 0..start+n-1 (not causal), reference.jl:105-107.
 * GQA: query head h uses KV head h / G (reference.jl:108-109).
 * mode 0: exact (double accumulation, no rounding: the fp32-accumulated reference of
 *         the tolerance contract, computed in double).
 * mode 1: eager (reference.jl:113-117 rounding points: S = rnd(rnd(KᵀQ) rnd(scale)),
 *         Float32 softmax, P = rnd(P), O = rnd(V P)), Float32 accumulation.
 * int8 != 0: keys/values come from the INT8 layer arrays, dequantized in Float32.
 */
void or_attention(int mode, int bf16, float *out, const float *q, const float *k_pages,
                  const float *v_pages, const int8_t *layer_q, const float *layer_scale,
                  const float *smooth, int int8, int pages, const int32_t *bt, int start, int n,
                  int Hq, int Hk, int D, int P, float scale, int causal) {
    int G = Hq / Hk, len = start + n;
    size_t half_q = (size_t)pages * Hk * P * D, half_s = (size_t)pages * Hk * P;
    double *sc = (double *)malloc(sizeof(double) * (len > 0 ? len : 1));
    double *acc = (double *)malloc(sizeof(double) * D);
    float scale_t = rnd(scale, bf16);
    for (int h = 0; h < Hq; h++) {
        int g = h / G;
        for (int t = 0; t < n; t++) {
            const float *qv = q + ((size_t)t * Hq + h) * D;
            int last = causal ? start + t : len - 1;       /* keys 0..last visible */
            double mx = -INFINITY;
            for (int i = 0; i <= last; i++) {
                size_t row = key_row(bt, i, g, P, Hk);
                if (mode == 0) {
                    double s = 0.0;
                    for (int d = 0; d < D; d++) {
                        double kd = int8 ? deq(layer_q, layer_scale, smooth, row, D, d) : k_pages[row * D + d];
                        s += kd * (double)qv[d];
                    }
                    sc[i] = s * (double)scale;
                } else {
                    float s = 0.0f;
                    for (int d = 0; d < D; d++) {
                        float kd = int8 ? deq(layer_q, layer_scale, smooth, row, D, d) : k_pages[row * D + d];
                        s += kd * qv[d];
                    }
                    sc[i] = rnd(rnd(s, bf16) * scale_t, bf16);
                }
                if (sc[i] > mx) mx = sc[i];
            }
            double sum = 0.0;
            for (int i = 0; i <= last; i++) {
                sc[i] = mode == 0 ? exp(sc[i] - mx) : (double)expf((float)(sc[i] - mx));
                sum += sc[i];
            }
            for (int d = 0; d < D; d++) acc[d] = 0.0;
            for (int i = 0; i <= last; i++) {
                double p = mode == 0 ? sc[i] / sum : (double)rnd((float)(sc[i] / sum), bf16);
                size_t row = key_row(bt, i, g, P, Hk);
                for (int d = 0; d < D; d++) {
                    /* values' smoothing is ones: (q s) 1 = q s */
                    double val = int8 ? (double)((float)layer_q[half_q + row * D + d] * layer_scale[half_s + row])
                                      : (double)v_pages[row * D + d];
                    acc[d] += val * p;
                }
            }
            float *o = out + ((size_t)t * Hq + h) * D;
            for (int d = 0; d < D; d++) o[d] = mode == 0 ? (float)acc[d] : rnd((float)acc[d], bf16);
        }
    }
    free(sc);
    free(acc);
}

