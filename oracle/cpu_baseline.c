/*
 * CPU BASELINE ONLY (timed by bench.py's cpu_baseline leg; never a checker, never the
 * product). The reference's eager attention op (src/ops/reference.jl:76-121) on Float32
 * host arrays: for each sequence and KV head, gather the sequence's keys and values
 * through the block table (gather_pages, reference.jl:80-93), then for each of the G query
 * heads of that KV head and each query token: scores K^T q * scale, causal mask, softmax,
 * V p. The gather is a table of row pointers into the pools (no copy of the rows). The
 * reference runs the two products as BLAS matrix products; here they are vectorizable
 * loops, and the file is compiled with -O3 -march=native -ffast-math for the host it runs
 * on, so the compiler may reassociate the sums as a BLAS kernel does.
 * OpenMP over (sequence, KV head).
 *
 * q/out: [sum n_b][Hq][D]; pools [pages][Hk][P][D]; block tables [B][bt_stride], 1-based;
 * starts[B] (position of each sequence's first query), counts[B] (its query tokens).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

void cb_attention_f32_batch(float *out, const float *q, const float *k_pages, const float *v_pages,
                            const int32_t *bts, int bt_stride, const int32_t *starts,
                            const int32_t *counts, int B, int Hq, int Hk, int D, int P,
                            float scale, int causal, int threads) {
    int *offs = (int *)malloc(sizeof(int) * (B + 1));
    offs[0] = 0;
    for (int b = 0; b < B; b++) offs[b + 1] = offs[b] + counts[b];
    const int G = Hq / Hk;
#pragma omp parallel for collapse(2) schedule(dynamic) num_threads(threads)
    for (int b = 0; b < B; b++)
        for (int h = 0; h < Hk; h++) {
            const int start = starts[b], n = counts[b], len = start + n;
            const int32_t *bt = bts + (size_t)b * bt_stride;
            /* gathered rows of this KV head: key i is row[i] of either pool */
            size_t *row = (size_t *)malloc(sizeof(size_t) * len);
            float *sc = (float *)malloc(sizeof(float) * len);
            for (int i = 0; i < len; i++) row[i] = (((size_t)(bt[i / P] - 1) * Hk + h) * P + i % P) * D;
            for (int t = 0; t < n; t++)
                for (int g = 0; g < G; g++) {
                    const int hq = h * G + g;
                    const float *qv = q + ((size_t)(offs[b] + t) * Hq + hq) * D;
                    const int last = causal ? start + t : len - 1;
                    float mx = -INFINITY;
                    for (int i = 0; i <= last; i++) {
                        const float *kr = k_pages + row[i];
                        float s = 0.0f;
                        for (int d = 0; d < D; d++) s += kr[d] * qv[d];
                        s *= scale;
                        sc[i] = s;
                        mx = s > mx ? s : mx;
                    }
                    float sum = 0.0f;
                    for (int i = 0; i <= last; i++) {
                        sc[i] = expf(sc[i] - mx);
                        sum += sc[i];
                    }
                    const float inv = 1.0f / sum;
                    float *o = out + ((size_t)(offs[b] + t) * Hq + hq) * D;
                    for (int d = 0; d < D; d++) o[d] = 0.0f;
                    for (int i = 0; i <= last; i++) {
                        const float *vr = v_pages + row[i];
                        const float p = sc[i] * inv;
                        for (int d = 0; d < D; d++) o[d] += vr[d] * p;
                    }
                }
            free(row);
            free(sc);
        }
    free(offs);
}
