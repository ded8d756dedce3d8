// Shared device helpers for the gfx950 (CDNA4) kernels of libtileinfer_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tileinfer_hip.h"

namespace ti {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;
// Finite stand-in for -inf as the initial running max: a row whose keys are all masked
// keeps m = NEG_BIG, l = 0 and gets weight 0 when splits are combined (no inf - inf).
constexpr float NEG_BIG = -3.402823466e38f;
constexpr float LOG2E = 1.4426950408889634f;

// bf16 storage is uint16_t; arithmetic is in float.
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// Round to nearest even (gfx950's v_cvt_pk_bf16_f32 through the __bf16 conversion).
__device__ __forceinline__ uint16_t f2bf(float f) {
    __bf16 h = (__bf16)f;
    return __builtin_bit_cast(uint16_t, h);
}

// Element type traits: load as float, round a float to T (kept as float), store.
template <typename T> struct Elt;
template <> struct Elt<float> {
    static __device__ __forceinline__ float ld(const float *p, size_t i) { return p[i]; }
    static __device__ __forceinline__ float rnd(float x) { return x; }
    static __device__ __forceinline__ void st(float *p, size_t i, float x) { p[i] = x; }
};
template <> struct Elt<uint16_t> {
    static __device__ __forceinline__ float ld(const uint16_t *p, size_t i) { return bf2f(p[i]); }
    static __device__ __forceinline__ float rnd(float x) { return bf2f(f2bf(x)); }
    static __device__ __forceinline__ void st(uint16_t *p, size_t i, float x) { p[i] = f2bf(x); }
};

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two floats -> one word of two bf16 (round to nearest even), low element first: one
// v_cvt_pk_bf16_f32 (a whole-vector conversion, never element inserts).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

// MFMA operands are assembled from 32-bit words and bit-cast whole; building bf16
// vectors element by element has been seen to miscompile (only element 0 kept).
__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 w) { return __builtin_bit_cast(bf16x8, w); }

// 4 int8 (one word) -> 2 words of bf16 (exact).
__device__ __forceinline__ void i8x4_to_bf16(uint32_t v, uint32_t &lo, uint32_t &hi) {
    lo = pack_bf16x2((float)(int8_t)(v), (float)(int8_t)(v >> 8));
    hi = pack_bf16x2((float)(int8_t)(v >> 16), (float)(int8_t)(v >> 24));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Block-table lookup: the index is clamped into the sequence's row [0, bt_stride) and the
// 1-based page id into the pool, so neither a malformed table nor a position past the
// table's width (or a negative one) can send a load outside the table or the pool.
__device__ __forceinline__ int page_of(const int32_t *bt, int idx, int bt_stride, int num_pages) {
    idx = idx < 0 ? 0 : (idx >= bt_stride ? bt_stride - 1 : idx);
    int p = bt[idx] - 1;
    p = p < 0 ? 0 : p;
    return p >= num_pages ? num_pages - 1 : p;
}

// The same lookup for a wave-uniform index, as a scalar load through the constant address
// space: it is counted by lgkmcnt, so waiting for it never waits for the vector loads of
// prefetched tiles (vmcnt is in order).
// Key splits that hold keys when every split takes at least `min_tiles` 16-key tiles (the
// fp32 matrix-core decode): the first `active` of the launch's `splits` work-groups take
// `per` tiles each, the rest have none and write nothing.
struct ActiveSplits {
    int per, active;
};
__device__ __forceinline__ ActiveSplits f32_active_splits(int ntiles, int splits, int min_tiles) {
    const int per = max((ntiles + splits - 1) / splits, min_tiles);
    return {per, (ntiles + per - 1) / per};
}

__device__ __forceinline__ int page_of_s(const int32_t *bt, int idx, int bt_stride, int num_pages) {
    idx = __builtin_amdgcn_readfirstlane(idx);
    idx = idx < 0 ? 0 : (idx >= bt_stride ? bt_stride - 1 : idx);
    const __attribute__((address_space(4))) int32_t *cbt =
        (const __attribute__((address_space(4))) int32_t *)bt;
    int p = cbt[idx] - 1;
    p = p < 0 ? 0 : p;
    return p >= num_pages ? num_pages - 1 : p;
}

// A wave-uniform int32 element as a scalar load (counted by lgkmcnt, never waiting on vector loads).
__device__ __forceinline__ int sload(const int32_t *a, int idx) {
    return ((const __attribute__((address_space(4))) int32_t *)a)[__builtin_amdgcn_readfirstlane(idx)];
}
// A raw block-table entry as a 0-based page inside the pool (as page_of_s).
__device__ __forceinline__ int clamp_page(int raw, int num_pages) { return min(max(raw - 1, 0), num_pages - 1); }

}  // namespace ti

// Launchers implemented per kernel file, dispatched by api.hip.
int ti_launch_rmsnorm(int dtype, void *y, const void *x, const void *w, int rows, int H, float eps,
                      hipStream_t s);
int ti_launch_rope(int dtype, void *y, const void *x, const void *cos_t, const void *sin_t,
                   int table_len, const int32_t *positions, int n, int heads, int D,
                   hipStream_t s);
int ti_launch_store_kv(int dtype, const ti_kv_cache *c, const void *k, const void *v,
                       const int32_t *slots, int n, hipStream_t s);
int ti_launch_attention_inputs(int dtype, void *q_out, const ti_kv_cache *c, const void *qkv,
                               const void *q_norm, const void *k_norm, const void *cos_sin,
                               int table_len, const int32_t *positions, const int32_t *slots,
                               int n, int q_heads, float eps, hipStream_t s);

struct ti_decode_plan {
    int splits;      // split-KV work-groups per (sequence, KV head)
    int waves;       // waves per work-group (4 or 8)
    int rows;        // packed query rows G * max_query_len
    int flat;        // > 0: work-groups per KV head shared out over the sequences by length
    size_t meta;     // flat: byte offset of the per-sequence {first work-group, pieces} table
    size_t bytes;    // workspace bytes
};
ti_decode_plan ti_plan_decode(const ti_attention_args *a, const ti_kv_cache *c);
int ti_launch_decode(const ti_attention_args *a, const ti_kv_cache *c, const ti_decode_plan &p,
                     hipStream_t s);
// Merge split partials [B][Hk][splits][rows][D + 2] from a->workspace into a->out; flat
// mode (flat work-groups per KV head): partials [Hk][flat][rows][D + 2], each sequence's
// pieces located by the decode kernel's table at meta. min_tiles > 0: a sequence's splits
// took at least min_tiles 16-key tiles each, and only those that held keys are merged.
int ti_launch_combine(const ti_attention_args *a, const ti_kv_cache *c, int rows, int splits,
                      hipStream_t s, int flat = 0, int *meta = nullptr, int min_tiles = 0);

struct ti_prefill_plan {
    int pp;          // 1: the 8-wave ping-pong kernel (pa_prefill_pp.hip)
    int dl;          // 1: direct global -> LDS tile loads in the four-wave kernel
    int pair;        // 1: paired heavy / light 32-row q-tiles per work-group (TQ, qtiles per 32 rows)
    int r16;         // 1 (with pair): the paired work-groups on 16-row waves (prefill16_kernel)
    int wpg;         // waves per key group (32 packed rows each)
    int ng;          // key groups per work-group
    int splits;      // key splits across work-groups (partials merged by the combine kernel)
    int TQ;          // query positions per q-tile
    int qtiles;      // q-tiles per (sequence, KV head)
    int rows;        // packed query rows G * max_query_len
    size_t bytes;    // workspace bytes
};
// bound_keys: limit the key splits by the keys the block tables can hold (a launch); the
// workspace query passes false and sizes for the most splits any block-table width allows.
ti_prefill_plan ti_plan_prefill(const ti_attention_args *a, const ti_kv_cache *c, bool bound_keys);
int ti_launch_prefill(const ti_attention_args *a, const ti_kv_cache *c, const ti_prefill_plan &p,
                      hipStream_t s);
bool ti_prefill_pp_eligible(const ti_attention_args *a, const ti_kv_cache *c);
int ti_launch_prefill_pp(const ti_attention_args *a, const ti_kv_cache *c, const ti_prefill_plan &p,
                         hipStream_t s);
// fp32 path: its key splits and workspace bytes (host shapes only).
int ti_plan_generic(const ti_attention_args *a, const ti_kv_cache *c, size_t *bytes);
int ti_launch_generic(const ti_attention_args *a, const ti_kv_cache *c, hipStream_t s);
