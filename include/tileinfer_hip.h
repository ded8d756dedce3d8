/*
 * tileinfer_hip.h — C ABI of libtileinfer_hip.so, the MI355X (gfx950) paged
 * flash-attention path of TileInfer.jl.
 *
 * Every entry point replaces one method of the reference's op interface
 * (src/ops/interface.jl) for its TileBackend kernels; each declaration cites the
 * reference function it stands in for. All pointers are device pointers unless noted;
 * calls enqueue work on `stream` and return without synchronizing. The library never
 * allocates device memory: the caller owns pools, inputs, outputs and the workspace.
 * Errors are returned as ti_status codes, never thrown; argument checks run on the host
 * before any HIP call, so they work without a GPU.
 *
 * Layouts are C-order, i.e. the reference's column-major shapes reversed, so a Julia
 * array is passed with no copy:
 *   per-head tensors (head_dim, heads, n)               -> [n][heads][head_dim]
 *   dense pools (head_dim, page_size, kv_heads, pages)  -> [pages][kv_heads][page_size][head_dim]
 *   INT8 layer arrays (int8_kv_pools, src/ops/quant.jl:104-109):
 *     layer_q     (D, P, Hk, pages, 2) int8             -> [2][pages][Hk][P][D] (keys first)
 *     layer_scale (P, Hk, pages, 2) Float32             -> [2][pages][Hk][P]
 *     smooth      (D,) Float32 (the keys' smoothing; values use ones)
 *   rotary table cos_sin (D, 2 max_len)                 -> [max_len][2][D] (cos, then sin)
 *   block tables: int32, 1-based page ids, zero-padded past a sequence's pages
 *   slots: int32, 1-based, slot s = offset (s-1) % P of page (s-1) / P + 1
 *   positions: int32, 0-based
 */
#ifndef TILEINFER_HIP_H
#define TILEINFER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    TI_OK = 0,
    TI_ERR_INVALID_ARG = 1,     /* null pointer, non-positive size, mismatched shapes */
    TI_ERR_UNSUPPORTED = 2,     /* a shape or type no kernel covers (e.g. head_dim 96) */
    TI_ERR_WORKSPACE = 3,       /* workspace missing or smaller than ti_attention_workspace_bytes */
    TI_ERR_LAUNCH = 4,          /* the HIP launch failed */
} ti_status;

typedef enum { TI_F32 = 0, TI_BF16 = 1 } ti_dtype;      /* activations / dense pools */
typedef enum { TI_KV_DENSE = 0, TI_KV_INT8 = 1 } ti_kv_kind;

/* Path selection for ti_attention. AUTO follows the reference's rule
 * (src/ops/tile/attention.jl:265, :351-352): split-KV decode for short steps, the prefill
 * kernel otherwise. PREFILL takes the prefill family and lets the library pick its
 * variant from host shapes; the last five pin one variant of it (for tests and tuning:
 * every variant gives results within the same tolerances, and pinned variants that the
 * shapes do not allow fall back to the library's pick):
 *   PREFILL_STAGED    four-wave kernel, K/V tiles staged through registers into LDS
 *   PREFILL_DIRECT    four-wave kernel, direct global -> LDS tile loads (bf16 dense cache,
 *                     head_dim 128, pages of 2^k >= 16 tokens; otherwise staged)
 *   PREFILL_PINGPONG  eight-wave ping-pong kernel (bf16 dense cache, head_dim 128, pages
 *                     of 2^k >= 16 tokens, 256 % (q_heads / kv_heads) == 0)
 *   PREFILL_PAIRED    four-wave kernel with direct loads whose work-groups each take a
 *                     heavy and a light 32-row q-tile of a causal step (direct-load shapes,
 *                     32 % (q_heads / kv_heads) == 0, the shapes' unsplit two-wave plan)
 *   PREFILL_PAIRED16  the same paired work-groups on sixteen waves of 16 rows each (four
 *                     per SIMD; the default where the paired plan applies) */
typedef enum {
    TI_PATH_AUTO = 0,
    TI_PATH_DECODE = 1,
    TI_PATH_PREFILL = 2,
    TI_PATH_PREFILL_STAGED = 3,
    TI_PATH_PREFILL_DIRECT = 4,
    TI_PATH_PREFILL_PINGPONG = 5,
    TI_PATH_PREFILL_PAIRED = 6,
    TI_PATH_PREFILL_PAIRED16 = 7,
} ti_path;

/* One layer's KV cache: dense pools in the activations' type, or an INT8 layer
 * (Int8Pages pair: src/ops/quant.jl:86-92). Host struct of device pointers. */
typedef struct {
    int32_t kind;               /* ti_kv_kind */
    int32_t head_dim;           /* D: 64 or 128 */
    int32_t page_size;          /* P: positions per page (any >= 1; 16 and 64 are tuned) */
    int32_t kv_heads;           /* Hk */
    int32_t num_pages;          /* pages in the pool; page ids are 1..num_pages */
    void *k_pages;              /* dense: [num_pages][Hk][P][D] */
    void *v_pages;
    int8_t *layer_q;            /* int8: [2][num_pages][Hk][P][D] */
    float *layer_scale;         /* int8: [2][num_pages][Hk][P] */
    const float *smooth;        /* int8: [D] keys' smoothing factors */
} ti_kv_cache;

/* Arguments of ti_attention. A batch of `num_seqs` sequences; sequence b owns the query
 * tokens [qsl[b], qsl[b+1]) of q (or [b*max_query_len, (b+1)*max_query_len) when
 * query_start_loc is NULL), its first query sits at positions[qsl[b]] and it attends to
 * keys 0 .. positions[qsl[b]] + n_b - 1 through block table row b. num_seqs = 1 is
 * exactly the reference's one-sequence op.
 * Contract on the device data (not checkable on the host): a row of block_tables must hold
 * at least ceil(len / page_size) page ids for the sequence's len = positions[qsl[b]] + n_b
 * keys, and n_b <= max_query_len. Out of contract, no access leaves the block-table row or
 * the pool (page indices are clamped to [0, block_table_stride), page ids to the pool,
 * n_b to max_query_len), but the output is unspecified. */
typedef struct {
    int32_t dtype;                    /* ti_dtype of q, out (and dense pools) */
    int32_t q_heads;                  /* Hq; Hq % Hk == 0 */
    int32_t num_seqs;                 /* B */
    int32_t max_query_len;            /* max n_b (sizes the grid; host value) */
    int32_t total_tokens;             /* sum n_b (rows of q and out) */
    int32_t block_table_stride;       /* entries per block-table row */
    const void *q;                    /* [total_tokens][Hq][D] */
    void *out;                        /* [total_tokens][Hq][D] */
    const int32_t *positions;         /* [total_tokens] 0-based positions */
    const int32_t *query_start_loc;   /* [B+1] token offsets, or NULL: uniform max_query_len */
    const int32_t *block_tables;      /* [B][block_table_stride] 1-based page ids */
    float scale;                      /* softmax scale, e.g. 1/sqrt(D); finite and > 0 */
    int32_t causal;                   /* 1: key i visible to query t iff i <= pos(t) */
    int32_t path;                     /* ti_path */
    void *workspace;                  /* split-KV partials; may be NULL for the prefill path */
    size_t workspace_bytes;
} ti_attention_args;

/* Library version string, e.g. "tileinfer_hip 0.1.0 gfx950". Host only. */
const char *ti_version(void);

/* Human-readable name of a status code. Host only. */
const char *ti_status_string(int status);

/*
 * Bytes of workspace ti_attention needs for these shapes (0 when the call needs none).
 * Replaces attention_workspace(::TileBackend, q, k_pages) and decode_workspace
 * (src/ops/tile/attention.jl:279-284, :351-352; interface src/ops/interface.jl:275-280).
 * Like the reference's, it depends only on the query shape (dtype, q_heads, num_seqs,
 * max_query_len, path) and the cache, never on the block tables or context length, so
 * a captured graph keeps a fixed workspace. Host only; writes the size to *bytes.
 */
int ti_attention_workspace_bytes(const ti_attention_args *args, const ti_kv_cache *cache,
                                 size_t *bytes);

/*
 * Paged causal (or non-causal) grouped-query attention over the KV cache.
 * Replaces attention!(::TileBackend, out, workspace, q, k_pages, v_pages, block_table,
 * positions, scale; causal) (src/ops/tile/attention.jl:359-366; interface
 * src/ops/interface.jl:152-158) and the allocating attention(...) when the caller
 * provides out and workspace (attention.jl:368-371). Kernels: split-KV decode + combine
 * (attention.jl:185-245) and the causal / chunked / non-causal prefill
 * (attention.jl:130-177), each for dense (bf16, fp32) and INT8 caches.
 * `stream` is a hipStream_t (NULL = default stream).
 */
int ti_attention(const ti_attention_args *args, const ti_kv_cache *cache, void *stream);

/* Bytes of the static device scratch behind ti_attention_noalloc (per GPU). */
#define TI_NOALLOC_SCRATCH_BYTES (32u << 20)

/*
 * ti_attention without a caller workspace and without any allocation: split-KV partials
 * go to a static device array of TI_NOALLOC_SCRATCH_BYTES per GPU (the library's own,
 * held until the process ends). No counterpart in the reference: this is for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). It calls no hipMalloc / hipFree and no allocating library routine.
 * Same arguments, kernels and results as ti_attention with a sufficient workspace;
 * args->workspace and args->workspace_bytes are ignored. Where the workspace
 * (ti_attention_workspace_bytes) exceeds the scratch, prefill and fp32 steps run unsplit
 * (as ti_attention does without a workspace) and decode steps, whose workspace is
 * mandatory, are rejected with TI_ERR_WORKSPACE before anything is launched. Every call on
 * one GPU shares that GPU's scratch: calls that overlap on one GPU (several streams,
 * several host threads) race and must be serialized by the caller. Nothing in the scratch
 * needs clearing between calls (every partial a launch reads is written by the same
 * launch). `stream` must belong to the current device (TI_ERR_INVALID_ARG otherwise).
 * The scratch is reserved on every GPU where the library's code object is loaded, whether
 * or not this entry point is called.
 */
int ti_attention_noalloc(const ti_attention_args *args, const ti_kv_cache *cache, void *stream);

/*
 * Write keys and values of n tokens at 1-based slots, bit-exact copies (dense) or
 * quantized per (token, KV head) vector (INT8: q = floor(x 127/max|x| + 1/2),
 * s = max|x|/127, keys divided by smooth first).
 * Replaces store_kv!(::TileBackend, k_pages, v_pages, k, v, slots)
 * (src/ops/tile/elementwise.jl:133-140 and :180-188; reference
 * src/ops/reference.jl:64-74, src/ops/quant.jl:147-159).
 * k, v: [n][Hk][D] in dtype. Slots outside the pool are skipped.
 */
int ti_store_kv(int dtype, const ti_kv_cache *cache, const void *k, const void *v,
                const int32_t *slots, int n, void *stream);

/*
 * RMS normalization of `rows` rows of `hidden` elements: y = rnd(rnd(x inv_rms) w) with
 * inv_rms = 1 / sqrt(sum x^2 / hidden + eps) in Float32, rnd = round to T (y may alias x).
 * Replaces rmsnorm!(::TileBackend, y, x, w, eps) (src/ops/tile/norm.jl:31-38; interface
 * src/ops/interface.jl:118-122), the q/k norm of the generic attention_inputs! chain
 * (interface.jl:175). Per-head rows (hidden <= 128) are bit-identical to the norm inside
 * ti_attention_inputs. x, y: [rows][hidden], w: [hidden], all in dtype.
 */
int ti_rmsnorm(int dtype, void *y, const void *x, const void *w, int rows, int hidden, float eps,
               void *stream);

/*
 * Rotary embedding ("rotate half") of x [n][heads][D] into y at 0-based positions,
 * rounding to T after every operation as the reference does.
 * Replaces rope!(::TileBackend, y, x, cos, sin, positions)
 * (src/ops/tile/elementwise.jl:10-36; reference src/ops/reference.jl:32-39).
 * cos_table, sin_table: [table_len][D]. Tokens whose position lies outside [0, table_len)
 * are skipped: their rows of y are left untouched (the reference indexes past its table
 * there; a kernel cannot raise, so the row keeps what it held).
 */
int ti_rope(int dtype, void *y, const void *x, const void *cos_table, const void *sin_table,
            int table_len, const int32_t *positions, int n, int heads, int head_dim, void *stream);

/*
 * Everything between the fused qkv projection and attention, in one launch: optional
 * Qwen3 q/k RMSNorm, RoPE at positions, queries into q_out, keys and values into the
 * cache at slots (quantized for an INT8 cache).
 * Replaces attention_inputs!(::TileBackend, q, k_pages, v_pages, qkv, q_norm, k_norm,
 * table, positions, slots, eps) (src/ops/tile/fused.jl:94-130; generic chain
 * src/ops/interface.jl:169-179).
 * qkv: [n][q_heads + 2 Hk][D]; q_out: [n][q_heads][D]; q_norm, k_norm: [D] or both NULL;
 * cos_sin: [table_len][2][D]. A token whose position lies outside [0, table_len) writes
 * nothing (its q_out rows are left untouched and its K/V slot is not written); a token
 * whose slot lies outside the pool writes no K/V row.
 */
int ti_attention_inputs(int dtype, void *q_out, const ti_kv_cache *cache, const void *qkv,
                        const void *q_norm, const void *k_norm, const void *cos_sin,
                        int table_len, const int32_t *positions, const int32_t *slots, int n,
                        int q_heads, float eps, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TILEINFER_HIP_H */
