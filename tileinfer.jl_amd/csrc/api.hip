// C ABI of libtileinfer_hip: argument validation (host only, before any HIP call) and
// dispatch to the kernels. See include/tileinfer_hip.h for the contract of each entry.
#include <mutex>

#include "common.hpp"

// Device scratch of ti_attention_noalloc: split-KV partials live here instead of in a
// caller's workspace. One copy per GPU, allocated when the library's code object is
// loaded on that GPU and held until the process ends. In host code `scratch` only names
// the symbol; its device address (per GPU) comes from hipGetSymbolAddress.
static __device__ __align__(256) char scratch[TI_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex scratch_mu;
void *scratch_ptr[MAX_DEVICES];   // device address of `scratch` on each GPU, once looked up

// The current GPU's scratch address: looked up once per GPU (with that GPU current, on
// its first no-alloc call), then cached. No allocation happens here.
int device_scratch(void **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return TI_ERR_LAUNCH;
    if (dev < 0 || dev >= MAX_DEVICES) return TI_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return TI_ERR_LAUNCH;
        scratch_ptr[dev] = p;
    }
    *out = scratch_ptr[dev];
    return TI_OK;
}

bool bad_cache(const ti_kv_cache *c) {
    if (!c) return true;
    if (c->kind != TI_KV_DENSE && c->kind != TI_KV_INT8) return true;
    if (c->head_dim <= 0 || (c->head_dim & 1) || c->page_size <= 0 || c->kv_heads <= 0 ||
        c->num_pages <= 0)
        return true;
    if (c->kind == TI_KV_DENSE && (!c->k_pages || !c->v_pages)) return true;
    if (c->kind == TI_KV_INT8 && (!c->layer_q || !c->layer_scale || !c->smooth)) return true;
    return false;
}

bool bad_dtype(int dtype) { return dtype != TI_F32 && dtype != TI_BF16; }

// Resolve the kernel family of an attention call: 0 generic (fp32), 1 decode, 2 prefill,
// or a negative ti_status. AUTO takes the decode kernel for up to 32 packed query rows
// (and for one query token with up to 64 heads per KV head); larger multi-token steps,
// such as speculative verify, run faster on the prefill kernel with key splits, which
// stages each K/V tile once in LDS for all its rows.
int resolve_path(const ti_attention_args *a, const ti_kv_cache *c) {
    const int G = a->q_heads / c->kv_heads;
    if (a->dtype == TI_F32) return 0;
    const int rows = G * a->max_query_len;
    const bool decode_ok = rows <= 64;
    const bool decode_auto = a->max_query_len <= 16 && (rows <= 32 || (a->max_query_len == 1 && decode_ok));
    switch (a->path) {
        case TI_PATH_AUTO: return decode_auto ? 1 : (G <= 64 ? 2 : -TI_ERR_UNSUPPORTED);
        case TI_PATH_DECODE: return decode_ok ? 1 : -TI_ERR_UNSUPPORTED;
        case TI_PATH_PREFILL:
        case TI_PATH_PREFILL_STAGED:
        case TI_PATH_PREFILL_DIRECT:
        case TI_PATH_PREFILL_PINGPONG:
        case TI_PATH_PREFILL_PAIRED:
        case TI_PATH_PREFILL_PAIRED16: return G <= 64 ? 2 : -TI_ERR_UNSUPPORTED;
        default: return -TI_ERR_INVALID_ARG;
    }
}

int check_attention(const ti_attention_args *a, const ti_kv_cache *c) {
    if (!a || bad_cache(c) || bad_dtype(a->dtype)) return TI_ERR_INVALID_ARG;
    if (c->head_dim != 64 && c->head_dim != 128) return TI_ERR_UNSUPPORTED;
    if (a->q_heads <= 0 || a->q_heads % c->kv_heads) return TI_ERR_INVALID_ARG;
    if (a->num_seqs <= 0 || a->max_query_len <= 0 || a->total_tokens <= 0 ||
        a->block_table_stride <= 0)
        return TI_ERR_INVALID_ARG;
    if (!a->q || !a->out || !a->positions || !a->block_tables) return TI_ERR_INVALID_ARG;
    if (!a->query_start_loc && (long long)a->num_seqs * a->max_query_len != a->total_tokens)
        return TI_ERR_INVALID_ARG;
    if (a->causal != 0 && a->causal != 1) return TI_ERR_INVALID_ARG;
    // A finite positive softmax scale (1/sqrt(D) or a model's own): the MFMA kernels take
    // each tile's running max on unscaled scores, which needs scale > 0.
    if (!(a->scale > 0.0f) || a->scale == INFINITY) return TI_ERR_INVALID_ARG;
    // launch grids put sequences in a dimension of at most 65535
    if (a->num_seqs > 65535) return TI_ERR_UNSUPPORTED;
    return TI_OK;
}

// Grid y of a prefill launch: paired plans hold two q-tiles per work-group, the others one
// q-tile per key split. At most 65535.
long long prefill_grid_y(const ti_prefill_plan &pl) {
    return pl.pair ? (pl.qtiles + 1LL) / 2 : (long long)pl.qtiles * pl.splits;
}

}  // namespace

extern "C" {

const char *ti_version(void) { return "tileinfer_hip 0.1.0 gfx950"; }

const char *ti_status_string(int status) {
    switch (status) {
        case TI_OK: return "ok";
        case TI_ERR_INVALID_ARG: return "invalid argument";
        case TI_ERR_UNSUPPORTED: return "unsupported shape or type";
        case TI_ERR_WORKSPACE: return "workspace missing or too small";
        case TI_ERR_LAUNCH: return "kernel launch failed";
        default: return "unknown status";
    }
}

int ti_attention_workspace_bytes(const ti_attention_args *a, const ti_kv_cache *c, size_t *bytes) {
    if (!bytes) return TI_ERR_INVALID_ARG;
    *bytes = 0;
    int st = check_attention(a, c);
    if (st) return st;
    const int path = resolve_path(a, c);
    if (path < 0) return -path;
    if (path == 0) ti_plan_generic(a, c, bytes);
    if (path == 1) *bytes = ti_plan_decode(a, c).bytes;
    if (path == 2) {
        ti_prefill_plan pp = ti_plan_prefill(a, c, false);
        if (prefill_grid_y(pp) > 65535) pp.splits = 1, pp.bytes = 0;   // runs unsplit
        if (prefill_grid_y(pp) > 65535) return TI_ERR_UNSUPPORTED;
        *bytes = pp.bytes;
    }
    return TI_OK;
}

int ti_attention(const ti_attention_args *a, const ti_kv_cache *c, void *stream) {
    int st = check_attention(a, c);
    if (st) return st;
    const int path = resolve_path(a, c);
    if (path < 0) return -path;
    hipStream_t s = (hipStream_t)stream;
    if (path == 0) return ti_launch_generic(a, c, s);
    if (path == 2) {
        // The prefill path never requires a workspace (the reference runs its prefill
        // kernel exactly when none is passed); without one it runs unsplit.
        ti_prefill_plan pp = ti_plan_prefill(a, c, true);
        if (prefill_grid_y(pp) > 65535) pp.splits = 1, pp.bytes = 0;
        if (prefill_grid_y(pp) > 65535) return TI_ERR_UNSUPPORTED;   // q-tiles share grid y
        if (pp.bytes > 0 && (!a->workspace || a->workspace_bytes < pp.bytes)) {
            pp.splits = 1;
            pp.bytes = 0;
        }
        return ti_launch_prefill(a, c, pp, s);
    }
    const ti_decode_plan pl = ti_plan_decode(a, c);
    if (pl.bytes > 0 && (!a->workspace || a->workspace_bytes < pl.bytes)) return TI_ERR_WORKSPACE;
    return ti_launch_decode(a, c, pl, s);
}

int ti_attention_noalloc(const ti_attention_args *a, const ti_kv_cache *c, void *stream) {
    // The same validation and the same plan as ti_attention. The plan's workspace (sized
    // as ti_attention_workspace_bytes, which bounds every launch of these shapes) comes from
    // the static scratch when it fits. Prefill and fp32 steps whose split partials would not
    // fit run unsplit, as ti_attention does without a workspace; a decode step, whose
    // workspace is mandatory, is rejected before any HIP call.
    size_t need = 0;
    int st = ti_attention_workspace_bytes(a, c, &need);
    if (st) return st;
    if (need > (size_t)TI_NOALLOC_SCRATCH_BYTES) {
        if (resolve_path(a, c) == 1) return TI_ERR_WORKSPACE;
        need = 0;
    }
    // The scratch address is per GPU: the stream must belong to the current GPU.
    if (stream) {
        int sdev = -1, dev = -1;
        if (hipStreamGetDevice((hipStream_t)stream, &sdev) != hipSuccess || hipGetDevice(&dev) != hipSuccess)
            return TI_ERR_INVALID_ARG;
        if (sdev != dev) return TI_ERR_INVALID_ARG;
    }
    ti_attention_args local = *a;
    local.workspace = nullptr;
    local.workspace_bytes = 0;
    if (need > 0) {
        st = device_scratch(&local.workspace);
        if (st) return st;
        local.workspace_bytes = TI_NOALLOC_SCRATCH_BYTES;
    }
    return ti_attention(&local, c, stream);
}

int ti_store_kv(int dtype, const ti_kv_cache *c, const void *k, const void *v,
                const int32_t *slots, int n, void *stream) {
    if (bad_dtype(dtype) || bad_cache(c) || n < 0) return TI_ERR_INVALID_ARG;
    if (c->head_dim > 512) return TI_ERR_UNSUPPORTED;
    if (n == 0) return TI_OK;
    if (!k || !v || !slots) return TI_ERR_INVALID_ARG;
    return ti_launch_store_kv(dtype, c, k, v, slots, n, (hipStream_t)stream);
}

int ti_rope(int dtype, void *y, const void *x, const void *cos_table, const void *sin_table,
            int table_len, const int32_t *positions, int n, int heads, int head_dim,
            void *stream) {
    if (bad_dtype(dtype) || n < 0 || heads <= 0 || head_dim <= 0 || (head_dim & 1) ||
        table_len <= 0)
        return TI_ERR_INVALID_ARG;
    if (n == 0) return TI_OK;
    if (!y || !x || !cos_table || !sin_table || !positions) return TI_ERR_INVALID_ARG;
    return ti_launch_rope(dtype, y, x, cos_table, sin_table, table_len, positions, n, heads,
                          head_dim, (hipStream_t)stream);
}

int ti_rmsnorm(int dtype, void *y, const void *x, const void *w, int rows, int hidden, float eps,
               void *stream) {
    if (bad_dtype(dtype) || rows < 0 || hidden <= 0 || !(eps >= 0.0f)) return TI_ERR_INVALID_ARG;
    if (rows == 0) return TI_OK;
    if (!y || !x || !w) return TI_ERR_INVALID_ARG;
    return ti_launch_rmsnorm(dtype, y, x, w, rows, hidden, eps, (hipStream_t)stream);
}

int ti_attention_inputs(int dtype, void *q_out, const ti_kv_cache *c, const void *qkv,
                        const void *q_norm, const void *k_norm, const void *cos_sin,
                        int table_len, const int32_t *positions, const int32_t *slots, int n,
                        int q_heads, float eps, void *stream) {
    if (bad_dtype(dtype) || bad_cache(c) || n < 0 || q_heads <= 0 || table_len <= 0)
        return TI_ERR_INVALID_ARG;
    if (c->head_dim > 128) return TI_ERR_UNSUPPORTED;
    if ((q_norm == nullptr) != (k_norm == nullptr)) return TI_ERR_INVALID_ARG;
    if (n == 0) return TI_OK;
    if (!q_out || !qkv || !cos_sin || !positions || !slots) return TI_ERR_INVALID_ARG;
    return ti_launch_attention_inputs(dtype, q_out, c, qkv, q_norm, k_norm, cos_sin, table_len,
                                      positions, slots, n, q_heads, eps, (hipStream_t)stream);
}

}  // extern "C"
