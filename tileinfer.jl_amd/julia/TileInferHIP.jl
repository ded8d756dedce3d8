# TileInferHIP: TileInfer.jl's attention ops on MI355X through libtileinfer_hip.so.
#
# A `HipBackend <: TileInfer.Backend` whose methods have the reference's signatures
# (src/ops/interface.jl) and forward to the C ABI in include/tileinfer_hip.h with `ccall`.
# Arrays are AMDGPU.jl `ROCArray`s in the reference's column-major layouts, which are the
# C ABI's row-major layouts reversed, so every argument is passed as a pointer, no copy.
#
# Not exercised in this repository (no Julia toolchain in the build image); the Python
# package tileinfer_hip drives the same entry points in the tests. It needs the reference's
# allocations made array-generic first: the Int8Pages fields and int8_kv_pools
# (src/ops/quant.jl:86-109), the cache pools (src/kv/paged_cache.jl:29), the rotary tables
# (src/model/rope.jl:47) and StepBuffers (src/model/decoder.jl:72-112). The INT8 and
# rotary methods below are typed on those generic types with ROCArray storage.
module TileInferHIP

using AMDGPU: ROCArray, ROCVector, stream
using TileInfer: TileInfer, Backend, Int8Pages, RotaryTable, layer_arrays

const LIB = joinpath(@__DIR__, "..", "tileinfer_hip", "libtileinfer_hip.so")

"MI355X kernels from libtileinfer_hip.so."
struct HipBackend <: Backend end

const TI_F32, TI_BF16 = Int32(0), Int32(1)
const TI_KV_DENSE, TI_KV_INT8 = Int32(0), Int32(1)
const TI_PATH_AUTO = Int32(0)

# ti_kv_cache
struct KVCache
    kind::Int32
    head_dim::Int32
    page_size::Int32
    kv_heads::Int32
    num_pages::Int32
    k_pages::Ptr{Cvoid}
    v_pages::Ptr{Cvoid}
    layer_q::Ptr{Int8}
    layer_scale::Ptr{Float32}
    smooth::Ptr{Float32}
end

# ti_attention_args
struct AttentionArgs
    dtype::Int32
    q_heads::Int32
    num_seqs::Int32
    max_query_len::Int32
    total_tokens::Int32
    block_table_stride::Int32
    q::Ptr{Cvoid}
    out::Ptr{Cvoid}
    positions::Ptr{Int32}
    query_start_loc::Ptr{Int32}
    block_tables::Ptr{Int32}
    scale::Float32
    causal::Int32
    path::Int32
    workspace::Ptr{Cvoid}
    workspace_bytes::Csize_t
end

dtype_code(::Type{Float32}) = TI_F32
dtype_code(::Type{<:Any}) = TI_BF16            # BFloat16

function check(status::Integer)
    status == 0 && return nothing
    msg = unsafe_string(ccall((:ti_status_string, LIB), Cstring, (Cint,), status))
    status in (1, 2, 3) ? throw(ArgumentError(msg)) : error(msg)
end

vptr(x) = Ptr{Cvoid}(UInt(pointer(x)))

function kv_cache(k::ROCArray{T,4}, v::ROCArray{T,4}) where {T}
    D, P, H, pages = size(k)
    KVCache(TI_KV_DENSE, D, P, H, pages, vptr(k), vptr(v), C_NULL, C_NULL, C_NULL)
end

function kv_cache(k::Int8Pages{<:ROCArray}, v::Int8Pages{<:ROCArray})
    q, s, c = layer_arrays(k, v)                   # ArgumentError unless paired halves
    D, P, H, pages = size(k)
    KVCache(TI_KV_INT8, D, P, H, pages, C_NULL, C_NULL, pointer(q), pointer(s), pointer(c))
end

function attention_args(out, q::ROCArray{T,3}, block_table, positions, scale, causal, ws) where {T}
    D, heads, n = size(q)
    AttentionArgs(dtype_code(T), heads, 1, n, n, length(block_table), vptr(q), vptr(out),
                  pointer(positions), C_NULL, pointer(block_table), Float32(scale), causal,
                  TI_PATH_AUTO, ws === nothing ? C_NULL : vptr(ws),
                  ws === nothing ? 0 : sizeof(ws))
end

# A shape-only ti_attention_args for ti_attention_workspace_bytes: the query's dtype and
# shape (one sequence of n tokens). The size query never dereferences a pointer, but the
# argument check wants them non-null, so they are a fixed non-null placeholder.
function workspace_query(q::ROCArray{T,3}) where {T}
    D, heads, n = size(q)
    nz = Ptr{Cvoid}(1)
    AttentionArgs(dtype_code(T), heads, 1, n, n, 1, nz, nz, Ptr{Int32}(1), C_NULL, Ptr{Int32}(1),
                  1.0f0, Int32(1), TI_PATH_AUTO, C_NULL, 0)
end

# The shape-only ti_kv_cache of a pool (dense ROCArray or either Int8Pages half).
function workspace_cache(k_pages::Union{ROCArray,Int8Pages{<:ROCArray}})
    D, P, H, pages = size(k_pages)
    nz = Ptr{Cvoid}(1)
    k_pages isa Int8Pages ?
        KVCache(TI_KV_INT8, D, P, H, pages, C_NULL, C_NULL, Ptr{Int8}(1), Ptr{Float32}(1), Ptr{Float32}(1)) :
        KVCache(TI_KV_DENSE, D, P, H, pages, nz, nz, C_NULL, C_NULL, C_NULL)
end

# attention_workspace(::TileBackend, q, k_pages): src/ops/tile/attention.jl:351-352
function TileInfer.attention_workspace(::HipBackend, q::ROCArray{T,3}, k_pages) where {T}
    c = Ref(workspace_cache(k_pages))
    a = Ref(workspace_query(q))
    n = Ref{Csize_t}(0)
    check(ccall((:ti_attention_workspace_bytes, LIB), Cint,
                (Ptr{AttentionArgs}, Ptr{KVCache}, Ptr{Csize_t}), a, c, n))
    return n[] == 0 ? nothing : ROCArray{UInt8}(undef, n[])
end

# attention!(::TileBackend, ...): src/ops/tile/attention.jl:359-366
function TileInfer.attention!(::HipBackend, out::ROCArray{T,3}, workspace, q::ROCArray{T,3},
                              k_pages, v_pages, block_table::ROCVector{Int32},
                              positions::ROCVector{Int32}, scale::Real; causal::Bool = true) where {T}
    a = Ref(attention_args(out, q, block_table, positions, scale, Int32(causal), workspace))
    c = Ref(kv_cache(k_pages, v_pages))
    check(ccall((:ti_attention, LIB), Cint, (Ptr{AttentionArgs}, Ptr{KVCache}, Ptr{Cvoid}),
                a, c, stream().stream))
    return out
end

TileInfer.attention(be::HipBackend, q::ROCArray{T,3}, k_pages, v_pages, block_table, positions,
                    scale::Real; causal::Bool = true) where {T} =
    TileInfer.attention!(be, similar(q), TileInfer.attention_workspace(be, q, k_pages), q, k_pages,
                         v_pages, block_table, positions, scale; causal)

# store_kv!(::TileBackend, ...): src/ops/tile/elementwise.jl:133-140, :180-188
function TileInfer.store_kv!(::HipBackend, k_pages, v_pages, k::ROCArray{T,3}, v::ROCArray{T,3},
                             slots::ROCVector{Int32}) where {T}
    c = Ref(kv_cache(k_pages, v_pages))
    check(ccall((:ti_store_kv, LIB), Cint,
                (Cint, Ptr{KVCache}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Int32}, Cint, Ptr{Cvoid}),
                dtype_code(T), c, vptr(k), vptr(v), pointer(slots), length(slots), stream().stream))
    return nothing
end

# rmsnorm!(::TileBackend, y, x, w, eps): src/ops/tile/norm.jl:31-38
function TileInfer.rmsnorm!(::HipBackend, y::ROCArray{T}, x::ROCArray{T}, w::ROCVector{T}, eps::Real) where {T}
    H = size(x, 1)
    check(ccall((:ti_rmsnorm, LIB), Cint, (Cint, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Cint, Cint, Cfloat, Ptr{Cvoid}),
                dtype_code(T), vptr(y), vptr(x), vptr(w), length(x) ÷ H, H, Float32(eps), stream().stream))
    return y
end

# rope!(::TileBackend, ...): src/ops/tile/elementwise.jl:29-36
function TileInfer.rope!(::HipBackend, y::ROCArray{T,3}, x::ROCArray{T,3}, cos::ROCArray{T,2},
                         sin::ROCArray{T,2}, positions::ROCVector{Int32}) where {T}
    D, heads, n = size(x)
    check(ccall((:ti_rope, LIB), Cint,
                (Cint, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Cint, Ptr{Int32}, Cint, Cint, Cint, Ptr{Cvoid}),
                dtype_code(T), vptr(y), vptr(x), vptr(cos), vptr(sin), size(cos, 2), pointer(positions),
                n, heads, D, stream().stream))
    return y
end

# attention_inputs!(::TileBackend, ...): src/ops/tile/fused.jl:94-130
function TileInfer.attention_inputs!(::HipBackend, q::ROCArray{T,3}, k_pages, v_pages, qkv,
                                     q_norm, k_norm, table::RotaryTable{T,<:ROCArray}, positions, slots,
                                     eps::Real) where {T}
    D, nq, n = size(q)
    c = Ref(kv_cache(k_pages, v_pages))
    check(ccall((:ti_attention_inputs, LIB), Cint,
                (Cint, Ptr{Cvoid}, Ptr{KVCache}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Ptr{Cvoid}, Cint,
                 Ptr{Int32}, Ptr{Int32}, Cint, Cint, Cfloat, Ptr{Cvoid}),
                dtype_code(T), vptr(q), c, vptr(qkv), q_norm === nothing ? C_NULL : vptr(q_norm),
                k_norm === nothing ? C_NULL : vptr(k_norm), vptr(table.cos_sin), size(table.cos_sin, 2) ÷ 2,
                pointer(positions), pointer(slots), n, nq, Float32(eps), stream().stream))
    return q
end

TileInfer.supports_graphs(::HipBackend) = true
TileInfer.has_kernel(::HipBackend, op) = op in (TileInfer.attention!, TileInfer.attention,
                                               TileInfer.store_kv!, TileInfer.rmsnorm!, TileInfer.rope!,
                                               TileInfer.attention_inputs!)

export HipBackend

end # module
