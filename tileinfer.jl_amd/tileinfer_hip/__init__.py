"""tileinfer_hip: TileInfer.jl's paged flash-attention path on MI355X (gfx950).

Host-side mirror of the reference's op interface (src/ops/interface.jl) and KV layout
(src/kv/), driving the HIP kernels of libtileinfer_hip.so through its C ABI.
"""
from ._lib import (ArgumentError, TileInferError, WorkspaceError, TI_PATH_AUTO, TI_PATH_DECODE,
                   TI_PATH_PREFILL, TI_PATH_PREFILL_STAGED, TI_PATH_PREFILL_DIRECT,
                   TI_PATH_PREFILL_PINGPONG, TI_PATH_PREFILL_PAIRED, TI_PATH_PREFILL_PAIRED16, EXPORTS, LIB_PATH, load as load_library)
from .backend import (HipBackend, attention, attention_, attention_inputs_, attention_workspace,
                      has_kernel, kv_cache_struct, paged_attention_, rmsnorm, rmsnorm_, rope, rope_, store_kv_,
                      supports_graphs, workspace_bytes)
from .kv import (DEFAULT_PAGE_SIZE, BlockManager, Int8Pages, OutOfPagesError, PagedKVCache,
                 Sequence, bytes_per_token, int8_kv_pools, key_smoothing, layer_arrays, release,
                 reserve, slots, truncate)
from .rope import Llama3RopeScaling, RotaryTable, inverse_frequencies, llama3_scaled

__version__ = "0.1.0"
