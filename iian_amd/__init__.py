"""iian_amd: MI355X-native paged-attention hot path of the iian inference engine.

The compute lives in libiian_pa.so (hand-written gfx950 HIP kernels behind the
C ABI of include/iian_pa.h); this package is its host-side mirror of iian's
operator interface.  Importing it does not require a GPU; calling into the
kernels does, and fails loudly when the library has not been built.
"""
from .paged_attn import (  # noqa: F401
    GGML_TYPE_F16,
    GGML_TYPE_F32,
    GGML_TYPE_Q8_0,
    KVPool,
    PagedAttnParams,
    PagedAttnRuntime,
    PagedBatch,
    RequestBlocks,
    RopeParams,
    bind_build_batch,
    bind_paged_attn,
    bind_rope_set_rows_kv,
    bind_set_rows_kv,
    bind_write_paged_attn,
    build_batch,
    build_paged_attn,
    dequant_q8_0,
    new_workspace,
    paged_attn_supported,
    rope_set_rows_kv,
    row_bytes,
    set_rows,
    set_rows_kv,
    swa_free_blocks,
    workspace_size,
    write_paged_attn,
)
from ._lib import PagedAttnError  # noqa: F401
