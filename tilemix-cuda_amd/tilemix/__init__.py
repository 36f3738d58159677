"""Python mirror of the TileMix API, bound to libtilemix_hip.so through ctypes.

Same entry-point names, argument meaning and error codes as the reference's C++
header (include/attention_fused.h:47-72): ``quantize_tilemix_qk`` and
``launch_fused_fp16_attention`` return the hipError_t code of the C ABI
(0 = success, 1 = invalid value, 9 = invalid configuration, 801 = not
supported). Tensors are torch device tensors (or raw device addresses as
ints, ``None`` for NULL); PyTorch only provides device memory and streams.

There is no CPU fallback: every call goes to the HIP library, and importing
the binding fails loudly if the library has not been built.
"""
from __future__ import annotations

from .api import (  # noqa: F401
    BatchedArgs,
    TileMixQuantized,
    TileMixRouting,
    attention_batched,
    check,
    launch_fused_fp16_attention,
    library,
    library_path,
    quantize_tilemix_qk,
    quantize_tilemix_qk_batched,
    quantize_tilemix_qk_strided,
    DTYPE_F32,
    DTYPE_F16,
    DTYPE_BF16,
    importance_noalloc_max_bytes,
    importance_workspace_bytes,
    routes_from_tiles,
    tiles_bernoulli,
    tiles_causal_band,
    tiles_importance,
    tiles_importance_noalloc,
    tiles_three_way,
    routing_word_count,
    routing_words_per_row,
    shared_bytes,
    version,
    ERROR_INVALID_VALUE,
    ERROR_INVALID_CONFIGURATION,
    ERROR_NOT_SUPPORTED,
    SUCCESS,
    TileMixError,
)
from . import routing  # noqa: F401

# Reference API constants (include/matmul_config.h:3-7, include/attention_fused.h:11-14).
kBlockM = 16
kBlockN = 32
kTileK = 16
kThreads = 64
kWarpSize = 32
kFusedMaxHeadDim = 128
kFusedRowThreads = kThreads // kBlockM
kTileMixQQuantRows = 128
kTileMixKQuantRows = 64
