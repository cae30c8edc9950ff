"""MI355X-native routed sparse path of the foveal sparse indexer.

Mirrors the public names of foveal_indexer/__init__.py:3-95 for the routed
sparse path (indexer routing, block-sparse Pattention MLP, foveal decode
attention, block-sparse linear / 2-D tiled matmul).  Compute runs in the HIP
library libfsi_amd.so (C ABI: include/fsi.h); there is no CPU path.
"""
from . import _lib
from .pattention import (
    HAS_HIP,
    HAS_TRITON,
    TritonSwiGLUPattentionMLP,
    convert_llm_mlp_to_pattention,
    PackedPattentionWeights,
    dense_block_targets,
    fused_swiglu,
    is_triton_available,
    pack_pattention_weights,
    pattention_decode_packed,
    pattention_forward,
    triton_fused_swiglu,
    triton_pattention,
    unpack_pattention_weights,
)
from .core import (
    FovealIndexer,
    Route,
    block_scores,
    index_rms_norm,
    masked_softmax,
    score_and_route,
    select_blocks,
)
from .attention import (
    FovealKVCache,
    FovealSparseAttention,
    decode_attention,
    decode_route,
    decode_step_attention,
    sparse_attention,
    sram_indexer_attention,
    triton_foveal_sparse_attention,
    triton_fused_sram_indexer_attention,
)
from .block_matmul import (
    BlockSparseLinear,
    BlockwiseMatMul2D,
    block_sparse_linear,
    blockwise_matmul,
    tile_route,
    triton_block_sparse_linear,
)
from .foveal_pattention import (
    FovealPattentionMLP,
    compute_teacher_dense_block_targets,
    load_foveal_pattention_mlps,
    mlp_pooled_route,
    release_unpacked_weights,
    sparsify_model_with_foveal_pattention,
)

__all__ = [
    "Route",
    "masked_softmax",
    "select_blocks",
    "score_and_route",
    "block_scores",
    "index_rms_norm",
    "FovealIndexer",
    "decode_route",
    "BlockSparseLinear",
    "BlockwiseMatMul2D",
    "block_sparse_linear",
    "blockwise_matmul",
    "tile_route",
    "triton_block_sparse_linear",
    "decode_attention",
    "decode_step_attention",
    "sparse_attention",
    "triton_foveal_sparse_attention",
    "triton_fused_sram_indexer_attention",
    "sram_indexer_attention",
    "FovealKVCache",
    "FovealSparseAttention",
    "FovealPattentionMLP",
    "sparsify_model_with_foveal_pattention",
    "mlp_pooled_route",
    "triton_pattention",
    "triton_fused_swiglu",
    "fused_swiglu",
    "pattention_forward",
    "pattention_decode_packed",
    "pack_pattention_weights",
    "unpack_pattention_weights",
    "release_unpacked_weights",
    "PackedPattentionWeights",
    "dense_block_targets",
    "compute_teacher_dense_block_targets",
    "load_foveal_pattention_mlps",
    "TritonSwiGLUPattentionMLP",
    "convert_llm_mlp_to_pattention",
    "HAS_HIP",
    "HAS_TRITON",
    "is_triton_available",
]
