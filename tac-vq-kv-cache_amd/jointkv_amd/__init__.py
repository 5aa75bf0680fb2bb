"""jointkv_amd — MI355X (gfx950) hard residual-quantization hot path.

Drop-in operator API of wrb1371/tac-vq-kv-cache's ``jointkv`` hot path
(hard residual VQ / grouped CQ encode with straight-through gradients, the
codec modules, codebook-gradient clipping, the rate ledger) plus fused decode
attention over packed code caches.  All device work runs in the hand-written
HIP kernels of ``libjkv.so``; there is no CPU fallback.
"""

from . import _lib, artifacts
from .additive_refinement import multi_exit_additive_block_refinement, multi_exit_additive_coordinate_refinement
from .attention import (
    DecodedWindowCache,
    PackedCodeCache,
    decode_attention,
    decode_attention_window,
    deploy_tables,
    prefill_attention,
    prefill_attention_from_codes,
)
from .budget import (
    CacheGeometry,
    StorageLedger,
    dynamic_bpa,
    paired_prefix_rates,
    prefix_index_bits,
    residual_vq_ledger,
    validate_stage_bits,
)
from .calibration import clip_codebook_gradients, sgd_step
from .closed_loop_attention import AttentionWeights, closed_loop_attention, relative_trajectory_attention_mse
from .closed_loop_vq import (
    QuantizedKV,
    frozen_assignment_reconstruction,
    hard_grouped_residual_vq,
    hard_residual_vq_exits,
)
from .cq_tac import ClosedLoopGroupedCQ, hard_grouped_cq
from .gain_shape import fit_residual_stages
from .packed_nested import (
    PackedLayoutLedger,
    PackedNestedKVCache,
    PackedProgressiveStream,
    estimate_block_shared_paired_progressive_layout,
    estimate_layered_paired_progressive_layout,
    estimate_paired_progressive_layout,
    pack_fixed_width,
    pack_paired_progressive_indices,
    unpack_action_depths,
    unpack_fixed_width,
    unpack_paired_progressive_indices,
    validate_packed_nested_cache,
)
from .uniform_depth_tac import ClosedLoopUniformResidualVQ
from .v_only import ClosedLoopRunContext, DecoderStack, causal_loss, run_loss, v_only_step

__all__ = [
    "multi_exit_additive_block_refinement",
    "multi_exit_additive_coordinate_refinement",
    "fit_residual_stages",
    "AttentionWeights",
    "artifacts",
    "causal_loss",
    "CacheGeometry",
    "ClosedLoopGroupedCQ",
    "ClosedLoopRunContext",
    "ClosedLoopUniformResidualVQ",
    "DecodedWindowCache",
    "DecoderStack",
    "PackedCodeCache",
    "PackedLayoutLedger",
    "PackedNestedKVCache",
    "PackedProgressiveStream",
    "QuantizedKV",
    "StorageLedger",
    "clip_codebook_gradients",
    "closed_loop_attention",
    "decode_attention",
    "decode_attention_window",
    "deploy_tables",
    "dynamic_bpa",
    "estimate_block_shared_paired_progressive_layout",
    "estimate_layered_paired_progressive_layout",
    "estimate_paired_progressive_layout",
    "frozen_assignment_reconstruction",
    "hard_grouped_cq",
    "hard_grouped_residual_vq",
    "hard_residual_vq_exits",
    "pack_fixed_width",
    "pack_paired_progressive_indices",
    "prefill_attention",
    "prefill_attention_from_codes",
    "paired_prefix_rates",
    "prefix_index_bits",
    "relative_trajectory_attention_mse",
    "residual_vq_ledger",
    "run_loss",
    "sgd_step",
    "unpack_action_depths",
    "unpack_fixed_width",
    "unpack_paired_progressive_indices",
    "validate_packed_nested_cache",
    "validate_stage_bits",
    "v_only_step",
]


def library_version() -> int:
    return int(_lib.load().jkv_version())
