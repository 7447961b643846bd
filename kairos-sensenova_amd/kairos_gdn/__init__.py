"""kairos_gdn: MI355X-native chunked GatedDeltaNet forward for Kairos.

Drop-in for ``chunk_gated_delta_rule`` of the fla library vendored by Kairos
(kairos/third_party/fla/ops/gated_delta_rule/chunk.py:217).  The compute runs
in hand-written gfx950 HIP kernels behind the C ABI of libkairos_gdn.so
(include/kairos_gdn.h); this package is the host side.
"""
from ._lib import KairosGdnError, LIB_PATH
from .chunk import (
    CHUNK,
    ChunkGatedDeltaRuleFunction,
    chunk_gated_delta_rule,
    chunk_fwd_o,
    chunk_gated_delta_rule_bwd_native,
    chunk_gated_delta_rule_conv,
    chunk_gated_delta_rule_fwd,
    chunk_gated_delta_rule_fwd_h,
    chunk_gated_delta_rule_gated_norm,
    chunk_local_cumsum,
    fwd_h,
    fwd_o,
    l2norm_fwd,
    num_chunks_bound,
    prepare_wy,
    recompute_w_u_fwd,
)
from .norm import FusedRMSNormGated, rms_norm_gated, rms_norm_gated_fwd
from .recurrent import FusedRecurrentFunction, fused_recurrent_gated_delta_rule, fused_recurrent_gated_delta_rule_fwd
from .conv import ShortConvolution, causal_conv1d, gdn_gates
from . import swap

__all__ = [
    "CHUNK", "ChunkGatedDeltaRuleFunction", "KairosGdnError", "LIB_PATH", "chunk_gated_delta_rule",
    "chunk_fwd_o", "chunk_gated_delta_rule_bwd_native", "chunk_gated_delta_rule_conv", "chunk_gated_delta_rule_fwd_h", "chunk_gated_delta_rule_fwd", "chunk_gated_delta_rule_gated_norm", "chunk_local_cumsum", "fwd_h", "fwd_o", "l2norm_fwd", "num_chunks_bound",
    "prepare_wy", "recompute_w_u_fwd", "swap", "FusedRMSNormGated", "rms_norm_gated", "rms_norm_gated_fwd",
    "FusedRecurrentFunction", "fused_recurrent_gated_delta_rule", "fused_recurrent_gated_delta_rule_fwd",
    "ShortConvolution", "causal_conv1d", "gdn_gates",
]
