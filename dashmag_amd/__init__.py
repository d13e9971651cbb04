"""dashmag_amd: dash-ops' attention, gated-delta-rule, causal-conv1d and chosen-token
log-probability hot path, native to MI355X (gfx950).

The operations run as hand-written HIP kernels in ``libdashmi.so`` behind the C ABI of
``include/dashmi.h``; this package is the host-side mirror of dash-ops' operation interface
(``ops``) and its contract types (``contract``).
"""
from .contract import (Activation, AttentionMask, AttentionOptions, CausalConv1dOptions,
                       CrossEntropyOptions, Reduction,
                       CausalConv1dStepOptions, ChunkGatedDeltaOptions, DType,
                       GatedDeltaStepOptions, LogprobOptions, UNBOUNDED, Unsupported, Window)
from .ops import (attention, attention_backward, attention_decode, attention_decode_packed,
                  attention_decode_paged, attention_with_lse,
                  causal_conv1d, causal_conv1d_backward, causal_conv1d_update, chosen_logprob,
                  chosen_logprob_with_grad, linear_cross_entropy,
                  linear_cross_entropy_backward,
                  chunk_gated_delta_rule, chunk_gated_delta_rule_backward, gated_delta_step,
                  gated_delta_step_backward)

__all__ = [
    "Activation", "AttentionMask", "AttentionOptions", "CausalConv1dOptions",
    "CausalConv1dStepOptions", "ChunkGatedDeltaOptions", "DType",
    "GatedDeltaStepOptions", "LogprobOptions", "UNBOUNDED", "Unsupported", "Window",
    "attention", "attention_backward", "attention_decode", "attention_decode_packed",
    "attention_decode_paged", "attention_with_lse",
    "causal_conv1d", "causal_conv1d_backward", "causal_conv1d_update", "chosen_logprob",
    "chosen_logprob_with_grad", "linear_cross_entropy", "linear_cross_entropy_backward",
    "CrossEntropyOptions", "Reduction",
    "chunk_gated_delta_rule", "chunk_gated_delta_rule_backward", "gated_delta_step",
    "gated_delta_step_backward",
]
