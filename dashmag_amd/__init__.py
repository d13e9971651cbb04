"""dashmag_amd: dash-ops' attention and gated-delta-rule hot path, native to MI355X (gfx950).

The operations run as hand-written HIP kernels in ``libdashmi.so`` behind the C ABI of
``include/dashmi.h``; this package is the host-side mirror of dash-ops' operation interface
(``ops``), its contract types (``contract``) and autograd wrappers (``autograd``).
"""
from .contract import (AttentionMask, AttentionOptions, ChunkGatedDeltaOptions, DType,
                       GatedDeltaStepOptions, UNBOUNDED, Unsupported, Window)
from .ops import (attention, attention_backward, attention_decode, attention_with_lse,
                  chunk_gated_delta_rule, chunk_gated_delta_rule_backward, gated_delta_step)

__all__ = [
    "AttentionMask", "AttentionOptions", "ChunkGatedDeltaOptions", "DType",
    "GatedDeltaStepOptions", "UNBOUNDED", "Unsupported", "Window",
    "attention", "attention_backward", "attention_decode", "attention_with_lse",
    "chunk_gated_delta_rule", "chunk_gated_delta_rule_backward", "gated_delta_step",
]
