"""The operation contract of the hot path, as plain data: dash-contract's option types and
semantics (``crates/dash-contract/src/attention.rs``, ``gated_delta/chunk.rs``,
``gated_delta/recurrent.rs``, ``lib.rs``), with the same names, fields and defaults.

Refusals follow ``crates/dash-contract/src/lib.rs:76-91``: a call outside the contract is refused
before anything is computed, the message naming the operation and what is wrong
(``"attention: key and value must have one shape"``). Operations that return results raise
:class:`Unsupported` (a :class:`ValueError`) with that message, as a ``Result``-returning
implementation returns it as its error (dash-mlx's convention, ``crates/dash-mlx/tests/common/
mod.rs:128-142``).
"""
from __future__ import annotations

import dataclasses
import enum
import math
from typing import Optional

#: ``usize::MAX`` of the contract: an unbounded window side.
UNBOUNDED = (1 << 64) - 1


class Unsupported(ValueError):
    """A call refused before compute; the message starts with ``"<operation>: "``."""


class DType(enum.Enum):
    """crates/dash-contract/src/lib.rs:106-115."""

    F32 = "f32"
    BF16 = "bf16"
    F16 = "f16"


@dataclasses.dataclass(frozen=True)
class Window:
    """A sliding window around each query's position (attention.rs:72-81): no key more than
    ``left`` positions before it or ``right`` after it; ``UNBOUNDED`` leaves a side open."""

    left: int
    right: int


@dataclasses.dataclass(frozen=True)
class AttentionOptions:
    """attention.rs:83-158: default is every key, no causality, no window, ``scale = 1/sqrt(D)``,
    a deterministic backward."""

    causal: bool = False
    scale: Optional[float] = None
    window: Optional[Window] = None
    deterministic: bool = True

    @staticmethod
    def causal_default() -> "AttentionOptions":
        return AttentionOptions(causal=True)

    def with_causal(self, causal: bool) -> "AttentionOptions":
        return dataclasses.replace(self, causal=causal)

    def with_scale(self, scale: float) -> "AttentionOptions":
        return dataclasses.replace(self, scale=float(scale))

    def with_window(self, left: int, right: int) -> "AttentionOptions":
        return dataclasses.replace(self, window=Window(int(left), int(right)))

    def with_deterministic(self, deterministic: bool) -> "AttentionOptions":
        return dataclasses.replace(self, deterministic=deterministic)

    def scale_for(self, d: int) -> float:
        """``scale.unwrap_or((1.0 / (d as f64).sqrt()) as f32)`` (attention.rs:156-158)."""
        if self.scale is not None:
            return float(self.scale)
        return _f32(1.0 / math.sqrt(d))

    def reach(self):
        """``(left, right)``, causality as ``right = 0`` (crates/dash-ops/src/attention.rs:
        235-241)."""
        left, right = (UNBOUNDED, UNBOUNDED) if self.window is None else (
            self.window.left, self.window.right)
        return left, 0 if self.causal else right


class AttentionMask:
    """attention.rs:160-183: ``none()``, ``key_padding(mask [B, Tk], True = left out)``, or
    ``packed(cu_seqlens_q, cu_seqlens_k)`` ([S + 1] each, B = 1)."""

    NONE, KEY_PADDING, PACKED = "none", "key_padding", "packed"

    def __init__(self, kind, padding=None, cu_seqlens_q=None, cu_seqlens_k=None):
        self.kind = kind
        self.padding = padding
        self.cu_seqlens_q = cu_seqlens_q
        self.cu_seqlens_k = cu_seqlens_k

    @classmethod
    def none(cls):
        return cls(cls.NONE)

    @classmethod
    def key_padding(cls, padding):
        return cls(cls.KEY_PADDING, padding=padding)

    @classmethod
    def packed(cls, cu_seqlens_q, cu_seqlens_k):
        return cls(cls.PACKED, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k)


@dataclasses.dataclass(frozen=True)
class ChunkGatedDeltaOptions:
    """gated_delta/chunk.rs:36-68: no normalisation, ``scale = 1/sqrt(Dk)``, no final state."""

    qk_l2norm: bool = False
    scale: Optional[float] = None
    output_final_state: bool = False

    def with_qk_l2norm(self, v: bool):
        return dataclasses.replace(self, qk_l2norm=v)

    def with_scale(self, s: float):
        return dataclasses.replace(self, scale=float(s))

    def with_final_state(self, v: bool):
        return dataclasses.replace(self, output_final_state=v)


@dataclasses.dataclass(frozen=True)
class GatedDeltaStepOptions:
    """gated_delta/recurrent.rs:39-71."""

    qk_l2norm: bool = False
    scale: Optional[float] = None

    def with_qk_l2norm(self, v: bool):
        return dataclasses.replace(self, qk_l2norm=v)

    def with_scale(self, s: float):
        return dataclasses.replace(self, scale=float(s))

    @staticmethod
    def from_chunk(options: ChunkGatedDeltaOptions) -> "GatedDeltaStepOptions":
        return GatedDeltaStepOptions(options.qk_l2norm, options.scale)


class Activation(enum.Enum):
    """crates/dash-contract/src/conv1d.rs:81-90: the conv1d's activation after the bias."""

    NONE = 0
    SILU = 1


@dataclasses.dataclass(frozen=True)
class CausalConv1dOptions:
    """crates/dash-contract/src/conv1d.rs:92-126: no activation, no final state; the final
    states' length ``None`` for the initial states' (``K - 1`` without them)."""

    activation: Activation = Activation.NONE
    output_final_state: bool = False
    final_state_len: Optional[int] = None

    def with_activation(self, activation: Activation):
        return dataclasses.replace(self, activation=activation)

    def with_final_state(self, v: bool):
        return dataclasses.replace(self, output_final_state=v)

    def with_final_state_len(self, n: int):
        return dataclasses.replace(self, output_final_state=True, final_state_len=int(n))


@dataclasses.dataclass(frozen=True)
class CausalConv1dStepOptions:
    """crates/dash-contract/src/conv1d.rs:128-140."""

    activation: Activation = Activation.NONE

    @staticmethod
    def from_sequence(options: CausalConv1dOptions) -> "CausalConv1dStepOptions":
        return CausalConv1dStepOptions(options.activation)


@dataclasses.dataclass(frozen=True)
class LogprobOptions:
    """How the vocabulary and the rows are chunked (crates/dash-contract/src/logprob.rs:33-56):
    ``vocab_chunk`` tokens per chunk (0: the implementation's own choice, 8192 tokens here;
    dash-ops takes 4096 below 2304 rows, crates/dash-ops/src/logprob.rs:90-101), ``row_chunk``
    the most rows per block."""

    vocab_chunk: int = 0
    row_chunk: int = 3072


class Reduction(enum.Enum):
    """How linear_cross_entropy reduces the rows' losses, as torch's ``reduction``
    (crates/dash-contract/src/loss.rs:52-63)."""

    MEAN = "mean"
    SUM = "sum"
    NONE = "none"


@dataclasses.dataclass(frozen=True)
class CrossEntropyOptions:
    """crates/dash-contract/src/loss.rs:65-95: torch's ``F.cross_entropy`` defaults (the mean,
    ignore index -100, no label smoothing), no z-loss, no masked id, no entropy."""

    reduction: Reduction = Reduction.MEAN
    ignore_index: int = -100
    label_smoothing: float = 0.0
    z_loss: float = 0.0
    masked: tuple = ()
    entropy: bool = False
    chunks: LogprobOptions = LogprobOptions()


def query_scale(scale: Optional[float], dk: int) -> float:
    """The gated delta rule's query scale: ``1/sqrt(Dk)`` unless given
    (crates/dash-ops/src/gated_delta.rs:17)."""
    return float(scale) if scale is not None else _f32(1.0 / math.sqrt(dk))


#: transformers' and fla's l2norm epsilon (chunk/reference.rs:29).
L2NORM_EPS = 1e-6
#: Tokens per chunk (chunk/reference.rs:26).
CHUNK = 64


def _f32(x: float) -> float:
    import struct

    return struct.unpack("f", struct.pack("f", x))[0]
