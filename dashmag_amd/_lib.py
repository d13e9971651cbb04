"""Loads ``libdashmi.so`` (the HIP library behind ``include/dashmi.h``) and declares its C ABI
for ctypes. There is no fallback: if the library is missing or the device is not a gfx950,
every operation raises."""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdashmi.so")

DM_OK, DM_ERR_REFUSED, DM_ERR_HIP = 0, 1, 2
DM_F32, DM_BF16, DM_F16 = 0, 1, 2
DM_MASK_NONE, DM_MASK_KEY_PADDING, DM_MASK_PACKED = 0, 1, 2
DM_UNBOUNDED = (1 << 64) - 1

PROBES = ["attn_fwd_mfma", "attn_fwd_generic", "attn_bwd_mfma", "attn_bwd_generic",
          "decode_split", "decode_merge", "gdr_chunk_fwd", "gdr_chunk_bwd", "gdr_step",
          "conv1d_fwd", "conv1d_bwd", "conv1d_update", "logprob", "lce_fwd", "lce_bwd",
          "gdr_chunk_fwd_mfma", "gdr_chunk_bwd_mfma", "gdr_step_bwd"]
DM_ACT_NONE, DM_ACT_SILU = 0, 1


class AttentionOptionsC(ctypes.Structure):
    _fields_ = [("causal", ctypes.c_int32), ("has_scale", ctypes.c_int32),
                ("scale", ctypes.c_float), ("has_window", ctypes.c_int32),
                ("window_left", ctypes.c_uint64), ("window_right", ctypes.c_uint64),
                ("deterministic", ctypes.c_int32)]


class Strides(ctypes.Structure):
    _fields_ = [("b", ctypes.c_int64), ("t", ctypes.c_int64), ("h", ctypes.c_int64)]


class AttentionDesc(ctypes.Structure):
    _fields_ = [("b", ctypes.c_int64), ("tq", ctypes.c_int64), ("tk", ctypes.c_int64),
                ("hq", ctypes.c_int64), ("hkv", ctypes.c_int64), ("d", ctypes.c_int64),
                ("dtype", ctypes.c_int32), ("mask_kind", ctypes.c_int32),
                ("key_padding", ctypes.c_void_p), ("cu_seqlens_q", ctypes.c_void_p),
                ("cu_seqlens_k", ctypes.c_void_p), ("nseq", ctypes.c_int64),
                ("options", AttentionOptionsC), ("strided", ctypes.c_int32),
                ("sq", Strides), ("sk", Strides), ("sv", Strides), ("so", Strides),
                ("sdo", Strides)]


class GdrDesc(ctypes.Structure):
    _fields_ = [("b", ctypes.c_int64), ("t", ctypes.c_int64), ("h", ctypes.c_int64),
                ("dk", ctypes.c_int64), ("dv", ctypes.c_int64), ("dtype", ctypes.c_int32),
                ("g_dtype", ctypes.c_int32), ("beta_dtype", ctypes.c_int32),
                ("cu_seqlens", ctypes.c_void_p), ("nseq", ctypes.c_int64),
                ("qk_l2norm", ctypes.c_int32), ("has_scale", ctypes.c_int32),
                ("scale", ctypes.c_float), ("strided", ctypes.c_int32), ("sq", Strides),
                ("sk", Strides), ("sv", Strides), ("sg", Strides), ("sbeta", Strides),
                ("sdo", Strides)]


class Conv1dDesc(ctypes.Structure):
    _fields_ = [("b", ctypes.c_int64), ("t", ctypes.c_int64), ("c", ctypes.c_int64),
                ("k", ctypes.c_int64), ("dtype", ctypes.c_int32),
                ("cu_seqlens", ctypes.c_void_p), ("nseq", ctypes.c_int64),
                ("has_bias", ctypes.c_int32), ("activation", ctypes.c_int32),
                ("has_initial", ctypes.c_int32), ("w", ctypes.c_int64),
                ("has_final", ctypes.c_int32), ("w_out", ctypes.c_int64)]


class LogprobDesc(ctypes.Structure):
    _fields_ = [("n", ctypes.c_int64), ("v", ctypes.c_int64), ("d", ctypes.c_int64),
                ("hidden_dtype", ctypes.c_int32), ("weight_dtype", ctypes.c_int32),
                ("vocab_chunk", ctypes.c_int64), ("row_chunk", ctypes.c_int64)]


class LceDesc(ctypes.Structure):
    _fields_ = [("lp", LogprobDesc), ("ignore_index", ctypes.c_int64),
                ("label_smoothing", ctypes.c_float), ("z_loss", ctypes.c_float),
                ("entropy", ctypes.c_int32)]


#: Every symbol include/dashmi.h declares, with (restype, argtypes).
_VP, _SZ, _I64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int64
_AD, _GD = ctypes.POINTER(AttentionDesc), ctypes.POINTER(GdrDesc)
_CD = ctypes.POINTER(Conv1dDesc)
_LD = ctypes.POINTER(LogprobDesc)
_XD = ctypes.POINTER(LceDesc)
SIGNATURES = {
    "dm_last_error": (ctypes.c_char_p, []),
    "dm_describe": (ctypes.c_int, [ctypes.c_char_p, _SZ]),
    "dm_device_alloc": (ctypes.c_int, [_SZ, ctypes.POINTER(ctypes.c_void_p)]),
    "dm_device_free": (ctypes.c_int, [_VP]),
    "dm_copy_to_device": (ctypes.c_int, [_VP, _VP, _SZ, _VP]),
    "dm_copy_to_host": (ctypes.c_int, [_VP, _VP, _SZ, _VP]),
    "dm_stream_synchronize": (ctypes.c_int, [_VP]),
    "dm_probe_count": (ctypes.c_uint64, [ctypes.c_int]),
    "dm_probe_reset": (None, []),
    "dm_kernel_timing": (ctypes.c_int, [ctypes.c_int]),
    "dm_kernel_time": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                      ctypes.POINTER(ctypes.c_uint64)]),
    "dm_attention_row_bounds": (ctypes.c_int, [_AD, _I64, _I64, ctypes.POINTER(_I64),
                                               ctypes.POINTER(_I64)]),
    "dm_attention_fwd_workspace": (_SZ, [_AD]),
    "dm_attention_fwd": (ctypes.c_int, [_AD, _VP, _VP, _VP, _VP, _VP, _VP, _SZ, _VP]),
    "dm_attention_bwd_workspace": (_SZ, [_AD]),
    "dm_attention_bwd": (ctypes.c_int, [_AD, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP,
                                        _SZ, _VP]),
    "dm_attention_decode_workspace": (_SZ, [_AD]),
    "dm_attention_decode": (ctypes.c_int, [_AD, _VP, _VP, _VP, _VP, _VP, _VP, _SZ, _VP]),
    "dm_attention_decode_noalloc": (ctypes.c_int, [_AD, _VP, _VP, _VP, _VP, _VP, _VP]),
    "dm_linear_cross_entropy_workspace": (_SZ, [_XD, ctypes.c_int]),
    "dm_linear_cross_entropy_fwd": (ctypes.c_int, [_XD, _VP, _VP, _VP, _VP, _I64, _VP, _VP, _SZ,
                                                   _VP]),
    "dm_linear_cross_entropy_bwd": (ctypes.c_int, [_XD, _VP, _VP, _VP, _VP, _I64, _VP, _VP, _VP,
                                                   _VP, _VP, _SZ, _VP]),
    "dm_chosen_logprob_workspace": (_SZ, [_LD, ctypes.c_int]),
    "dm_chosen_logprob": (ctypes.c_int, [_LD, _VP, _VP, _VP, _VP, _I64, _VP, _VP, _VP, _VP,
                                         _SZ, _VP]),
    "dm_attention_decode_paged_workspace": (_SZ, [_AD, ctypes.c_int64]),
    "dm_attention_decode_paged": (ctypes.c_int, [_AD, _VP, _VP, _VP, ctypes.c_int64,
                                                 ctypes.c_int64, _VP, ctypes.c_int64, _VP, _VP,
                                                 _VP, _SZ, _VP]),
    "dm_gdr_chunk_fwd_workspace": (_SZ, [_GD]),
    "dm_gdr_chunk_fwd": (ctypes.c_int, [_GD, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _VP, _SZ,
                                        _VP]),
    "dm_gdr_chunk_bwd_workspace": (_SZ, [_GD]),
    "dm_gdr_chunk_bwd": (ctypes.c_int, [_GD] + [_VP] * 15 + [_SZ, _VP]),
    "dm_gdr_step": (ctypes.c_int, [_GD] + [_VP] * 9),
    "dm_gdr_step_bwd_workspace": (_SZ, [_GD]),
    "dm_gdr_step_bwd": (ctypes.c_int, [_GD] + [_VP] * 15 + [_SZ, _VP]),
    "dm_causal_conv1d_fwd": (ctypes.c_int, [_CD] + [_VP] * 7),
    "dm_causal_conv1d_bwd_workspace": (_SZ, [_CD]),
    "dm_causal_conv1d_bwd": (ctypes.c_int, [_CD] + [_VP] * 5 + [ctypes.c_int] + [_VP] * 6
                             + [_SZ, _VP]),
    "dm_causal_conv1d_update": (ctypes.c_int, [_CD] + [_VP] * 7),
}

_lib = None


class LibraryMissing(RuntimeError):
    pass


def lib():
    """The loaded library; raises :class:`LibraryMissing` if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise LibraryMissing(
                f"{LIB_PATH} is not built: run `python -m dashmag_amd.build` (or "
                "__graft_entry__.build()); there is no CPU fallback")
        lb = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(lb, name)
            f.restype = res
            f.argtypes = args
        _lib = lb
    return _lib


def last_error() -> str:
    return lib().dm_last_error().decode()


def probe_counts() -> dict:
    return {name: int(lib().dm_probe_count(i)) for i, name in enumerate(PROBES)}


def probe_reset() -> None:
    lib().dm_probe_reset()


KERNELS = ["attn_fwd", "attn_bwd_dkdv", "attn_bwd_dq", "decode_split", "gdr_prep", "gdr_state",
           "gdr_output", "gdr_step", "gdr_bwd_pre", "gdr_bwd_state", "gdr_bwd_grads",
           "conv1d_fwd", "conv1d_bwd", "conv1d_update", "logprob_stats", "decode_merge",
           "gdr_step_bwd"]


def kernel_timing(enable: bool) -> None:
    """Starts (and zeroes) or stops the library's per-kernel HIP event timers."""
    lib().dm_kernel_timing(1 if enable else 0)


def kernel_times() -> dict:
    """{kernel: (total ms, launches)} since timing was enabled; waits for the recorded events."""
    out = {}
    for i, name in enumerate(KERNELS):
        ms, n = ctypes.c_double(), ctypes.c_uint64()
        lib().dm_kernel_time(i, ctypes.byref(ms), ctypes.byref(n))
        out[name] = (ms.value, int(n.value))
    return out


def describe() -> str:
    buf = ctypes.create_string_buffer(256)
    lib().dm_describe(buf, 256)
    return buf.value.decode()
