"""ctypes mirror of include/ninfer_amd.h and include/ninfer_amd_runtime.h.

The library is loaded from this package directory only (the in-tree build). A missing library is
an ImportError at first use: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libninfer_amd.so"

# nmi_status
OK, INVALID_ARGUMENT, OVERFLOW, HIP_ERROR, UNSUPPORTED = 0, 1, 2, 3, 4
# nmi_dtype
# ninfer::DType values (src/core/dtype.h:8-16)
BF16, FP32, I32, U8, I64, I8, FP16 = 0, 1, 2, 3, 4, 5, 6
DTYPE_SIZE = {BF16: 2, FP16: 2, FP32: 4, I8: 1, U8: 1, I32: 4, I64: 8}


class Tensor(C.Structure):
    """nmi_tensor — the reference's non-owning view (src/core/tensor.h:11-15)."""

    _fields_ = [
        ("data", C.c_void_p),
        ("dtype", C.c_int32),
        ("ne", C.c_int32 * 4),
        ("nb", C.c_int64 * 4),
    ]

    @classmethod
    def make(cls, data: int | None, dtype: int, shape) -> "Tensor":
        """Contiguous view, shape in the reference's ne order (first index fastest)."""
        shape = list(shape) + [1] * (4 - len(shape))
        t = cls()
        t.data = data or None
        t.dtype = dtype
        stride = DTYPE_SIZE[dtype]
        for i in range(4):
            t.ne[i] = int(shape[i])
            t.nb[i] = stride
            stride *= int(shape[i])
        return t


class Weight(C.Structure):
    """nmi_weight (src/core/tensor.h:47-66), field for field."""

    _fields_ = [
        ("payload", C.c_void_p),
        ("payload_bytes", C.c_uint64),
        ("high_plane_bytes", C.c_uint64),
        ("qtype", C.c_int32),
        ("group_size", C.c_uint32),
        ("shape", C.c_int32 * 4),
        ("padded_shape", C.c_int32 * 4),
        ("ndim", C.c_uint32),
        ("qdata", C.c_void_p),
        ("qhigh", C.c_void_p),
        ("scales", C.c_void_p),
        ("n", C.c_int32),
        ("k", C.c_int32),
        ("group", C.c_int32),
        ("layout", C.c_int32),
        ("scale_dtype", C.c_int32),
    ]


Q6G64_F16S = 2
ROW_SPLIT = 0


class KVLayerView(C.Structure):
    """nmi_kv_layer_view (src/core/kv_cache.h:13-24)."""

    _fields_ = [
        ("k", Tensor),
        ("v", Tensor),
        ("k_scale", Tensor),
        ("v_scale", Tensor),
        ("max_context", C.c_uint32),
        ("padded_context", C.c_uint32),
        ("num_kv_heads", C.c_int32),
        ("head_dim", C.c_int32),
        ("dtype", C.c_int32),
        ("quant_group", C.c_int32),
    ]


class CyclicKVLayerView(C.Structure):
    """nmi_cyclic_kv_layer_view (src/core/kv_cache.h:32-43)."""

    _fields_ = [
        ("k", Tensor),
        ("v", Tensor),
        ("k_scale", Tensor),
        ("v_scale", Tensor),
        ("capacity", C.c_uint32),
        ("padded_capacity", C.c_uint32),
        ("num_kv_heads", C.c_int32),
        ("head_dim", C.c_int32),
        ("dtype", C.c_int32),
        ("quant_group", C.c_int32),
    ]


class GqaEnvelope(C.Structure):
    _fields_ = [("min_visible_keys", C.c_uint32), ("max_visible_keys", C.c_uint32)]


class CommitEnvelope(C.Structure):
    _fields_ = [("min_count", C.c_uint32), ("max_count", C.c_uint32)]


class SamplingConfig(C.Structure):
    """nmi_sampling_config — byte-identical to the reference SamplingConfig (40 bytes)."""

    _fields_ = [
        ("temperature", C.c_float),
        ("top_k", C.c_int32),
        ("top_p", C.c_float),
        ("min_p", C.c_float),
        ("presence_penalty", C.c_float),
        ("frequency_penalty", C.c_float),
        ("seed", C.c_uint64),
        ("token_counts", C.c_void_p),
    ]


class GeneralConfig(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float)]


assert C.sizeof(SamplingConfig) == 40

P = C.POINTER
_T = P(Tensor)
_STREAM = C.c_void_p

_SIGNATURES = {
    "nmi_last_error": (C.c_char_p, []),
    "nmi_build_info": (C.c_char_p, []),
    "nmi_gqa_attention_workspace_bytes": (C.c_size_t, [C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_uint32]),
    "nmi_gqa_attention_workspace_bound": (C.c_int, [C.c_int32, C.c_int32, P(C.c_size_t)]),
    "nmi_gqa_attention": (C.c_int, [_T, _T, _T, _T, C.c_float, P(KVLayerView), GqaEnvelope, C.c_void_p, C.c_size_t, _T, _STREAM]),
    "nmi_gqa_attention_noalloc": (C.c_int, [_T, _T, _T, _T, C.c_float, P(KVLayerView), GqaEnvelope, _T, _STREAM]),
    "nmi_gqa_kv_append": (C.c_int, [_T, _T, _T, P(KVLayerView), _STREAM]),
    "nmi_gqa_attention_cached": (C.c_int, [_T, _T, C.c_float, P(KVLayerView), GqaEnvelope, C.c_void_p, C.c_size_t, _T, _STREAM]),
    "nmi_gqa_attention_tree": (C.c_int, [_T, _T, _T, _T, _T, C.c_float, P(KVLayerView), GqaEnvelope, C.c_int32, C.c_void_p, C.c_size_t, _T, _STREAM]),
    "nmi_argmax": (C.c_int, [_T, _T, C.c_int32, _STREAM]),
    "nmi_sampling_workspace_bytes": (C.c_size_t, [C.c_int32, C.c_int32, C.c_int32]),
    "nmi_speculative_prepare_verify_inputs": (C.c_int, [_T, _T, _T, _T, _T, _STREAM]),
    "nmi_speculative_accept_greedy_drafts": (C.c_int, [_T, _T, _T, _T, _T, _T, _T, _T, _T, C.c_int32, C.c_void_p, C.c_void_p, C.c_size_t, _STREAM]),
    "nmi_general_accept_workspace_bytes": (C.c_size_t, [C.c_int32, C.c_int32, C.c_int32]),
    "nmi_speculative_accept_general": (C.c_int, [_T, _T, _T, _T, _T, _T, _T, _T, _T, _T, _T, C.c_int32, C.c_void_p, C.c_void_p, C.c_size_t, _STREAM]),
    "nmi_speculative_select_accepted_hidden": (C.c_int, [_T, _T, _T, _STREAM]),
    "nmi_mtp_prepare_alignment_ids": (C.c_int, [_T, _T, _T, _T, _STREAM]),
    "nmi_linear": (C.c_int, [_T, P(Weight), _T, _STREAM]),
    "nmi_linear_argmax_workspace_bytes": (C.c_size_t, [C.c_int32]),
    "nmi_linear_argmax": (C.c_int, [_T, P(Weight), C.c_int32, C.c_void_p, C.c_size_t, _T, _STREAM]),
    "nmi_speculative_accept_fused_head_workspace_bytes": (C.c_size_t, [C.c_int32, C.c_int32]),
    "nmi_speculative_accept_fused_head": (C.c_int, [_T, P(Weight), _T, _T, _T, _T, _T, _T, _T, C.c_int32, C.c_void_p,
                                                    C.c_void_p, C.c_size_t, _STREAM]),
    "nmi_gated_delta_rule_workspace_bytes": (C.c_int, [C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, P(C.c_size_t)]),
    "nmi_gated_delta_rule": (C.c_int, [_T, _T, _T, _T, _T, C.c_float, C.c_int32, _T, _T, _T, _STREAM]),
    "nmi_gated_delta_rule_snapshot": (C.c_int, [_T, _T, _T, _T, _T, C.c_float, C.c_int32, _T, _T, _T, _STREAM]),
    "nmi_causal_conv1d_silu": (C.c_int, [_T, _T, _T, _T, _T, _STREAM]),
    "nmi_causal_conv1d_silu_snapshot": (C.c_int, [_T, _T, _T, _T, _T, _STREAM]),
    "nmi_set_i32_scalar": (C.c_int, [_T, C.c_int32, _STREAM]),
    "nmi_assign_i32_scalar": (C.c_int, [_T, _T, _STREAM]),
    "nmi_increment_i32_scalar": (C.c_int, [_T, _STREAM]),
    "nmi_increment_i64_scalar": (C.c_int, [_T, _STREAM]),
    "nmi_kv_cache_append_prefix": (C.c_int, [_T, _T, _T, _T, CommitEnvelope, P(KVLayerView), _STREAM]),
    "nmi_kv_cache_append_prefix_cyclic": (C.c_int, [_T, _T, _T, _T, CommitEnvelope, P(CyclicKVLayerView), _STREAM]),
    "nmi_kv_cache_rollback": (C.c_int, [_T, _T, P(KVLayerView), _STREAM]),
    "nmi_kv_cache_compact_path": (C.c_int, [_T, _T, _T, P(KVLayerView), _STREAM]),
    "nmi_tree_accept_greedy": (C.c_int, [_T, _T, _T, _T, _T, _T, _T, _T, _T, _T, _T, _STREAM]),
    # runtime helpers
    "nmi_rt_device_count": (C.c_int, [P(C.c_int32)]),
    "nmi_rt_device_name": (C.c_int, [C.c_char_p, C.c_size_t]),
    "nmi_rt_malloc": (C.c_int, [P(C.c_void_p), C.c_size_t]),
    "nmi_rt_free": (C.c_int, [C.c_void_p]),
    "nmi_rt_memcpy_htod": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "nmi_rt_memcpy_dtoh": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "nmi_rt_memcpy_dtod": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, _STREAM]),
    "nmi_rt_fill_u8": (C.c_int, [C.c_void_p, C.c_uint8, C.c_size_t, _STREAM]),
    "nmi_rt_next_row_i32": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_void_p, C.c_void_p, _STREAM]),
    "nmi_rt_stream_create": (C.c_int, [P(C.c_void_p)]),
    "nmi_rt_stream_destroy": (C.c_int, [_STREAM]),
    "nmi_rt_stream_synchronize": (C.c_int, [_STREAM]),
    "nmi_rt_device_synchronize": (C.c_int, []),
    "nmi_rt_event_create": (C.c_int, [P(C.c_void_p)]),
    "nmi_rt_event_destroy": (C.c_int, [C.c_void_p]),
    "nmi_rt_event_record": (C.c_int, [C.c_void_p, _STREAM]),
    "nmi_rt_event_elapsed_ms": (C.c_int, [P(C.c_float), C.c_void_p, C.c_void_p]),
    "nmi_rt_capture_begin": (C.c_int, [_STREAM]),
    "nmi_rt_capture_end": (C.c_int, [_STREAM, P(C.c_void_p)]),
    "nmi_rt_graph_launch": (C.c_int, [C.c_void_p, _STREAM]),
    "nmi_rt_graph_destroy": (C.c_int, [C.c_void_p]),
    "nmi_rt_stream_copy": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, _STREAM]),
    "nmi_rt_read_ceiling": (C.c_int, [C.c_void_p, C.c_size_t, C.c_int32, C.c_void_p, _STREAM]),
}

_lib: C.CDLL | None = None


def lib() -> C.CDLL:
    """Load the in-tree gfx950 library (raises if it was never built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: run `python -m ninfer_amd.build` (or __graft_entry__.build())"
            )
        handle = C.CDLL(os.fspath(LIB_PATH), mode=C.RTLD_GLOBAL)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


class NmiError(RuntimeError):
    pass


def check(status: int) -> None:
    """Map an nmi_status to the Python analogue of the reference's exception."""
    if status == OK:
        return
    msg = (lib().nmi_last_error() or b"").decode()
    if status == INVALID_ARGUMENT:
        raise ValueError(msg)  # std::invalid_argument
    if status == OVERFLOW:
        raise OverflowError(msg)  # std::overflow_error
    if status == UNSUPPORTED:
        raise NotImplementedError(msg)
    raise NmiError(msg)
