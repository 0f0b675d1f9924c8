"""KV cache planes for one attention layer (reference src/core/kv_cache.{h,cpp}).

Layout per layer (reference plan_kv_cache, src/core/kv_cache.cpp:55-99): codes I8 [D, P, Hkv]
and FP16 scales [D/64, P, Hkv] for K and for V, or BF16 values [D, P, Hkv] and no scales, with
P = align_up(max_context, 128). A trailing batch dimension B stacks independent sequences (one
contiguous region per sequence).
"""
from __future__ import annotations

import ctypes as C

from . import _capi
from ._capi import KVLayerView, Tensor
from .device import DeviceArray

QUANT_GROUP = 64


def align_up(v: int, a: int) -> int:
    return (v + a - 1) // a * a


class KVCacheLayer:
    """Owning cache planes (INT8-G64 by default, or BF16) and the matching nmi_kv_layer_view."""

    def __init__(self, max_context: int, num_kv_heads: int, head_dim: int, batch: int = 1,
                 dtype: int = _capi.I8):
        if max_context <= 0 or max_context > 0x7FFFFFFF:
            raise ValueError("KVCache max_context out of range")
        if num_kv_heads <= 0 or head_dim <= 0 or head_dim % QUANT_GROUP:
            raise ValueError("KVCache geometry invalid")
        if dtype not in (_capi.I8, _capi.BF16):
            raise ValueError("KVCache dtype must be I8 or BF16")
        self.dtype = dtype
        self.max_context = max_context
        self.padded_context = align_up(max_context, 128)
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.batch = batch
        P = self.padded_context
        G = head_dim // QUANT_GROUP
        self.k = DeviceArray(dtype, (head_dim, P, num_kv_heads, batch))
        self.v = DeviceArray(dtype, (head_dim, P, num_kv_heads, batch))
        if dtype == _capi.I8:
            self.k_scale = DeviceArray(_capi.FP16, (G, P, num_kv_heads, batch))
            self.v_scale = DeviceArray(_capi.FP16, (G, P, num_kv_heads, batch))
        else:
            self.k_scale = self.v_scale = None

    def _planes(self):
        return [a for a in (self.k, self.v, self.k_scale, self.v_scale) if a is not None]

    def zero(self, stream=None) -> None:
        for a in self._planes():
            a.zero(stream)

    def view(self) -> KVLayerView:
        v = KVLayerView()
        v.k = self.k.tensor()
        v.v = self.v.tensor()
        if self.k_scale is not None:
            v.k_scale = self.k_scale.tensor()
            v.v_scale = self.v_scale.tensor()
        v.max_context = self.max_context
        v.padded_context = self.padded_context
        v.num_kv_heads = self.num_kv_heads
        v.head_dim = self.head_dim
        v.dtype = self.dtype
        v.quant_group = QUANT_GROUP if self.dtype == _capi.I8 else 0
        return v

    def payload_bytes(self) -> int:
        return sum(a.nbytes for a in self._planes())

    # host views in the reference's order: codes[b][h][pos][d], scales[b][h][pos][g]
    # (BF16: (k, v) values[b][h][pos][d])
    def download(self):
        P, H, D, B = self.padded_context, self.num_kv_heads, self.head_dim, self.batch
        if self.dtype == _capi.BF16:
            return (self.k.numpy().reshape(B, H, P, D), self.v.numpy().reshape(B, H, P, D))
        G = D // QUANT_GROUP
        return (
            self.k.numpy().reshape(B, H, P, D),
            self.v.numpy().reshape(B, H, P, D),
            self.k_scale.numpy().reshape(B, H, P, G),
            self.v_scale.numpy().reshape(B, H, P, G),
        )

    def upload(self, k_codes, v_codes, k_scales=None, v_scales=None) -> None:
        self.k.upload(k_codes)
        self.v.upload(v_codes)
        if self.k_scale is not None:
            self.k_scale.upload(k_scales)
            self.v_scale.upload(v_scales)
