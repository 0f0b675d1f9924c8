"""ninfer_amd — MI355X (gfx950) MTP speculative-decoding verify step.

Layers:
  include/ninfer_amd.h          C ABI (the drop-in boundary)
  include/ninfer_amd/ops.hpp    C++20 mirror of the reference ninfer::ops signatures
  ninfer_amd/csrc/              hand-written gfx950 kernels and the C ABI implementation
  ninfer_amd.ops                Python mirror of the op surface (ctypes over the C ABI)
"""
from __future__ import annotations

from . import _capi
from ._capi import (BF16, FP16, FP32, I8, I32, I64, U8, CommitEnvelope, CyclicKVLayerView, GeneralConfig,
                    GqaEnvelope, KVLayerView, SamplingConfig, Tensor, Weight, lib)

__all__ = [
    "BF16", "FP16", "FP32", "I8", "I32", "I64", "Tensor", "KVLayerView", "CyclicKVLayerView", "GqaEnvelope",
    "Weight",
    "CommitEnvelope", "SamplingConfig", "GeneralConfig", "lib", "build_info",
]


def build_info() -> str:
    return lib().nmi_build_info().decode()
