"""sycl_minimax_h3_amd: MI355X (gfx950) HIP kernels for MiniMax H3's per-token layer work, behind the C ABI of
include/h3hip.h (a drop-in for maxfridbe/sycl_minimax_h3's kernels/h3sycl.h), and a Python host mirror of the
reference engine's device and ops layers (engine/h3-core/src/device.rs, ops.rs).

The compute is libh3hip.so; there is no other path. ``load()`` opens it and fails loudly when it is not built.
"""
from . import api
from .api import (ACT_GELU_TANH, ACT_NONE, ACT_SILU, BF16, F16, F32, NORM_LAYER, NORM_RMS, ROT_NONE, ROT_REGULAR,
                  ROT_SYLVESTER, load)
from .device import Buf, Device, DType, Error, Tensor
from . import ops

__all__ = ["api", "ops", "load", "Device", "Buf", "Tensor", "DType", "Error", "F32", "F16", "BF16", "ROT_NONE",
           "ROT_REGULAR", "ROT_SYLVESTER", "ACT_NONE", "ACT_GELU_TANH", "ACT_SILU", "NORM_RMS", "NORM_LAYER"]
