"""Raw bindings to libh3hip.so: one ctypes function per declaration of include/h3hip.h.

Mirrors engine/h3-sys/src/lib.rs (the Rust engine's loader of the reference library): the library is opened at run
time, every function of the reference's header (kernels/h3sycl.h) is resolved by name, and a library missing any of
them is refused (lib.rs:215-283). It is looked for at $H3SYCL_LIB, then beside this package (lib.rs:181-193 looks
beside the executable). There is no fallback: without the built library nothing here works.
"""
from __future__ import annotations

import ctypes as C
import os

F32, F16, BF16 = 0, 1, 2
ROT_NONE, ROT_REGULAR, ROT_SYLVESTER = 0, 1, 2
ACT_NONE, ACT_GELU_TANH, ACT_SILU = 0, 1, 2
NORM_RMS, NORM_LAYER = 0, 1

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libh3hip.so"

vp, i64, i32, f32, u64, cp = C.c_void_p, C.c_int64, C.c_int, C.c_float, C.c_uint64, C.c_char_p

# every function of kernels/h3sycl.h (the 48 engine/h3-sys resolves, lib.rs:234-281, plus h3s_create)
REFERENCE = {
    "h3s_last_error": (cp, []),
    "h3s_open": (vp, []),
    "h3s_gpu_count": (i32, []),
    "h3s_gpu_info": (i32, [i32, vp, i32, vp, vp, i32]),
    "h3s_open_gpu": (vp, [i32]),
    "h3s_create": (vp, [vp]),
    "h3s_destroy": (None, [vp]),
    "h3s_device_name": (cp, [vp]),
    "h3s_alloc": (vp, [vp, u64]),
    "h3s_free": (None, [vp, vp]),
    "h3s_mem_used": (u64, [vp]),
    "h3s_mem_cap": (u64, [vp]),
    "h3s_mem_free": (u64, [vp]),
    "h3s_write": (i32, [vp, vp, vp, u64]),
    "h3s_read": (i32, [vp, vp, vp, u64]),
    "h3s_copy": (i32, [vp, vp, vp, u64]),
    "h3s_wait": (i32, [vp]),
    "h3s_alloc_host": (vp, [vp, u64]),
    "h3s_free_host": (None, [vp, vp]),
    "h3s_upload": (i32, [vp, vp, vp, u64]),
    "h3s_upload_wait": (i32, [vp]),
    "h3s_int8_linear": (i32, [vp, vp, i32, i64, i64, vp, i64, vp, i64, vp, vp, i32, i32]),
    "h3s_linear_acc": (i32, [vp, vp, i32, i64, i64, vp, i64, vp, vp]),
    "h3s_scale_rows": (i32, [vp, vp, i32, i64, i64, vp]),
    "h3s_linear": (i32, [vp, vp, i32, i64, i64, vp, i64, vp, vp, i32]),
    "h3s_dequant": (i32, [vp, vp, i32, i64, vp, i32]),
    "h3s_attention_causal": (i32, [vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, i64, vp]),
    "h3s_conv3d": (i32, [vp, vp, i32, i64, i64, i64, i64, vp, i64, i64, vp, vp]),
    "h3s_group_norm_silu": (i32, [vp, vp, i32, i64, i64, i64, i64, vp, vp, f32, vp, vp, vp]),
    "h3s_pad3d": (i32, [vp, vp, i32, i64, i64, i64, i64, i64, i64, i64, i64, i64, vp]),
    "h3s_conv2d": (i32, [vp, vp, i32, i64, i64, i64, i64, vp, i64, i64, vp, vp]),
    "h3s_prelu": (i32, [vp, vp, i32, i64, i64, vp]),
    "h3s_pixel_shuffle_add": (i32, [vp, vp, i32, i64, i64, i64, i64, i64, vp, vp]),
    "h3s_resize_area": (i32, [vp, vp, i32, i64, i64, i64, i64, i64, i64, vp]),
    "h3s_conv3d_ex": (i32, [vp, vp, i32, i64, i64, i64, i64, vp, i64, i64, i64, i64, i64, i64, i64, vp, vp]),
    "h3s_temporal_dwconv": (i32, [vp, vp, i32, i64, i64, i64, vp, i64, vp, vp]),
    "h3s_trilinear": (i32, [vp, vp, i32, i64, i64, i64, i64, i64, i64, i64, vp]),
    "h3s_conv1d": (i32, [vp, vp, i64, i64, i64, vp, i64, i64, vp, i64, i64, i64, vp, i64]),
    "h3s_conv_transpose1d": (i32, [vp, vp, i64, i64, i64, vp, i64, i64, vp, i64, i64, vp, i64]),
    "h3s_aa_snake": (i32, [vp, vp, i64, i64, i64, vp, vp, vp, vp, vp]),
    "h3s_scale": (i32, [vp, vp, i64, f32]),
    "h3s_snake": (i32, [vp, vp, i64, i64, i64, vp, vp]),
    "h3s_layer_norm": (i32, [vp, vp, i32, i64, i64, vp, vp, f32, vp, i32]),
    "h3s_rms_norm_mod": (i32, [vp, vp, i32, i64, i64, vp, f32, vp, vp, vp, vp, i32]),
    "h3s_rms_rope": (i32, [vp, vp, i32, i64, i64, i64, i64, vp, f32, vp, i32]),
    "h3s_swiglu": (i32, [vp, vp, i32, i64, i64, vp, i32]),
    "h3s_gate_add": (i32, [vp, vp, i32, i64, i64, vp, i32, vp, vp]),
    "h3s_attention": (i32, [vp, vp, vp, vp, i32, i64, i64, i64, i64, vp, i32]),
    "h3s_attention_batch": (i32, [vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, vp, i32]),
}

# the additions of include/h3hip.h
ADDITIONS = {
    "h3s_stream": (vp, [vp]),
    "h3s_norm_quant": (i32, [vp, vp, i32, i64, i64, vp, f32, vp, vp, vp, i32, i32, i32, i32, vp, vp]),
    "h3s_swiglu_quant": (i32, [vp, vp, i32, i64, i64, i32, i32, i32, vp, vp]),
    "h3s_adaln_tables": (i32, [vp, vp, vp, vp, i64, i64, i64, i64, vp]),
    "h3s_rotations": (i32, [vp, vp, i64, vp, i64, vp]),
    "h3s_norm_mod_act_gate": (i32, [vp, vp, i32, i64, i64, i32, vp, vp, f32, vp, vp, vp, vp, i32, i32, vp, i32, vp, i32]),
    "h3s_qk_rms_rope": (i32, [vp, vp, vp, i32, i64, i64, i64, i64, vp, vp, f32, vp, i32]),
    "h3s_int8_gemm_dequant": (i32, [vp, vp, vp, i64, i64, vp, i64, vp, i64, vp, i32, vp, i32]),
    "h3s_int8_linear_noalloc": (i32, [vp, vp, i32, i64, i64, vp, i64, vp, i64, vp, vp, i32, i32]),
    "h3s_int8_quantize": (i32, [vp, vp, i32, i64, i64, i32, vp, vp]),
    "h3s_alloc_count": (u64, []),
    "h3s_layout_plan": (i64, [i64, i64, i64, i64, i64, vp, i64, vp, i64, vp, vp, vp, i64]),
    "h3s_layout": (i32, [vp, i64, i64, i64, i64, i64, vp, i64, vp, i64, vp, vp, vp, i64]),
}


def candidates() -> list[str]:
    """Where the library is looked for: $H3SYCL_LIB, then beside this package (engine/h3-sys/src/lib.rs:181-193)."""
    out = []
    if os.environ.get("H3SYCL_LIB"):
        out.append(os.environ["H3SYCL_LIB"])
    out.append(os.path.join(_HERE, LIB_NAME))
    return out


class Api:
    """The functions of include/h3hip.h, resolved once (engine/h3-sys/src/lib.rs:198-211)."""

    def __init__(self, path: str):
        self.path = path
        self.lib = C.CDLL(path, mode=C.RTLD_GLOBAL)
        for name, (res, args) in {**REFERENCE, **ADDITIONS}.items():
            try:
                fn = getattr(self.lib, name)
            except AttributeError:
                raise OSError(f"{name} is missing from the library ({path})") from None
            fn.restype = res
            fn.argtypes = args
            setattr(self, name[len("h3s_"):], fn)

    def error(self) -> str:
        """The library's last error on this thread."""
        return (self.lib.h3s_last_error() or b"").decode(errors="replace")


_api: Api | None = None


def load() -> Api:
    """Opens the library and resolves every function; raises with every place tried when it cannot."""
    global _api
    if _api is not None:
        return _api
    tried = []
    for p in candidates():
        if not os.path.exists(p):
            tried.append(f"{p} (no such file)")
            continue
        try:
            _api = Api(p)
            return _api
        except OSError as e:
            tried.append(f"{p}: {e}")
    raise OSError("libh3hip.so could not be loaded (build it with __graft_entry__.build()):\n  " + "\n  ".join(tried))
