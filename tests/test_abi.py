"""The C ABI without a GPU: libh3hip.so loads, exports every function of include/h3hip.h (and so every name
engine/h3-sys resolves), and refuses bad arguments with a message before touching the device. CPU only: no call
here launches a kernel."""
import ctypes as C
import os
import re
import subprocess

import pytest

from sycl_minimax_h3_amd import api as A

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "h3hip.h")
# the 48 names engine/h3-sys resolves (engine/h3-sys/src/lib.rs:234-281), plus h3s_create (kernels/h3sycl.h:35)
H3SYS = """last_error open gpu_count gpu_info open_gpu destroy device_name alloc free mem_used mem_cap mem_free write read
wait copy alloc_host free_host upload upload_wait int8_linear linear linear_acc scale_rows dequant attention_causal conv3d
conv2d prelu pixel_shuffle_add resize_area group_norm_silu pad3d conv3d_ex temporal_dwconv trilinear conv1d
conv_transpose1d aa_snake scale snake layer_norm rms_norm_mod rms_rope swiglu gate_add attention attention_batch""".split()


@pytest.fixture(scope="module")
def api():
    return A.load()


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(h3s_[a-z0-9_]+)\s*\(", text)))


def test_header_and_library_agree(api):
    names = declared()
    # the 49 of kernels/h3sycl.h, 11 additions, the allocation-free int8 linear and the allocation counter
    assert len(names) == 62
    out = subprocess.run(["nm", "-D", "--defined-only", api.path], capture_output=True, text=True, check=True).stdout
    exported = sorted(set(l.split()[-1] for l in out.splitlines() if l.split()[-1].startswith("h3s_")))
    assert exported == names, f"missing {set(names) - set(exported)}, extra {set(exported) - set(names)}"
    # nothing else leaks out of the library
    others = [l.split()[-1] for l in out.splitlines() if l.split()[1] == "T" and not l.split()[-1].startswith("h3s_")]
    assert others == [], others[:10]


def test_every_name_h3sys_resolves(api):
    assert len(H3SYS) == 48
    lib = C.CDLL(api.path)
    for n in H3SYS + ["create"]:
        assert hasattr(lib, "h3s_" + n), n
    assert set("h3s_" + n for n in H3SYS + ["create"]) == set(A.REFERENCE)


def test_alloc_count_is_a_counter(api):
    n = api.alloc_count()
    assert isinstance(n, int) and n >= 0 and api.alloc_count() == n


def test_no_context_is_an_error(api):
    assert api.rms_norm_mod(None, 16, 2, 4, 4096, 16, 1e-6, None, None, None, 16, 2) == -1
    assert "no context" in api.error()
    assert api.wait(None) == -1
    assert not api.alloc(None, 16)


def test_arguments_are_checked_before_the_device(api):
    p = 1 << 20   # a 16-byte aligned address that is never dereferenced: every call below fails its checks first
    assert api.int8_quantize(None, p, 2, 8, 256, 128, p, p) == -1
    assert "group" in api.error()
    assert api.int8_quantize(None, p + 8, 2, 8, 256, 64, p, p) == -1
    assert "aligned" in api.error()
    assert api.int8_linear(None, p, 2, 8, 256, p, 8, p, 1, None, p, 2, 128) == -1
    assert "group" in api.error()
    assert api.int8_linear(None, p, 2, 8, 100, p, 8, p, 1, None, p, 2, 0) == -1
    assert "multiple of 64" in api.error()
    assert api.int8_linear(None, p, 2, 8, 256, p, 8, p, 3, None, p, 2, 0) == -1
    assert "weight scales" in api.error()
    # the allocation-free int8 linear refuses rows longer than its fixed scratch takes, before the device
    assert api.int8_linear_noalloc(None, p, 2, 8, 131072, p, 8, p, 1, None, p, 2, 0) == -1
    assert "65536" in api.error()
    assert api.int8_linear_noalloc(None, p, 2, 8, 256, p, 8, p, 1, None, p, 2, 128) == -1
    assert "group" in api.error()
    assert api.rms_rope(None, p, 2, 4, 32, 128, 4096, p, 1e-5, p, 127) == -1
    assert "rot_dim" in api.error()
    assert api.rms_rope(None, p, 2, 4, 32, 128, 4000, p, 1e-5, p, 128) == -1
    assert "stride" in api.error()
    # any even rot_dim with an even remainder passes the checks (kernels/h3sycl.cpp:1280-1282): 12 and 126 reach the
    # context check; a head that is not whole 16-byte vectors does not
    assert api.rms_rope(None, p, 2, 4, 32, 128, 4096, p, 1e-5, p, 12) == -1
    assert "no context" in api.error()
    assert api.rms_rope(None, p, 2, 4, 56, 128, 3 * 7168, p, 1e-5, p, 126) == -1
    assert "no context" in api.error()
    assert api.rms_rope(None, p, 2, 4, 32, 100, 3200, p, 1e-5, p, 96) == -1
    assert "16-byte" in api.error()
    assert api.rms_norm_mod(None, p, 2, 4, 4100, p, 1e-6, None, None, None, p, 2) == -1
    assert "multiple of 8" in api.error()
    assert api.rms_norm_mod(None, p + 2, 2, 4, 4096, p, 1e-6, None, None, None, p, 2) == -1
    assert "aligned" in api.error()
    assert api.rms_norm_mod(None, p, 7, 4, 4096, p, 1e-6, None, None, None, p, 2) == -1
    assert "element type" in api.error()
    assert api.rms_norm_mod(None, p, 2, 4, 16392, p, 1e-6, None, None, None, p, 2) == -1
    assert "not supported" in api.error()
    assert api.gate_add(None, p, 2, 4, 4096, p, 2, None, p) == -1
    assert "row table" in api.error()
    assert api.norm_quant(None, p, 2, 4, 4096, p, 1e-6, None, None, None, 0, 2, 2, 96, p, p) == -1
    assert "Sylvester" in api.error()
    assert api.norm_quant(None, p, 2, 4, 4096, p, 1e-6, None, None, None, 0, 2, 1, 128, p, p) == -1
    assert "power of 4" in api.error()
    assert api.norm_mod_act_gate(None, p, 2, 4, 4096, 5, None, None, 1e-5, None, None, None, None, 0, 0, None, 2, p, 2) == -1
    assert "norm" in api.error()
    assert api.swiglu_quant(None, p, 2, 4, 4100, 2, 0, 0, p, p) == -1
    assert "multiple of 8" in api.error()
    assert api.swiglu_quant(None, p, 2, 4, 4096, 2, 1, 32, p, p) == -1
    assert "power of 4" in api.error()
    assert api.swiglu_quant(None, p, 2, 4, 4096, 2, 0, 0, p, None) == -1
    assert "required" in api.error()


def test_empty_shapes_do_nothing(api):
    # kernels/h3sycl.cpp:636, 787: zero-size calls return 0 before anything else, context or not
    assert api.rms_norm_mod(None, None, 2, 0, 4096, None, 1e-6, None, None, None, None, 2) == 0
    assert api.int8_linear(None, None, 2, 0, 4096, None, 8, None, 1, None, None, 2, 0) == 0
    assert api.rms_rope(None, None, 2, 4, 0, 128, 4096, None, 1e-5, None, 128) == 0
    assert api.swiglu(None, None, 2, 0, 64, None, 2) == 0
    assert api.swiglu_quant(None, None, 2, 0, 64, 2, 0, 0, None, None) == 0


def test_out_of_scope_entry_points_refuse(api):
    assert api.linear(None, None, 7, 1, 1, None, 1, None, None, 2) == -1
    assert "element type" in api.error()
    assert api.conv3d(None, None, 2, 1, 1, 1, 1, None, 1, 3, None, None) == -1
    assert "not implemented" in api.error()
    assert api.attention_causal(None, None, None, None, 2, 4, 3, 2, 64, 192, 128, None) == -1
    assert "multiple" in api.error()
    # attention's argument checks run before the context is looked at
    assert api.attention(None, None, None, None, 2, 1, 1, 300, 300, None, 2) == -1
    assert "at most 256" in api.error()
    assert api.attention_causal(None, None, None, None, 2, 4, 2, 2, 257, 514, 514, None) == -1
    assert "D <= 256" in api.error()
    # any head size up to 256 passes the size check (and then needs its buffers)
    assert api.attention(None, None, None, None, 2, 1, 1, 96, 96, None, 2) == -1
    assert "required" in api.error()
    assert api.attention(None, None, None, None, 2, 1, 2, 64, 100, None, 2) == -1
    assert "stride" in api.error()
    assert api.conv3d(None, None, 2, 1, 1, 1, 1, None, 1, 3, None, None) == -1
    assert "not implemented" in api.error()


def test_ops_layer_checks_shapes(api):
    """The Python mirror of ops.rs refuses shapes that do not fit before calling the library."""
    from sycl_minimax_h3_amd import DType, Error, Tensor, ops

    class FakeDev:
        pass

    d = FakeDev()
    x = Tensor(DType.BF16, [4, 4096], 1 << 20, None, d)
    w = Tensor(DType.F32, [4096], 1 << 20, None, d)
    bad_out = Tensor(DType.BF16, [4, 4095], 1 << 20, None, d)
    with pytest.raises(Error, match="rms_norm"):
        ops.rms_norm_mod(x, w, 1e-6, None, bad_out)
    with pytest.raises(Error, match="float32"):
        ops.rms_norm_mod(x, Tensor(DType.BF16, [4096], 1 << 20, None, d), 1e-6, None, x)
    with pytest.raises(Error, match="do not fit"):
        ops.rms_rope(ops.Rows(x, 0, 4000, 4, 32, 128), w, 1e-5, w, 128)
    with pytest.raises(Error, match="int8"):
        ops.Int8Linear(x, w).forward(x, x)
    with pytest.raises(Error, match="twice"):
        ops.swiglu(x, x)
