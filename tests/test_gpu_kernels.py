"""GPU parity: every kernel of libh3hip.so, called through the C ABI (the Python mirror of engine/h3-core/src/ops.rs),
against the CPU oracle on the same seeded inputs. Bit-exact where the arithmetic is +, -, *, /, sqrt and fma;
the parity tolerance (1 bf16 ulp on few elements, relative L2 < 1e-3) where it goes through exp or tanh."""
import numpy as np
import pytest

from oracle import oracle as o
from helpers import assert_bits_equal, assert_close_16, codes_close, new, up

pytestmark = pytest.mark.gpu

from sycl_minimax_h3_amd import DType, Error, ops  # noqa: E402

DTS = {o.F32: DType.F32, o.F16: DType.F16, o.BF16: DType.BF16}
o.set_threads(8)


def inputs(seed, n, dt, scale=1.0):
    return o.to_dt(np.random.default_rng(seed).standard_normal(n).astype(np.float32) * scale, dt)


def weight(seed, n):
    return (1.0 + 0.1 * np.random.default_rng(seed).standard_normal(n)).astype(np.float32)


# ---- context and memory (kernels/h3sycl.h:22-70) ----
def test_context_and_memory(dev):
    assert dev.mem_cap() > 0
    used = dev.mem_used()
    a = np.arange(1 << 20, dtype=np.uint8)
    t = up(dev, a, "U8", [a.size])
    assert dev.mem_used() == used + a.size
    assert np.array_equal(t.to_numpy(), a)
    t2 = new(dev, "U8", [a.size])
    dev.check(dev.api.copy(dev.ctx, t2.ptr(), t.ptr(), a.size))
    dev.wait()
    assert np.array_equal(t2.to_numpy(), a)
    # pinned upload beside the kernels
    p = dev.api.alloc_host(dev.ctx, a.size)
    assert p
    import ctypes

    ctypes.memmove(p, a.ctypes.data, a.size)
    t3 = new(dev, "U8", [a.size])
    dev.check(dev.api.upload(dev.ctx, t3.ptr(), p, a.size))
    dev.check(dev.api.upload_wait(dev.ctx))
    assert np.array_equal(t3.to_numpy(), a)
    # a pageable source is refused (kernels/h3sycl.h:65-67)
    assert dev.api.upload(dev.ctx, t3.ptr(), a.ctypes.data, a.size) == -1
    dev.api.free_host(dev.ctx, p)
    # the cap refuses, with a message, instead of asking the driver
    assert not dev.api.alloc(dev.ctx, dev.mem_cap() + 1)
    assert "budget" in dev.api.error()
    assert dev.mem_used() == used + 3 * a.size                      # the refused request took nothing
    assert dev.api.gpu_count() >= 1
    name = dev.name()
    assert name


# ---- h3s_rms_norm_mod (kernels/h3sycl.cpp:766-810) ----
# row lengths that reach every launch plan (lanes per row x chunks per lane) for 16-bit and float32 rows
ROW_SHAPES = [(7, 4096), (33, 5376), (5, 64), (9, 520), (6, 1536), (4, 2040), (5, 2048), (3, 8192), (3, 8200), (2, 16384)]


def too_long(C, x_dt):
    return C // (16 // (4 if x_dt == o.F32 else 2)) > 2048


@pytest.mark.parametrize("x_dt,out_dt", [(o.BF16, o.BF16), (o.BF16, o.F32), (o.F16, o.F16), (o.F32, o.F32), (o.F32, o.BF16)])
@pytest.mark.parametrize("M,C", ROW_SHAPES)
@pytest.mark.parametrize("mod", [False, True])
def test_rms_norm_mod(dev, x_dt, out_dt, M, C, mod):
    if C % (16 // (4 if x_dt == o.F32 else 2)):
        pytest.skip("not whole vectors")
    x = inputs(1, M * C, x_dt, 2.0)
    w = weight(2, C)
    R = 3
    rows = (np.arange(M) % R).astype(np.int32) if mod else None
    sc = (0.5 * np.random.default_rng(3).standard_normal((R, C))).astype(np.float32) if mod else None
    sh = (0.5 * np.random.default_rng(4).standard_normal((R, C))).astype(np.float32) if mod else None
    xt = up(dev, x, DTS[x_dt], [M, C])
    out = new(dev, DTS[out_dt], [M, C])
    m = ops.Mod(up(dev, rows, "I32", [M]), up(dev, sc, "F32", [R, C]), up(dev, sh, "F32", [R, C])) if mod else None
    if too_long(C, x_dt):
        # rows are held in registers, at most 2048 16-byte vectors a row: longer ones are refused, with the reason
        with pytest.raises(Error, match="not supported"):
            ops.rms_norm_mod(xt, up(dev, w, "F32", [C]), 1e-6, m, out)
        return
    want = o.rms_norm_mod(x, x_dt, M, C, w, 1e-6, rows, sc, sh, out_dt)
    ops.rms_norm_mod(xt, up(dev, w, "F32", [C]), 1e-6, m, out)
    assert_bits_equal(out.to_numpy(), want, "rms_norm_mod")


def test_rms_norm_in_place(dev):
    M, C = 17, 4096
    x = inputs(5, M * C, o.BF16)
    w = weight(6, C)
    want = o.rms_norm_mod(x, o.BF16, M, C, w, 1e-5)
    xt = up(dev, x, "BF16", [M, C])
    ops.rms_norm_mod(xt, up(dev, w, "F32", [C]), 1e-5, None, xt)
    assert_bits_equal(xt.to_numpy(), want, "rms_norm_mod in place")


# ---- h3s_layer_norm (kernels/h3sycl.cpp:1248-1274) ----
@pytest.mark.parametrize("affine", [False, True])
@pytest.mark.parametrize("x_dt,out_dt,C", [(o.BF16, o.F32, 4096), (o.BF16, o.BF16, 1024), (o.F32, o.F32, 260), (o.F32, o.BF16, 4096),
                                           (o.BF16, o.BF16, 16384), (o.F16, o.F32, 5376)])
def test_layer_norm(dev, affine, x_dt, out_dt, C):
    M = 11
    x = o.to_dt(np.random.default_rng(7).standard_normal(M * C).astype(np.float32) * 3 + 1, x_dt)
    w = weight(8, C) if affine else None
    b = (0.1 * np.random.default_rng(9).standard_normal(C)).astype(np.float32) if affine else None
    want = o.layer_norm(x, x_dt, M, C, w, b, 1e-5, out_dt)
    out = new(dev, DTS[out_dt], [M, C])
    ops.layer_norm(up(dev, x, DTS[x_dt], [M, C]), C, up(dev, w, "F32", [C]) if affine else None,
                   up(dev, b, "F32", [C]) if affine else None, 1e-5, out)
    assert_bits_equal(out.to_numpy(), want, "layer_norm")


# ---- h3s_gate_add, h3s_swiglu (kernels/h3sycl.cpp:1378-1431) ----
@pytest.mark.parametrize("x_dt,o_dt", [(o.BF16, o.BF16), (o.BF16, o.F32), (o.F32, o.BF16)])
@pytest.mark.parametrize("gated", [False, True])
def test_gate_add(dev, x_dt, o_dt, gated):
    M, C, R = 19, 1536, 4
    x = inputs(10, M * C, x_dt)
    other = inputs(11, M * C, o_dt)
    rows = (np.arange(M) % R).astype(np.int32)
    gate = (0.5 * np.random.default_rng(12).standard_normal((R, C))).astype(np.float32)
    want = o.gate_add(x, x_dt, M, C, other, o_dt, rows if gated else None, gate if gated else None)
    xt = up(dev, x, DTS[x_dt], [M, C])
    if gated:
        ops.gate_add(xt, up(dev, other, DTS[o_dt], [M, C]), up(dev, rows, "I32", [M]), up(dev, gate, "F32", [R, C]))
    else:
        ops.add(xt, up(dev, other, DTS[o_dt], [M, C]))
    assert_bits_equal(xt.to_numpy(), want, "gate_add")


@pytest.mark.parametrize("x_dt,out_dt", [(o.BF16, o.BF16), (o.F16, o.F16), (o.F32, o.F32)])
def test_swiglu(dev, x_dt, out_dt):
    M, C = 23, 2048
    x = inputs(13, M * 2 * C, x_dt, 3.0)
    want = o.swiglu(x, x_dt, M, C, out_dt)
    out = new(dev, DTS[out_dt], [M, C])
    ops.swiglu(up(dev, x, DTS[x_dt], [M, 2 * C]), out)
    got = out.to_numpy()
    if out_dt == o.F32:
        rel, _ = o.compare(got.ravel(), want)
        assert rel < 1e-6
        assert np.allclose(got.ravel(), want, rtol=2e-6, atol=1e-7)
    else:
        assert_close_16(got, want, out_dt, "swiglu", max_frac=2e-2)


# ---- h3s_rms_rope / h3s_qk_rms_rope (kernels/h3sycl.cpp:1276-1376) ----
def cs_table(seed, M, rot):
    ang = np.random.default_rng(seed).uniform(-50, 50, (M, rot // 2))
    return np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32).ravel()


@pytest.mark.parametrize("x_dt", [o.BF16, o.F16, o.F32])
@pytest.mark.parametrize("H,D,rot,pad", [(32, 128, 128, 0), (4, 64, 48, 0), (3, 128, 0, 64), (5, 128, 96, 8), (2, 64, 64, 0),
                                         (7, 128, 126, 0), (5, 128, 120, 8), (3, 128, 60, 0), (4, 64, 2, 0), (2, 64, 62, 16),
                                         (9, 64, 36, 0)])
def test_rms_rope(dev, x_dt, H, D, rot, pad):
    M = 13
    stride = H * D + pad
    x = inputs(14, M * stride, x_dt)
    w = weight(15, D)
    cs = cs_table(16, M, rot) if rot else np.zeros(4, dtype=np.float32)
    want = o.rms_rope(x, x_dt, M, H, D, stride, w, 1e-5, cs if rot else None, rot)
    xt = up(dev, x, DTS[x_dt], [M * stride])
    ops.rms_rope(ops.Rows(xt, 0, stride, M, H, D), up(dev, w, "F32", [D]), 1e-5, up(dev, cs, "F32", [cs.size]), rot)
    assert_bits_equal(xt.to_numpy(), want, "rms_rope")


def test_rms_rope_long(dev):
    """A long launch, two wavefronts a token: q alone and the fused q and k, 33000 tokens of 16 heads of 128, all
    features rotated."""
    M, H, D, rot = 33000, 16, 128, 128
    w_ = H * D
    qk = inputs(17, M * 2 * w_, o.BF16)
    wq, wk = weight(18, D), weight(19, D)
    cs = cs_table(20, M, rot)
    want_q = o.rms_rope(qk, o.BF16, M, H, D, 2 * w_, wq, 1e-5, cs, rot)
    want = o.rms_rope(want_q[w_:], o.BF16, M, H, D, 2 * w_, wk, 1e-5, cs, rot)
    want = np.concatenate([want_q[:w_], want])
    t = up(dev, qk, "BF16", [M * 2 * w_])
    ops.qk_rms_rope(ops.Rows(t, 0, 2 * w_, M, H, D), ops.Rows(t, w_, 2 * w_, M, H, D), up(dev, wq, "F32", [D]),
                    up(dev, wk, "F32", [D]), 1e-5, up(dev, cs, "F32", [cs.size]), rot)
    assert_bits_equal(t.to_numpy(), want, "qk_rms_rope, 33000 tokens")
    t2 = up(dev, qk, "BF16", [M * 2 * w_])
    ops.rms_rope(ops.Rows(t2, 0, 2 * w_, M, H, D), up(dev, wq, "F32", [D]), 1e-5, up(dev, cs, "F32", [cs.size]), rot)
    assert_bits_equal(t2.to_numpy(), want_q, "rms_rope, 33000 tokens")


def test_qk_rms_rope_in_a_qkv_buffer(dev):
    """q and k inside the qkv linear's output, stride 3 H D (engine/h3-core/src/dit.rs:345-348)."""
    M, H, D, rot = 37, 32, 128, 128
    w_ = H * D
    qkv = inputs(17, M * 3 * w_, o.BF16)
    wq, wk = weight(18, D), weight(19, D)
    cs = cs_table(20, M, rot)
    want = o.rms_rope(qkv, o.BF16, M, H, D, 3 * w_, wq, 1e-5, cs, rot)
    want = o.rms_rope(want[w_:], o.BF16, M, H, D, 3 * w_, wk, 1e-5, cs, rot)
    t = up(dev, qkv, "BF16", [M, 3 * w_])
    ops.qk_rms_rope(ops.Rows(t, 0, 3 * w_, M, H, D), ops.Rows(t, w_, 3 * w_, M, H, D), up(dev, wq, "F32", [D]),
                    up(dev, wk, "F32", [D]), 1e-5, up(dev, cs, "F32", [cs.size]), rot)
    got = t.to_numpy().ravel()
    assert_bits_equal(got[w_:], want, "qk_rms_rope")
    # q as rms_rope leaves it, v untouched
    q_only = o.rms_rope(qkv, o.BF16, M, H, D, 3 * w_, wq, 1e-5, cs, rot)
    g3 = got.reshape(M, 3, w_)
    assert_bits_equal(g3[:, 0], q_only.reshape(M, 3, w_)[:, 0], "q")
    assert_bits_equal(g3[:, 2], qkv.reshape(M, 3, w_)[:, 2], "v")


@pytest.mark.parametrize("rot", [126, 120, 60, 96, 128])
def test_qk_rms_rope_dit_call(dev, rot):
    """The DiT's call (engine/h3-core/src/dit.rs:345-348): 56 heads of 128 in the qkv buffer of stride 3 x 7168, with
    rot_dim = 6 x the checkpoint's frequencies (dit.rs:71): 21, 20 and 10 frequencies split a 16-byte chunk."""
    M, H, D = 41, 56, 128
    w_ = H * D
    qkv = inputs(60, M * 3 * w_, o.BF16)
    wq, wk = weight(61, D), weight(62, D)
    cs = cs_table(63, M, rot)
    want = o.rms_rope(qkv, o.BF16, M, H, D, 3 * w_, wq, 1e-5, cs, rot)
    want = o.rms_rope(want[w_:], o.BF16, M, H, D, 3 * w_, wk, 1e-5, cs, rot)
    t = up(dev, qkv, "BF16", [M, 3 * w_])
    ops.qk_rms_rope(ops.Rows(t, 0, 3 * w_, M, H, D), ops.Rows(t, w_, 3 * w_, M, H, D), up(dev, wq, "F32", [D]),
                    up(dev, wk, "F32", [D]), 1e-5, up(dev, cs, "F32", [cs.size]), rot)
    got = t.to_numpy().ravel()
    assert_bits_equal(got[w_:], want, "qk_rms_rope")
    # and q alone through h3s_rms_rope, as the reference's graph calls it
    t2 = up(dev, qkv, "BF16", [M, 3 * w_])
    ops.rms_rope(ops.Rows(t2, 0, 3 * w_, M, H, D), up(dev, wq, "F32", [D]), 1e-5, up(dev, cs, "F32", [cs.size]), rot)
    q_only = o.rms_rope(qkv, o.BF16, M, H, D, 3 * w_, wq, 1e-5, cs, rot)
    assert_bits_equal(t2.to_numpy().ravel(), q_only, "rms_rope q")


# ---- h3s_norm_quant: rms_norm_mod -> bf16 h -> quantizer (configs 1, 4, 5a) ----
@pytest.mark.parametrize("rot,group", [(o.ROT_NONE, 0), (o.ROT_SYLVESTER, 128), (o.ROT_SYLVESTER, 16), (o.ROT_SYLVESTER, 512),
                                       (o.ROT_REGULAR, 256), (o.ROT_REGULAR, 64), (o.ROT_REGULAR, 16), (o.ROT_REGULAR, 4)])
@pytest.mark.parametrize("x_dt,C", [(o.BF16, 4096), (o.BF16, 5376), (o.F32, 1024), (o.BF16, 1024), (o.BF16, 16384), (o.F32, 4096),
                                    (o.F16, 2048)])
@pytest.mark.parametrize("layout", ["four", "wave"])
def test_norm_quant(request, layout, rot, group, x_dt, C):
    dev = request.getfixturevalue("dev" if layout == "four" else "dev_wave")
    if group and C % group:
        pytest.skip("group does not divide C")
    if rot == o.ROT_SYLVESTER and group > 64 * (16 // (4 if x_dt == o.F32 else 2)):
        pytest.skip("group longer than a wave's vectors")
    M = 21
    x = o.to_dt(np.random.default_rng(21).standard_normal((M, C)).astype(np.float32)
                * np.where(np.random.default_rng(22).random(C) < 0.01, 20.0, 1.0).astype(np.float32), x_dt).ravel()
    w = weight(23, C)
    want_q, want_s = o.norm_quant(x, x_dt, M, C, w, 1e-6, rot=rot, group=group, h_dt=o.BF16)
    q, s = new(dev, "I8", [M, C]), new(dev, "F32", [M])
    ops.norm_quant(up(dev, x, DTS[x_dt], [M, C]), up(dev, w, "F32", [C]), 1e-6, None, q, s, rot=rot, group=group,
                   h_dtype=DType.BF16)
    assert_bits_equal(s.to_numpy(), want_s, "scales")
    codes_close(q.to_numpy(), want_q, "codes")


@pytest.mark.parametrize("tab_dt", [o.F32, o.BF16])
@pytest.mark.parametrize("with_rows", [False, True])
@pytest.mark.parametrize("h_dt", [o.BF16, o.F32, o.F16])
@pytest.mark.parametrize("layout", ["four", "wave"])
def test_norm_quant_modulated(request, layout, tab_dt, with_rows, h_dt):
    dev = request.getfixturevalue("dev" if layout == "four" else "dev_wave")
    M, C, R = 29, 4096, 3
    x = inputs(24, M * C, o.BF16)
    w = weight(25, C)
    rows = (np.arange(M) % R).astype(np.int32) if with_rows else None
    nt = R if with_rows else 1
    sc = o.to_dt(0.5 * np.random.default_rng(26).standard_normal(nt * C).astype(np.float32), tab_dt)
    sh = o.to_dt(0.5 * np.random.default_rng(27).standard_normal(nt * C).astype(np.float32), tab_dt)
    want_q, want_s = o.norm_quant(x, o.BF16, M, C, w, 1e-6, rows, sc, sh, tab_dt, h_dt)
    q, s = new(dev, "I8", [M, C]), new(dev, "F32", [M])
    tb = ops.Tables(scale=up(dev, sc, DTS[tab_dt], [nt, C]), shift=up(dev, sh, DTS[tab_dt], [nt, C]),
                    rows=up(dev, rows, "I32", [M]) if with_rows else None)
    ops.norm_quant(up(dev, x, "BF16", [M, C]), up(dev, w, "F32", [C]), 1e-6, tb, q, s, h_dtype=DTS[h_dt])
    assert_bits_equal(s.to_numpy(), want_s, "scales")
    codes_close(q.to_numpy(), want_q, "codes")


@pytest.mark.parametrize("layout", ["four", "wave"])
def test_norm_quant_edge_rows(request, layout):
    """A zero row (scale 1e-30, codes 0), a constant row, huge and tiny rows, and a row count not a multiple of 4."""
    dev = request.getfixturevalue("dev" if layout == "four" else "dev_wave")
    M, C = 6, 4096
    x = np.random.default_rng(28).standard_normal((M, C)).astype(np.float32)
    x[0] = 0.0
    x[1] = 3.0
    x[2] *= 1e30
    x[3] *= 1e-30
    xb = o.to_bf16(x).ravel()
    w = weight(29, C)
    want_q, want_s = o.norm_quant(xb, o.BF16, M, C, w, 1e-6, h_dt=o.BF16)
    q, s = new(dev, "I8", [M, C]), new(dev, "F32", [M])
    ops.norm_quant(up(dev, xb, "BF16", [M, C]), up(dev, w, "F32", [C]), 1e-6, None, q, s)
    assert_bits_equal(s.to_numpy(), want_s, "scales")
    codes_close(q.to_numpy(), want_q, "codes")
    assert s.to_numpy()[0] == np.float32(1e-30) and not q.to_numpy()[0].any()


@pytest.mark.parametrize("pattern", ["segments", "random"])
def test_norm_quant_long_segments(dev, pattern):
    """A long input at the default settings (the one-wavefront-a-row layout), 8200 rows, with the Sylvester rotation
    of config 4. segments: three table segments, so blocks meet a segment boundary between their steps (the cached
    table row is re-decoded) and inside a step (rows that decode their own table row); random: a table row drawn per
    row, so the cached row changes at almost every step."""
    M, C = 8200, 4096
    x = inputs(30, M * C, o.BF16)
    w = weight(31, C)
    if pattern == "segments":
        rows = np.where(np.arange(M) < 1500, 0, np.where(np.arange(M) < 5000, 2, 1)).astype(np.int32)
    else:
        rows = np.random.default_rng(34).integers(0, 3, M).astype(np.int32)
    sc = o.to_dt(0.5 * np.random.default_rng(32).standard_normal(3 * C).astype(np.float32), o.BF16)
    sh = o.to_dt(0.5 * np.random.default_rng(33).standard_normal(3 * C).astype(np.float32), o.BF16)
    want_q, want_s = o.norm_quant(x, o.BF16, M, C, w, 1e-6, rows, sc, sh, o.BF16, o.BF16, rot=o.ROT_SYLVESTER, group=128)
    q, s = new(dev, "I8", [M, C]), new(dev, "F32", [M])
    tb = ops.Tables(scale=up(dev, sc, "BF16", [3, C]), shift=up(dev, sh, "BF16", [3, C]), rows=up(dev, rows, "I32", [M]))
    ops.norm_quant(up(dev, x, "BF16", [M, C]), up(dev, w, "F32", [C]), 1e-6, tb, q, s, rot=o.ROT_SYLVESTER, group=128,
                   h_dtype=DType.BF16)
    assert_bits_equal(s.to_numpy(), want_s, "scales")
    codes_close(q.to_numpy(), want_q, "codes")


def test_norm_quant_fixture_rows(dev):
    """The reference fixture's 2,159-token layout: the table rows of its first step (text, audio and video segments,
    tests/golden/layout_384x288_2s.json), float32 tables of the AdaLN's shape [rows, C]."""
    import json
    import os

    gold = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "layout_384x288_2s.json")))
    rows = np.concatenate([np.full(n, r, np.int32) for r, n in gold["mod_rows_rle"]])
    M, C = rows.size, 4096
    R = int(rows.max()) + 1
    x = inputs(64, M * C, o.BF16)
    w = weight(65, C)
    sc = (0.5 * np.random.default_rng(66).standard_normal(R * C)).astype(np.float32)
    sh = (0.5 * np.random.default_rng(67).standard_normal(R * C)).astype(np.float32)
    want_q, want_s = o.norm_quant(x, o.BF16, M, C, w, 1e-6, rows, sc, sh, o.F32, o.BF16)
    q, s = new(dev, "I8", [M, C]), new(dev, "F32", [M])
    tb = ops.Tables(scale=up(dev, sc, "F32", [R, C]), shift=up(dev, sh, "F32", [R, C]), rows=up(dev, rows, "I32", [M]))
    ops.norm_quant(up(dev, x, "BF16", [M, C]), up(dev, w, "F32", [C]), 1e-6, tb, q, s, h_dtype=DType.BF16)
    assert_bits_equal(s.to_numpy(), want_s, "scales")
    codes_close(q.to_numpy(), want_q, "codes")


@pytest.mark.parametrize("rot,group", [(o.ROT_NONE, 0), (o.ROT_REGULAR, 256)])
def test_norm_quant_units_of_many_rows(dev, rot, group):
    """The real model's width (5376) at 16896 tokens with three table segments: every unit of the persistent
    quantizer takes many rows, prefetching the next row and reloading the table row at the segment boundaries."""
    M, C = 16896, 5376
    rows = np.where(np.arange(M) < 137, 1, np.where(np.arange(M) < 323, 2, 0)).astype(np.int32)
    x = inputs(68, M * C, o.BF16)
    w = weight(69, C)
    sc = o.to_dt(0.5 * np.random.default_rng(70).standard_normal(3 * C).astype(np.float32), o.BF16)
    sh = o.to_dt(0.5 * np.random.default_rng(71).standard_normal(3 * C).astype(np.float32), o.BF16)
    want_q, want_s = o.norm_quant(x, o.BF16, M, C, w, 1e-6, rows, sc, sh, o.BF16, o.BF16, rot=rot, group=group)
    q, s = new(dev, "I8", [M, C]), new(dev, "F32", [M])
    tb = ops.Tables(scale=up(dev, sc, "BF16", [3, C]), shift=up(dev, sh, "BF16", [3, C]), rows=up(dev, rows, "I32", [M]))
    ops.norm_quant(up(dev, x, "BF16", [M, C]), up(dev, w, "F32", [C]), 1e-6, tb, q, s, rot=rot, group=group,
                   h_dtype=DType.BF16)
    assert_bits_equal(s.to_numpy(), want_s, "scales")
    codes_close(q.to_numpy(), want_q, "codes")


def sample_rows(M, band=256):
    """one row from every band of rows (at an offset that moves from band to band), and the last row"""
    r = [b * band + (b * 37) % band for b in range((M + band - 1) // band)]
    return np.unique(np.minimum(np.array(r + [M - 1]), M - 1))


def read_rows(t, rows, width, esize):
    """rows of a [M, width] device tensor, read one at a time"""
    return np.stack([t._owner.read(width * esize, (t.ptr() - t._owner.ptr()) + int(r) * width * esize) for r in rows])


@pytest.mark.parametrize("config", ["4", "5a"])
def test_norm_quant_full_size(dev, config):
    """Configs 4 and 5a at their full size (47104 x 4096, the one-wavefront-a-row layout): every row's largest code is
    127 in magnitude, and sampled rows (one from every 256-row band, and the last) equal the oracle's bit for bit."""
    M, C = 47104, 4096
    rng = np.random.default_rng(72)
    heavy = np.where(rng.random(C) < 0.01, 20.0, 1.0).astype(np.float32) if config == "4" else np.ones(C, np.float32)
    x = o.to_bf16(rng.standard_normal((M, C), dtype=np.float32) * heavy)
    w = weight(73, C)
    if config == "4":
        tb, sc, sh, rot, group = None, None, None, o.ROT_SYLVESTER, 128
    else:
        sc = o.to_bf16((0.5 * rng.standard_normal(C)).astype(np.float32))
        sh = o.to_bf16((0.5 * rng.standard_normal(C)).astype(np.float32))
        tb, rot, group = ops.Tables(scale=up(dev, sc, "BF16", [1, C]), shift=up(dev, sh, "BF16", [1, C])), o.ROT_NONE, 0
    q, s = new(dev, "I8", [M, C]), new(dev, "F32", [M])
    ops.norm_quant(up(dev, x, "BF16", [M, C]), up(dev, w, "F32", [C]), 1e-6, tb, q, s, rot=rot, group=group,
                   h_dtype=DType.BF16)
    gq = q.to_numpy().reshape(M, C)
    assert np.all(np.abs(gq.astype(np.int32)).max(1) == 127)
    rows = sample_rows(M)
    xs = np.ascontiguousarray(x.reshape(M, C)[rows])
    want_q, want_s = o.norm_quant(xs.ravel(), o.BF16, rows.size, C, w, 1e-6, None, sc, sh, o.BF16, o.BF16, rot=rot,
                                  group=group)
    assert_bits_equal(s.to_numpy()[rows], want_s, "scales")
    codes_close(gq[rows], want_q, "codes")


@pytest.mark.parametrize("config", ["4", "5a"])
@pytest.mark.parametrize("M", [100, 96, 8])
def test_norm_quant_tail_rows(config, M):
    """Configs 4 and 5a end their launch with a last round at most a quarter full four wavefronts a row: on a
    context that sizes its grids for 2 compute units (H3S_CUS=2) the one-wavefront layout takes M = 100 rows as 96
    in whole rounds and 4 in the tail form (96: whole rounds only; 8: less than a round, one form), each bit for bit
    the oracle's."""
    import os
    from sycl_minimax_h3_amd import Device

    old = {k: os.environ.get(k) for k in ("H3S_CUS", "H3S_QUANT_WAVE_MIN_ROWS")}
    os.environ.update({"H3S_CUS": "2", "H3S_QUANT_WAVE_MIN_ROWS": "0"})
    try:
        dev = Device.open()
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v
    try:
        C = 4096
        rng = np.random.default_rng(74 + M)
        heavy = np.where(rng.random(C) < 0.01, 20.0, 1.0).astype(np.float32) if config == "4" else np.ones(C, np.float32)
        x = o.to_bf16(rng.standard_normal((M, C), dtype=np.float32) * heavy).ravel()
        w = weight(75, C)
        if config == "4":
            tb, sc, sh, rot, group = None, None, None, o.ROT_SYLVESTER, 128
        else:
            sc = o.to_bf16((0.5 * rng.standard_normal(C)).astype(np.float32))
            sh = o.to_bf16((0.5 * rng.standard_normal(C)).astype(np.float32))
            tb, rot, group = ops.Tables(scale=up(dev, sc, "BF16", [1, C]), shift=up(dev, sh, "BF16", [1, C])), o.ROT_NONE, 0
        q, s = new(dev, "I8", [M, C]), new(dev, "F32", [M])
        ops.norm_quant(up(dev, x, "BF16", [M, C]), up(dev, w, "F32", [C]), 1e-6, tb, q, s, rot=rot, group=group,
                       h_dtype=DType.BF16)
        want_q, want_s = o.norm_quant(x, o.BF16, M, C, w, 1e-6, None, sc, sh, o.BF16, o.BF16, rot=rot, group=group)
        assert_bits_equal(s.to_numpy(), want_s, "scales")
        codes_close(q.to_numpy(), want_q, "codes")
    finally:
        dev.close()


# ---- h3s_swiglu_quant: swiglu -> the MLP's act scratch -> fc2's quantizer, in one pass ----
@pytest.mark.parametrize("rot,group", [(o.ROT_NONE, 0), (o.ROT_REGULAR, 256), (o.ROT_REGULAR, 16), (o.ROT_SYLVESTER, 128)])
@pytest.mark.parametrize("x_dt,h_dt", [(o.BF16, o.BF16), (o.F16, o.F16), (o.F32, o.F32), (o.F32, o.BF16), (o.BF16, o.F32)])
@pytest.mark.parametrize("M,C", [(23, 2048), (7, 4096), (6, 8192), (3, 16384), (11, 1792), (5, 64), (9, 528)])
def test_swiglu_quant(dev, rot, group, x_dt, h_dt, M, C):
    if group and C % group:
        pytest.skip("group does not divide C")
    if C % (16 // (4 if x_dt == o.F32 else 2)) or too_long(C, x_dt):
        pytest.skip("not whole vectors, or a row longer than the kernels take")
    x = inputs(40, M * 2 * C, x_dt, 3.0)
    xt = up(dev, x, DTS[x_dt], [M, 2 * C])
    q, s = new(dev, "I8", [M, C]), new(dev, "F32", [M])
    ops.swiglu_quant(xt, q, s, rot=rot, group=group, h_dtype=DTS[h_dt])
    gq, gs = q.to_numpy().ravel(), s.to_numpy()
    # bit for bit: the library's own swiglu into act, then the oracle's quantizer on those bits
    act = new(dev, DTS[h_dt], [M, C])
    ops.swiglu(xt, act)
    want_q, want_s = o.quantize_act(act.to_numpy().ravel(), h_dt, M, C, rot, group)
    assert_bits_equal(gs, want_s, "scales")
    codes_close(gq, want_q, "codes")
    # against the oracle's whole chain (its expf and division): the parity tolerance
    oq, os_ = o.swiglu_quant(x, x_dt, M, C, h_dt, rot, group)
    rel, _ = o.compare(gs, os_)
    assert rel < 1e-3 and np.all(np.abs(gs / os_ - 1) <= 2.0 ** -7), "scales"
    d = np.abs(gq.astype(np.int32) - oq.astype(np.int32))
    assert d.max() <= 1 and (d > 0).mean() <= 1e-2, f"codes: {(d > 0).mean():.2e} differ by 1"


# ---- h3s_norm_mod_act_gate (config 2's chain) ----
@pytest.mark.parametrize("norm", [o.NORM_LAYER, o.NORM_RMS])
@pytest.mark.parametrize("act", [o.ACT_GELU_TANH, o.ACT_SILU, o.ACT_NONE])
@pytest.mark.parametrize("tab_dt", [o.BF16, o.F32])
@pytest.mark.parametrize("M,C", [(40, 4096), (9, 1024), (5, 16384)])
def test_norm_mod_act_gate(dev, norm, act, tab_dt, M, C):
    x = inputs(30, M * C, o.BF16)
    res = inputs(31, M * C, o.BF16)
    tabs = [o.to_dt(0.5 * np.random.default_rng(32 + i).standard_normal(C).astype(np.float32), tab_dt) for i in range(3)]
    w = weight(35, C) if norm == o.NORM_RMS else None
    want = o.norm_mod_act_gate(x, o.BF16, M, C, norm, w, None, 1e-5, None, tabs[0], tabs[1], tabs[2], tab_dt, act, res,
                               o.BF16, o.BF16)
    out = new(dev, "BF16", [M, C])
    tb = ops.Tables(scale=up(dev, tabs[0], DTS[tab_dt], [1, C]), shift=up(dev, tabs[1], DTS[tab_dt], [1, C]),
                    gate=up(dev, tabs[2], DTS[tab_dt], [1, C]))
    ops.norm_mod_act_gate(up(dev, x, "BF16", [M, C]), norm, up(dev, w, "F32", [C]) if w is not None else None, None, 1e-5, tb,
                          act, up(dev, res, "BF16", [M, C]), out)
    if act == o.ACT_NONE:
        assert_bits_equal(out.to_numpy(), want, "norm_mod_act_gate")
    else:
        assert_close_16(out.to_numpy(), want, o.BF16, "norm_mod_act_gate", max_frac=5e-3)


def test_norm_mod_act_gate_float32_and_affine(dev):
    """float32 rows, residual, tables and output, with an affine layer norm and per-token table rows."""
    M, C, R = 13, 2048, 3
    rng = np.random.default_rng(36)
    x = (rng.standard_normal(M * C) * 2 + 0.5).astype(np.float32)
    res = rng.standard_normal(M * C).astype(np.float32)
    w, b = weight(37, C), (0.1 * rng.standard_normal(C)).astype(np.float32)
    rows = (np.arange(M) % R).astype(np.int32)
    tabs = [(0.5 * rng.standard_normal(R * C)).astype(np.float32) for _ in range(3)]
    want = o.norm_mod_act_gate(x, o.F32, M, C, o.NORM_LAYER, w, b, 1e-5, rows, tabs[0], tabs[1], tabs[2], o.F32,
                               o.ACT_NONE, res, o.F32, o.F32)
    out = new(dev, "F32", [M, C])
    tb = ops.Tables(scale=up(dev, tabs[0], "F32", [R, C]), shift=up(dev, tabs[1], "F32", [R, C]),
                    gate=up(dev, tabs[2], "F32", [R, C]), rows=up(dev, rows, "I32", [M]))
    ops.norm_mod_act_gate(up(dev, x, "F32", [M, C]), o.NORM_LAYER, up(dev, w, "F32", [C]), up(dev, b, "F32", [C]), 1e-5, tb,
                          o.ACT_NONE, up(dev, res, "F32", [M, C]), out)
    assert_bits_equal(out.to_numpy(), want, "norm_mod_act_gate f32")


def segment_rows(seed, M, R):
    """table rows in runs of 1 to 9 rows: many runs change between the two rows of a block of two"""
    lens = np.random.default_rng(seed).integers(1, 10, M)
    return np.repeat(np.arange(M) % R, lens)[:M].astype(np.int32)


@pytest.mark.parametrize("M", [5001, 4401, 5201])
@pytest.mark.parametrize("C", [2048, 4096])
@pytest.mark.parametrize("kind", ["ada_ln_gelu", "ada_rms_silu", "ada_ln", "rms_mod_f32", "layer_norm_affine"])
def test_chain_two_rows_a_block(dev, kind, C, M):
    """Enough rows (an odd count) that rows of 256 lanes go two to a block: the weights and table rows are loaded
    once for both, and reloaded for the second row where its table row differs; the last block's second row is
    past the end. Where the pairs leave a last round of the resident blocks at most half full, the launch ends with
    one-row blocks instead: 4401 rows (2201 pairs) do so for rounds of 1536 to 2048 blocks, 5201 rows for 1280,
    1792 and 2048, 5001 rows for 1792 and 2048 (and take two-row blocks to the end for 1280 and 1536)."""
    R = 5                   # at least 16 rows a compute unit of the 256
    x = inputs(40, M * C, o.BF16, 2.0)
    res = inputs(41, M * C, o.BF16)
    rows = segment_rows(42, M, R)
    assert np.count_nonzero(rows[1::2] != rows[0:-1:2]) > M // 10
    out = new(dev, "BF16", [M, C])
    xt = up(dev, x, "BF16", [M, C])
    if kind.startswith("ada"):
        norm = o.NORM_LAYER if "_ln" in kind else o.NORM_RMS
        act = o.ACT_GELU_TANH if "gelu" in kind else o.ACT_SILU if "silu" in kind else o.ACT_NONE
        tabs = [o.to_dt(0.5 * np.random.default_rng(43 + i).standard_normal(R * C).astype(np.float32), o.BF16)
                for i in range(3)]
        w = weight(46, C) if norm == o.NORM_RMS else None
        want = o.norm_mod_act_gate(x, o.BF16, M, C, norm, w, None, 1e-5, rows, tabs[0], tabs[1], tabs[2], o.BF16, act,
                                   res, o.BF16, o.BF16)
        tb = ops.Tables(scale=up(dev, tabs[0], "BF16", [R, C]), shift=up(dev, tabs[1], "BF16", [R, C]),
                        gate=up(dev, tabs[2], "BF16", [R, C]), rows=up(dev, rows, "I32", [M]))
        ops.norm_mod_act_gate(xt, norm, up(dev, w, "F32", [C]) if w is not None else None, None, 1e-5, tb, act,
                              up(dev, res, "BF16", [M, C]), out)
        if act == o.ACT_NONE:
            assert_bits_equal(out.to_numpy(), want, kind)
        else:
            assert_close_16(out.to_numpy(), want, o.BF16, kind, max_frac=5e-3)
    elif kind == "rms_mod_f32":
        w = weight(47, C)
        sc = (0.5 * np.random.default_rng(48).standard_normal((R, C))).astype(np.float32)
        sh = (0.5 * np.random.default_rng(49).standard_normal((R, C))).astype(np.float32)
        want = o.rms_norm_mod(x, o.BF16, M, C, w, 1e-6, rows, sc, sh, o.BF16)
        m = ops.Mod(up(dev, rows, "I32", [M]), up(dev, sc, "F32", [R, C]), up(dev, sh, "F32", [R, C]))
        ops.rms_norm_mod(xt, up(dev, w, "F32", [C]), 1e-6, m, out)
        assert_bits_equal(out.to_numpy(), want, kind)
    else:
        w, b = weight(50, C), (0.1 * np.random.default_rng(51).standard_normal(C)).astype(np.float32)
        want = o.layer_norm(x, o.BF16, M, C, w, b, 1e-5, o.BF16)
        ops.layer_norm(xt, C, up(dev, w, "F32", [C]), up(dev, b, "F32", [C]), 1e-5, out)
        assert_bits_equal(out.to_numpy(), want, kind)


# ---- h3s_int8_linear and h3s_int8_gemm_dequant (kernels/h3sycl.cpp:404-652) ----
@pytest.mark.parametrize("M,K,N", [(1, 64, 5), (300, 256, 300), (257, 4096, 129), (64, 1024, 512), (33, 320, 70)])
@pytest.mark.parametrize("group", [0, 4, 16, 64, 256])
@pytest.mark.parametrize("per_n,bias,out_dt", [(False, False, o.BF16), (True, True, o.BF16), (True, False, o.F32)])
@pytest.mark.parametrize("layout", ["four", "wave"])
def test_int8_linear(request, layout, M, K, N, group, per_n, bias, out_dt):
    dev = request.getfixturevalue("dev" if layout == "four" else "dev_wave")
    if group and K % group:
        pytest.skip("group does not divide K")
    rng = np.random.default_rng(M * 7 + K + N + group)
    x = o.to_bf16((0.7 * rng.standard_normal(M * K)).astype(np.float32))
    w = rng.integers(-127, 128, N * K, dtype=np.int8)
    ws = rng.uniform(0.005, 0.02, N if per_n else 1).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    want = o.int8_linear(x, o.BF16, M, K, w, N, ws, b, out_dt, group)
    layer = ops.Int8Linear(up(dev, w, "I8", [N, K]), up(dev, ws, "F32", [ws.size]), up(dev, b, "F32", [N]) if bias else None,
                           group or None)
    out = new(dev, DTS[out_dt], [M, N])
    layer.forward(up(dev, x, "BF16", [M, K]), out)
    assert_bits_equal(out.to_numpy(), want, "int8_linear")


@pytest.mark.parametrize("act", [o.ACT_NONE, o.ACT_SILU])
@pytest.mark.parametrize("K", [4096, 320, 192])   # whole 128-byte K steps, and a last step of 64
def test_int8_gemm_dequant(dev, act, K):
    M, N = 515, 770
    rng = np.random.default_rng(40)
    q = rng.integers(-128, 128, M * K, dtype=np.int8)
    s = rng.uniform(0.001, 0.05, M).astype(np.float32)
    w = rng.integers(-127, 128, N * K, dtype=np.int8)
    ws = rng.uniform(0.005, 0.02, N).astype(np.float32)
    want = o.gemm_dequant(q, s, M, K, w, N, ws, None, act, o.BF16)
    layer = ops.Int8Linear(up(dev, w, "I8", [N, K]), up(dev, ws, "F32", [N]))
    out = new(dev, "BF16", [M, N])
    ops.int8_gemm_dequant(up(dev, q, "I8", [M, K]), up(dev, s, "F32", [M]), layer, act, out)
    if act == o.ACT_NONE:
        assert_bits_equal(out.to_numpy(), want, "gemm")
    else:
        assert_close_16(out.to_numpy(), want, o.BF16, "gemm silu", max_frac=5e-3)


@pytest.mark.parametrize("act", [o.ACT_NONE, o.ACT_SILU])
@pytest.mark.parametrize("M,N,K", [(2560, 1024, 4096), (2716, 776, 4096), (1297, 763, 12288)])
def test_int8_gemm_tile_order(dev_cus16, act, M, N, K):
    """Grids of more than 8 tile rows, renumbered across the XCDs in groups of 8 tile rows as at config 5b's size:
    10 x 4 tiles (a multiple of 8), and 11 x 4 = 44 (not one: the first four XCDs take one tile more), with a
    partial last tile row and column; and K = 12288, whose groups are 4 tile rows high (6 x 3 tiles: a full group and
    a partial one). On a context sized for 16 CUs, so that the tiles run whole (on the whole device, so few tiles
    would split along K), the 18 tiles at K = 12288 as 16 whole and 2 in parts."""
    dev = dev_cus16
    rng = np.random.default_rng(74)
    q = rng.integers(-128, 128, M * K, dtype=np.int8)
    s = rng.uniform(0.001, 0.05, M).astype(np.float32)
    w = rng.integers(-127, 128, N * K, dtype=np.int8)
    ws = rng.uniform(0.005, 0.02, N).astype(np.float32)
    want = o.gemm_dequant(q, s, M, K, w, N, ws, None, act, o.BF16)
    layer = ops.Int8Linear(up(dev, w, "I8", [N, K]), up(dev, ws, "F32", [N]))
    out = new(dev, "BF16", [M, N])
    ops.int8_gemm_dequant(up(dev, q, "I8", [M, K]), up(dev, s, "F32", [M]), layer, act, out)
    if act == o.ACT_NONE:
        assert_bits_equal(out.to_numpy(), want, "gemm")
    else:
        assert_close_16(out.to_numpy(), want, o.BF16, "gemm silu", max_frac=5e-3)


def test_int8_gemm_full_size(dev):
    """Config 5b at its full size, 47104 x 16384 x 4096 with the SiLU epilogue: one row from every 256-row tile band
    (and the last row), all 16384 columns, against the oracle."""
    M, N, K = 47104, 16384, 4096
    rng = np.random.default_rng(75)
    q = rng.integers(-127, 128, (M, K), dtype=np.int8)
    s = rng.uniform(0.001, 0.05, M).astype(np.float32)
    w = rng.integers(-127, 128, N * K, dtype=np.int8)
    ws = rng.uniform(0.005, 0.02, N).astype(np.float32)
    layer = ops.Int8Linear(up(dev, w, "I8", [N, K]), up(dev, ws, "F32", [N]))
    out = new(dev, "BF16", [M, N])
    ops.int8_gemm_dequant(up(dev, q, "I8", [M, K]), up(dev, s, "F32", [M]), layer, o.ACT_SILU, out)
    rows = sample_rows(M)
    got = read_rows(out, rows, N, 2).view(np.uint16)
    want = o.gemm_dequant(np.ascontiguousarray(q[rows]).ravel(), np.ascontiguousarray(s[rows]), rows.size, K, w, N, ws,
                          None, o.ACT_SILU, o.BF16)
    assert_close_16(got, want, o.BF16, "gemm silu full size", max_frac=5e-3)


# ---- errors through the ABI on the device ----
def test_errors_are_reported(dev):
    M, C = 4, 4096
    xt = new(dev, "BF16", [M, C])
    q, s = new(dev, "I8", [M, C]), new(dev, "F32", [M])
    with pytest.raises(Error, match="aligned"):
        dev.check(dev.api.norm_quant(dev.ctx, xt.ptr() + 2, 2, M, C - 8, None, 1e-6, None, None, None, 0, 2, 0, 0, q.ptr(), s.ptr()))
    with pytest.raises(Error, match="group"):
        dev.check(dev.api.int8_linear(dev.ctx, xt.ptr(), 2, M, C, q.ptr(), 8, s.ptr(), 1, None, xt.ptr(), 2, 128))
    with pytest.raises(Error, match="rot_dim"):
        dev.check(dev.api.rms_rope(dev.ctx, xt.ptr(), 2, M, 32, 128, 4096, s.ptr(), 1e-5, s.ptr(), 127))
    with pytest.raises(Error, match="not implemented"):
        dev.check(dev.api.conv3d(dev.ctx, xt.ptr(), 2, 1, 1, 1, 8, xt.ptr(), 8, 3, None, xt.ptr()))
    assert dev.api.rms_norm_mod(dev.ctx, xt.ptr(), 2, 0, C, s.ptr(), 1e-6, None, None, None, xt.ptr(), 2) == 0
    dev.wait()
