"""GPU parity at the widths of the reference's model (docs/BASELINE.md:13: hidden 5376, 56 heads of 128, an MLP of
5376 -> 2 x 14336 -> 5376; rot_dim 6 x 21 = 126, engine/h3-core/src/dit.rs:71), through the calls the unchanged
graph makes (dit.rs:329-369) and the fused pairs that replace two of them, against the CPU oracle on the same
seeded inputs. Bit-exact: codes, scales, norms, rotations and the GEMM without activation."""
import numpy as np
import pytest

from oracle import oracle as o
from helpers import assert_bits_equal, codes_close, new, up

pytestmark = pytest.mark.gpu

from sycl_minimax_h3_amd import DType, ops  # noqa: E402

o.set_threads(8)
DH, DHEADS, DHD, DFF = 5376, 56, 128, 14336


def bf16_rows(seed, M, C, scale=1.0, heavy=True):
    """[M, C] bfloat16 bit patterns drawn directly (fast at tens of millions of values): random sign and 7-bit
    mantissa, magnitudes log-uniform over [2^-9, 2^2) x scale's power of two, and with `heavy` 1 % of the channels
    x16 (the outlier channels a rotation spreads)"""
    rng = np.random.default_rng(seed)
    shift = int(np.floor(np.log2(scale)))
    e = rng.integers(118 + shift, 129 + shift, size=(M, C), dtype=np.uint16)
    if heavy:
        e += np.where(rng.random(C) < 0.01, 4, 0).astype(np.uint16)[None, :]
    bits = (rng.integers(0, 2, size=(M, C), dtype=np.uint16) << np.uint16(15)) | (e << np.uint16(7)) | \
        rng.integers(0, 128, size=(M, C), dtype=np.uint16)
    return bits.ravel()


def dit_rows(M):
    """the reference harness's row table: the first 5 % of the tokens on table row 1 (engine/h3d/src/jobs.rs:213)"""
    r = np.zeros(M, dtype=np.int32)
    r[: M // 20] = 1
    return r


# ---- h3s_int8_linear at the block's four (K, N) shapes, group 256, one scale per output (dit.rs:341-364) ----
@pytest.mark.parametrize("K", [DH, DHEADS * DHD, DFF])
@pytest.mark.parametrize("M,N,per_n,bias,out_dt", [(37, 192, True, False, o.BF16), (300, 96, True, True, o.BF16),
                                                   (9, 130, False, False, o.F32)])
@pytest.mark.parametrize("layout", ["four", "wave"])
def test_int8_linear_dit_widths(request, layout, K, M, N, per_n, bias, out_dt):
    dev = request.getfixturevalue("dev" if layout == "four" else "dev_wave")
    rng = np.random.default_rng(K + M + N)
    x = bf16_rows(K + M, M, K, 0.7)
    w = rng.integers(-127, 128, N * K, dtype=np.int8)
    ws = rng.uniform(0.005, 0.02, N if per_n else 1).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    want = o.int8_linear(x, o.BF16, M, K, w, N, ws, b, out_dt, 256)
    layer = ops.Int8Linear(up(dev, w, "I8", [N, K]), up(dev, ws, "F32", [ws.size]), up(dev, b, "F32", [N]) if bias else None, 256)
    out = new(dev, {o.BF16: DType.BF16, o.F32: DType.F32}[out_dt], [M, N])
    layer.forward(up(dev, x, "BF16", [M, K]), out)
    assert_bits_equal(out.to_numpy(), want, f"int8_linear K={K}")


# ---- the int8 linear's quantizer on its own (h3s_int8_quantize), at the three input widths and many rows ----
@pytest.mark.parametrize("K", [DH, DHEADS * DHD, DFF])
@pytest.mark.parametrize("group", [256, 0])
@pytest.mark.parametrize("layout", ["four", "wave"])
def test_int8_quantize_dit_widths(request, layout, K, group):
    dev = request.getfixturevalue("dev" if layout == "four" else "dev_wave")
    M = 8200 if K == DH else 2100                  # past the one-wavefront form's row threshold at the hidden width
    x = bf16_rows(K + group, M, K)
    want_q, want_s = o.quantize_act(x, o.BF16, M, K, o.ROT_REGULAR if group else o.ROT_NONE, group)
    q, s = new(dev, "I8", [M, K]), new(dev, "F32", [M])
    ops.int8_quantize(up(dev, x, "BF16", [M, K]), q, s, group)
    assert_bits_equal(s.to_numpy(), want_s, "scales")
    codes_close(q.to_numpy(), want_q, "codes")


# ---- the two-chunks-a-lane (16 features) layout of the regular-256 rotation at the other widths it serves ----
@pytest.mark.parametrize("layout", ["four", "wave"])
def test_int8_quantize_4096_pairs(request, layout):
    dev = request.getfixturevalue("dev" if layout == "four" else "dev_wave")
    M, K = 1025, 4096
    x = bf16_rows(90, M, K)
    want_q, want_s = o.quantize_act(x, o.BF16, M, K, o.ROT_REGULAR, 256)
    q, s = new(dev, "I8", [M, K]), new(dev, "F32", [M])
    ops.int8_quantize(up(dev, x, "BF16", [M, K]), q, s, 256)
    assert_bits_equal(s.to_numpy(), want_s, "scales")
    codes_close(q.to_numpy(), want_q, "codes")


@pytest.mark.parametrize("layout", ["four", "wave"])
def test_swiglu_quant_8192_pairs(request, layout):
    dev = request.getfixturevalue("dev" if layout == "four" else "dev_wave")
    M, C = 301, 8192
    x = bf16_rows(91, M, 2 * C, 4.0, heavy=False)
    xt = up(dev, x, "BF16", [M, 2 * C])
    q, s = new(dev, "I8", [M, C]), new(dev, "F32", [M])
    ops.swiglu_quant(xt, q, s, rot=o.ROT_REGULAR, group=256)
    act = new(dev, "BF16", [M, C])
    ops.swiglu(xt, act)
    want_q, want_s = o.quantize_act(act.to_numpy().ravel(), o.BF16, M, C, o.ROT_REGULAR, 256)
    assert_bits_equal(s.to_numpy(), want_s, "scales")
    codes_close(q.to_numpy(), want_q, "codes")


# ---- h3s_swiglu_quant at fc2's width: 14336 features, 1792 16-byte chunks a row ----
@pytest.mark.parametrize("M,rot,group", [(9, o.ROT_REGULAR, 256), (2500, o.ROT_REGULAR, 256), (33, o.ROT_NONE, 0)])
@pytest.mark.parametrize("layout", ["four", "wave"])
def test_swiglu_quant_fc2_width(request, layout, M, rot, group):
    dev = request.getfixturevalue("dev" if layout == "four" else "dev_wave")
    C = DFF
    x = bf16_rows(M + 41, M, 2 * C, 4.0, heavy=False)
    xt = up(dev, x, "BF16", [M, 2 * C])
    q, s = new(dev, "I8", [M, C]), new(dev, "F32", [M])
    ops.swiglu_quant(xt, q, s, rot=rot, group=group)
    # bit for bit: the library's own swiglu into act, then the oracle's quantizer on those bits
    act = new(dev, "BF16", [M, C])
    ops.swiglu(xt, act)
    want_q, want_s = o.quantize_act(act.to_numpy().ravel(), o.BF16, M, C, rot, group)
    assert_bits_equal(s.to_numpy(), want_s, "scales")
    codes_close(q.to_numpy(), want_q, "codes")
    # and the two-call path the graph takes: h3s_swiglu then h3s_int8_quantize on act
    q2, s2 = new(dev, "I8", [M, C]), new(dev, "F32", [M])
    if rot == o.ROT_REGULAR:
        ops.int8_quantize(act, q2, s2, group)
        assert_bits_equal(s2.to_numpy(), want_s, "two-call scales")
        codes_close(q2.to_numpy(), want_q, "two-call codes")


# ---- the regular-256 quantizers leave the rotated values unscaled (fl(1/sqrt(256)) = 2^-4) and fold the power of
# two into the codes' divisor, except in rows whose unscaled maximum is below 2^-60: rows of every magnitude from 1
# down to 2^-115 and zero rows, on both sides of that threshold, bit for bit against the oracle's scaled arithmetic ----
def tiny_rows(seed, C, heavy=True):
    shifts = [0, -50, -56, -58, -60, -62, -64, -66, -68, -70, -80, -100, -115]
    blocks = [bf16_rows(seed + i, 8, C, 2.0 ** k, heavy=heavy) for i, k in enumerate(shifts)]
    blocks.append(np.zeros(4 * C, dtype=np.uint16))
    return np.concatenate(blocks), 8 * len(shifts) + 4


@pytest.mark.parametrize("K", [DH, DHEADS * DHD, DFF, 4096])
@pytest.mark.parametrize("layout", ["four", "wave"])
def test_int8_quantize_tiny_rows(request, layout, K):
    dev = request.getfixturevalue("dev" if layout == "four" else "dev_wave")
    x, M = tiny_rows(K, K)
    want_q, want_s = o.quantize_act(x, o.BF16, M, K, o.ROT_REGULAR, 256)
    q, s = new(dev, "I8", [M, K]), new(dev, "F32", [M])
    ops.int8_quantize(up(dev, x, "BF16", [M, K]), q, s, 256)
    assert_bits_equal(s.to_numpy(), want_s, "scales")
    codes_close(q.to_numpy(), want_q, "codes")


@pytest.mark.parametrize("C", [DFF, 8192])
@pytest.mark.parametrize("layout", ["four", "wave"])
def test_swiglu_quant_tiny_rows(request, layout, C):
    dev = request.getfixturevalue("dev" if layout == "four" else "dev_wave")
    x, M = tiny_rows(C + 7, 2 * C, heavy=False)
    xt = up(dev, x, "BF16", [M, 2 * C])
    q, s = new(dev, "I8", [M, C]), new(dev, "F32", [M])
    ops.swiglu_quant(xt, q, s, rot=o.ROT_REGULAR, group=256)
    act = new(dev, "BF16", [M, C])
    ops.swiglu(xt, act)
    want_q, want_s = o.quantize_act(act.to_numpy().ravel(), o.BF16, M, C, o.ROT_REGULAR, 256)
    assert_bits_equal(s.to_numpy(), want_s, "scales")
    codes_close(q.to_numpy(), want_q, "codes")


@pytest.mark.parametrize("layout", ["four", "wave"])
def test_norm_quant_tiny_weight(request, layout):
    """the norm's rows are O(|w|) whatever x is: weights of 2^-62 .. 2^-75 put the rotated rows on both sides of the
    threshold"""
    dev = request.getfixturevalue("dev" if layout == "four" else "dev_wave")
    M, C = 96, DH
    x = bf16_rows(53, M, C)
    rng = np.random.default_rng(54)
    for k in (-62, -66, -70, -75):
        w = (2.0 ** k * (1.0 + 0.1 * rng.standard_normal(C))).astype(np.float32)
        sc = (0.3 * rng.standard_normal(2 * C)).astype(np.float32) * np.float32(2.0 ** k)
        sh = (0.3 * rng.standard_normal(2 * C)).astype(np.float32) * np.float32(2.0 ** k)
        rows = dit_rows(M)
        want_q, want_s = o.norm_quant(x, o.BF16, M, C, w, 1e-5, rows, sc, sh, o.F32, o.BF16, o.ROT_REGULAR, 256)
        q, s = new(dev, "I8", [M, C]), new(dev, "F32", [M])
        tb = ops.Tables(scale=up(dev, sc, "F32", [2, C]), shift=up(dev, sh, "F32", [2, C]), rows=up(dev, rows, "I32", [M]))
        ops.norm_quant(up(dev, x, "BF16", [M, C]), up(dev, w, "F32", [C]), 1e-5, tb, q, s, rot=o.ROT_REGULAR, group=256)
        assert_bits_equal(s.to_numpy(), want_s, f"scales (w ~ 2^{k})")
        codes_close(q.to_numpy(), want_q, f"codes (w ~ 2^{k})")


# ---- h3s_norm_quant at the hidden width with float32 tables and a row table, 16896 rows ----
@pytest.mark.parametrize("rot,group", [(o.ROT_REGULAR, 256), (o.ROT_NONE, 0)])
@pytest.mark.parametrize("layout", ["four", "wave"])
def test_norm_quant_dit_width(request, layout, rot, group):
    dev = request.getfixturevalue("dev" if layout == "four" else "dev_wave")
    M, C = 16896, DH
    x = bf16_rows(51, M, C)
    rng = np.random.default_rng(52)
    w = (1.0 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    sc = (0.3 * rng.standard_normal(2 * C)).astype(np.float32)
    sh = (0.3 * rng.standard_normal(2 * C)).astype(np.float32)
    rows = dit_rows(M)
    want_q, want_s = o.norm_quant(x, o.BF16, M, C, w, 1e-5, rows, sc, sh, o.F32, o.BF16, rot, group)
    q, s = new(dev, "I8", [M, C]), new(dev, "F32", [M])
    tb = ops.Tables(scale=up(dev, sc, "F32", [2, C]), shift=up(dev, sh, "F32", [2, C]), rows=up(dev, rows, "I32", [M]))
    ops.norm_quant(up(dev, x, "BF16", [M, C]), up(dev, w, "F32", [C]), 1e-5, tb, q, s, rot=rot, group=group)
    assert_bits_equal(s.to_numpy(), want_s, "scales")
    codes_close(q.to_numpy(), want_q, "codes")
    # the graph's two calls: rms_norm_mod into the bf16 scratch h, then the int8 linear's quantizer on h
    if rot == o.ROT_REGULAR:
        h = new(dev, "BF16", [M, C])
        ops.rms_norm_mod(up(dev, x, "BF16", [M, C]), up(dev, w, "F32", [C]), 1e-5,
                         ops.Mod(up(dev, rows, "I32", [M]), up(dev, sc, "F32", [2, C]), up(dev, sh, "F32", [2, C])), h)
        want_h = o.rms_norm_mod(x, o.BF16, M, C, w, 1e-5, rows, sc, sh, o.BF16)
        assert_bits_equal(h.to_numpy(), want_h, "h")
        q2, s2 = new(dev, "I8", [M, C]), new(dev, "F32", [M])
        ops.int8_quantize(h, q2, s2, group)
        assert_bits_equal(s2.to_numpy(), want_s, "two-call scales")
        codes_close(q2.to_numpy(), want_q, "two-call codes")


# ---- the hidden width's norm kernels stream their rows over the resident blocks, each block keeping the weight and
# one decoded table row in LDS: on a context sized for 2 compute units (H3S_CUS=2) every block takes many steps; the
# row table has segments of three table rows whose boundaries fall inside steps (a step's rows then read table rows
# other than the block's cached one from memory) and between them (the cache is refilled) ----
@pytest.fixture(scope="module")
def dev_cus2():
    import os
    from sycl_minimax_h3_amd import Device

    old = {k: os.environ.get(k) for k in ("H3S_CUS", "H3S_QUANT_WAVE_MIN_ROWS")}
    os.environ.update({"H3S_CUS": "2", "H3S_QUANT_WAVE_MIN_ROWS": "0"})
    try:
        d = Device.open()
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v
    yield d
    d.close()


def segment_rows(M):
    r = np.zeros(M, dtype=np.int32)
    r[:37] = 1
    r[37:41] = 2
    r[41:90] = 0
    r[90:91] = 1
    r[91:300] = 2
    r[300:] = 0
    return r


@pytest.mark.parametrize("M", [401, 130])
@pytest.mark.parametrize("rot,group", [(o.ROT_REGULAR, 256), (o.ROT_NONE, 0)])
def test_norm_quant_streamed_steps(dev_cus2, M, rot, group):
    dev, C = dev_cus2, DH
    x = bf16_rows(61 + M, M, C)
    rng = np.random.default_rng(62)
    w = (1.0 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    sc = (0.3 * rng.standard_normal(3 * C)).astype(np.float32)
    sh = (0.3 * rng.standard_normal(3 * C)).astype(np.float32)
    rows = segment_rows(M)
    want_q, want_s = o.norm_quant(x, o.BF16, M, C, w, 1e-5, rows, sc, sh, o.F32, o.BF16, rot, group)
    q, s = new(dev, "I8", [M, C]), new(dev, "F32", [M])
    tb = ops.Tables(scale=up(dev, sc, "F32", [3, C]), shift=up(dev, sh, "F32", [3, C]), rows=up(dev, rows, "I32", [M]))
    ops.norm_quant(up(dev, x, "BF16", [M, C]), up(dev, w, "F32", [C]), 1e-5, tb, q, s, rot=rot, group=group)
    assert_bits_equal(s.to_numpy(), want_s, "scales")
    codes_close(q.to_numpy(), want_q, "codes")


@pytest.mark.parametrize("M", [401, 130])
@pytest.mark.parametrize("mod", [True, False])
def test_rms_norm_mod_streamed_steps(dev_cus2, M, mod):
    dev, C = dev_cus2, DH
    x = bf16_rows(63 + M, M, C)
    rng = np.random.default_rng(64)
    w = (1.0 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    sc = (0.3 * rng.standard_normal(3 * C)).astype(np.float32) if mod else None
    sh = (0.3 * rng.standard_normal(3 * C)).astype(np.float32) if mod else None
    rows = segment_rows(M) if mod else None
    want = o.rms_norm_mod(x, o.BF16, M, C, w, 1e-5, rows, sc, sh, o.BF16)
    h = new(dev, "BF16", [M, C])
    m = ops.Mod(up(dev, rows, "I32", [M]), up(dev, sc, "F32", [3, C]), up(dev, sh, "F32", [3, C])) if mod else None
    ops.rms_norm_mod(up(dev, x, "BF16", [M, C]), up(dev, w, "F32", [C]), 1e-5, m, h)
    assert_bits_equal(h.to_numpy(), want, "h")


# ---- h3s_rms_norm_mod at the hidden width in both layouts (the one-wavefront form stores h itself) ----
@pytest.mark.parametrize("mod", [True, False])
@pytest.mark.parametrize("M", [1, 37, 300])
@pytest.mark.parametrize("layout", ["four", "wave"])
def test_rms_norm_mod_dit_width(request, layout, mod, M):
    dev = request.getfixturevalue("dev" if layout == "four" else "dev_wave")
    C = DH
    x = bf16_rows(80 + M, M, C)
    rng = np.random.default_rng(81)
    w = (1.0 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    R = 3
    rows = (np.arange(M) * 7 % R).astype(np.int32) if mod else None
    sc = (0.3 * rng.standard_normal(R * C)).astype(np.float32) if mod else None
    sh = (0.3 * rng.standard_normal(R * C)).astype(np.float32) if mod else None
    want = o.rms_norm_mod(x, o.BF16, M, C, w, 1e-5, rows, sc, sh, o.BF16)
    h = new(dev, "BF16", [M, C])
    m = ops.Mod(up(dev, rows, "I32", [M]), up(dev, sc, "F32", [R, C]), up(dev, sh, "F32", [R, C])) if mod else None
    ops.rms_norm_mod(up(dev, x, "BF16", [M, C]), up(dev, w, "F32", [C]), 1e-5, m, h)
    assert_bits_equal(h.to_numpy(), want, f"rms_norm_mod M={M}")


# ---- h3s_gate_add and h3s_swiglu at the block's shapes, many rows ----
def test_gate_add_dit_width(dev):
    M, C = 3000, DH
    x, other = bf16_rows(61, M, C, heavy=False), bf16_rows(62, M, C, heavy=False)
    gate = (0.5 * np.random.default_rng(63).standard_normal(2 * C)).astype(np.float32)
    rows = dit_rows(M)
    want = o.gate_add(x, o.BF16, M, C, other, o.BF16, rows, gate)
    xt = up(dev, x, "BF16", [M, C])
    ops.gate_add(xt, up(dev, other, "BF16", [M, C]), up(dev, rows, "I32", [M]), up(dev, gate, "F32", [2, C]))
    assert_bits_equal(xt.to_numpy(), want, "gate_add")


def test_swiglu_dit_width(dev):
    M, C = 1500, DFF
    x = bf16_rows(64, M, 2 * C, 4.0, heavy=False)
    want = o.swiglu(x, o.BF16, M, C, o.BF16)
    out = new(dev, "BF16", [M, C])
    ops.swiglu(up(dev, x, "BF16", [M, 2 * C]), out)
    from helpers import assert_close_16

    assert_close_16(out.to_numpy(), want, o.BF16, "swiglu", max_frac=2e-2)


# ---- h3s_rms_rope on q and on k inside the qkv buffer (stride 3 x 7168), many tokens ----
@pytest.mark.parametrize("rot", [126, 96])
def test_rms_rope_dit_many_tokens(dev, rot):
    M, H, D = 1100, DHEADS, DHD
    w_ = H * D
    qkv = bf16_rows(70 + rot, M, 3 * w_, heavy=False)
    rng = np.random.default_rng(71)
    wq, wk = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32), (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    ang = rng.uniform(-50, 50, (M, rot // 2))
    cs = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32).ravel()
    want = o.rms_rope(qkv, o.BF16, M, H, D, 3 * w_, wq, 1e-5, cs, rot)
    want = np.concatenate([want[:w_], o.rms_rope(want[w_:], o.BF16, M, H, D, 3 * w_, wk, 1e-5, cs, rot)])
    t = up(dev, qkv, "BF16", [M, 3 * w_])
    cst, wqt, wkt = up(dev, cs, "F32", [cs.size]), up(dev, wq, "F32", [D]), up(dev, wk, "F32", [D])
    ops.rms_rope(ops.Rows(t, 0, 3 * w_, M, H, D), wqt, 1e-5, cst, rot)
    ops.rms_rope(ops.Rows(t, w_, 3 * w_, M, H, D), wkt, 1e-5, cst, rot)
    assert_bits_equal(t.to_numpy(), want, f"rms_rope q then k, rot {rot}")
