"""Pins the CPU oracle (oracle/h3oracle.c) against the reference's own known answers and against what the mathematics
fixes: closed forms, brute force, invariants. CPU only."""
import math

import numpy as np
import pytest

from oracle import oracle as o


def f32_bits(u):
    return np.frombuffer(np.uint32(u).tobytes(), dtype=np.float32)[0]


# ---- element types: engine/h3-core/src/dtype.rs:137-155 ----
def test_bf16_round_trip_and_ties(oracle):
    L = oracle.lib()
    for v in [0.0, 1.0, -1.0, 0.5, 3.140625, -1234.0, 1e-20]:
        r = L.h3o_bf16_to_f32(L.h3o_f32_to_bf16(v))
        assert abs(r - v) <= abs(v) * 0.004
    # ties go to even (dtype.rs:144-145)
    assert L.h3o_f32_to_bf16(f32_bits(0x3F808000)) == 0x3F80
    assert L.h3o_f32_to_bf16(f32_bits(0x3F818000)) == 0x3F82
    # inf truncated, not rounded (dtype.rs:61-63)
    assert L.h3o_f32_to_bf16(float("inf")) == 0x7F80
    # the numpy restatement in oracle.py agrees with the C one on every pattern class
    x = np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 1000
    ref = np.array([L.h3o_f32_to_bf16(float(v)) for v in x[:2000]], dtype=np.uint16)
    assert np.array_equal(o.to_bf16(x[:2000]), ref)


def test_f16_values(oracle):
    L = oracle.lib()
    assert L.h3o_f16_to_f32(0x3C00) == 1.0
    assert L.h3o_f16_to_f32(0xC000) == -2.0
    assert L.h3o_f16_to_f32(0x0001) == pytest.approx(5.9604645e-08, rel=1e-7)
    assert L.h3o_f16_to_f32(0x7C00) == float("inf")
    assert L.h3o_f16_to_f32(0) == 0.0
    # f32 -> f16 agrees with numpy's IEEE conversion (round to nearest even) on random and subnormal values
    x = np.concatenate([np.random.default_rng(1).standard_normal(5000) * 100, np.linspace(-1e-5, 1e-5, 999)]).astype(np.float32)
    mine = np.array([L.h3o_f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(mine, x.astype(np.float16).view(np.uint16))


# ---- seeded inputs: engine/h3-core/src/rng.rs ----
def test_rng_published_vectors(oracle):
    # xoshiro256** from state {1, 2, 3, 4}: the published first outputs of the algorithm
    r = oracle.Rng(state=[1, 2, 3, 4])
    assert [r.next_u64() for _ in range(4)] == [11520, 0, 1509978240, 1215971899390074240]
    # splitmix64 seeded with 0: its published first output is the first state word
    assert oracle.Rng(0).state[0] == 0xE220A8397B1DCDAF


def test_rng_uniform_and_normal_moments(oracle):
    r = oracle.Rng(3)
    u = np.array([r.uniform() for _ in range(20000)])
    assert 0.0 <= u.min() and u.max() < 1.0 and abs(u.mean() - 0.5) < 0.01
    z = oracle.normal(5, 200000)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    # Box-Muller from two uniforms, restated in float64: the draws agree to float32 rounding
    r1, r2 = oracle.Rng(11), oracle.Rng(11)
    for _ in range(100):
        a, b = r2.uniform(), r2.uniform()
        want = math.sqrt(-2.0 * math.log(max(a, 1e-7))) * math.cos(2 * math.pi * b)
        assert abs(r1.normal() - want) < 1e-5 * max(1.0, abs(want))


# ---- rotations: engine/h3-core/src/reference.rs:4-23, 101-112; kernels/h3sycl.cpp:184-213, 433-459 ----
@pytest.mark.parametrize("g", [4, 16, 64, 256])
def test_regular_hadamard_orthonormal_and_symmetric(oracle, g):
    h = oracle.hadamard(g, oracle.ROT_REGULAR).astype(np.float64)
    assert np.abs(h @ h.T - np.eye(g)).max() < 1e-5
    assert np.array_equal(h, h.T)


def test_regular_hadamard_closed_form(oracle):
    h4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)
    want = np.kron(np.kron(h4, h4), h4) / 8.0
    # the digit of lowest weight is the innermost Kronecker factor
    assert np.allclose(oracle.hadamard(64, oracle.ROT_REGULAR), want, atol=1e-7)


@pytest.mark.parametrize("g", [2, 8, 128, 512])
def test_sylvester_closed_form_and_involution(oracle, g):
    h2 = np.array([[1, 1], [1, -1]], dtype=np.float64)
    want = np.array([[1.0]])
    for _ in range(int(math.log2(g))):
        want = np.kron(want, h2)
    want /= math.sqrt(g)
    h = oracle.hadamard(g, oracle.ROT_SYLVESTER).astype(np.float64)
    assert np.allclose(h, want, atol=1e-7)
    assert np.abs(h @ h - np.eye(g)).max() < 1e-5        # symmetric and orthonormal: its own inverse


@pytest.mark.parametrize("kind,g", [(o.ROT_REGULAR, 4), (o.ROT_REGULAR, 16), (o.ROT_REGULAR, 256), (o.ROT_SYLVESTER, 2),
                                    (o.ROT_SYLVESTER, 32), (o.ROT_SYLVESTER, 128)])
def test_butterfly_equals_dense_product(oracle, kind, g):
    rng = np.random.default_rng(g)
    h = oracle.hadamard(g, kind).astype(np.float64)
    for _ in range(20):
        x = rng.standard_normal(g).astype(np.float32) * rng.choice([1.0, 20.0])
        got = oracle.rotate_group(x, kind).astype(np.float64)
        want = x.astype(np.float64) @ h
        assert np.abs(got - want).max() <= 4e-6 * max(1.0, np.abs(x).sum() / math.sqrt(g))
    # a transposed or sign-flipped matrix would fail this: a unit vector picks out one row of H
    for i in [0, 1, g - 1]:
        e = np.zeros(g, dtype=np.float32)
        e[i] = 1.0
        assert np.allclose(oracle.rotate_group(e, kind), h[i], atol=1e-7)


# ---- quantizer: kernels/h3sycl.h:74-83, engine/h3-core/src/reference.rs:68-70 ----
def test_quantizer_invariants(oracle):
    rng = np.random.default_rng(2)
    M, K = 64, 512
    y = rng.standard_normal((M, K)).astype(np.float32) * rng.uniform(1e-3, 1e3, (M, 1)).astype(np.float32)
    y[5] = 0.0
    q, s = oracle.quantize_rows(y, M, K)
    q = q.reshape(M, K).astype(np.int32)
    assert s[5] == np.float32(1e-30) and not q[5].any()
    nz = [r for r in range(M) if r != 5]
    assert (np.abs(q[nz]).max(axis=1) == 127).all()
    assert np.array_equal(s[nz], np.maximum(np.abs(y[nz]).max(axis=1) / np.float32(127), np.float32(1e-30)))
    err = np.abs(y - q * s[:, None])
    assert (err <= s[:, None] * 0.5 * (1 + 1e-5)).all()


def test_quantizer_ties_to_even(oracle):
    # s = 127 / 127 = 1: values k + 0.5 are exact ties
    y = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5]], dtype=np.float32)
    q, s = oracle.quantize_rows(y, 1, 8)
    assert s[0] == 1.0
    assert list(q) == [127, 0, 2, 2, 0, -2, -2, 126]


def test_int8_linear_matches_a_plain_linear_within_quantization(oracle):
    """engine/h3-core/src/reference.rs:114-131, on the oracle."""
    m, k, n = 3, 64, 5
    r = oracle.Rng(7)
    x = np.array([r.normal() for _ in range(m * k)], dtype=np.float32)
    w = np.array([(r.next_u64() % 255) - 127 for _ in range(n * k)], dtype=np.int8)
    ws = np.array([0.01], dtype=np.float32)
    got = oracle.int8_linear(x, oracle.F32, m, k, w, n, ws, out_dt=oracle.F32)
    want = (x.reshape(m, k).astype(np.float64) @ w.reshape(n, k).T.astype(np.float64) * 0.01).astype(np.float32)
    rel, cos = oracle.compare(got, want.ravel())
    assert rel < 0.02 and cos > 0.999


def test_gemm_dequant_brute_force(oracle):
    rng = np.random.default_rng(4)
    M, K, N = 7, 128, 9
    q = rng.integers(-128, 128, (M, K), dtype=np.int8)
    w = rng.integers(-127, 128, (N, K), dtype=np.int8)
    s = rng.uniform(0.001, 0.1, M).astype(np.float32)
    acc = q.astype(np.int64) @ w.astype(np.int64).T
    bias = rng.standard_normal(N).astype(np.float32)
    # N scales: (acc * s) * ws[n] + b, each step rounded to float32
    ws = rng.uniform(0.005, 0.02, N).astype(np.float32)
    want = (acc.astype(np.float32) * s[:, None]) * ws[None, :] + bias[None, :]
    got = oracle.gemm_dequant(q.ravel(), s, M, K, w.ravel(), N, ws, bias, out_dt=oracle.F32).reshape(M, N)
    assert np.array_equal(got, want.astype(np.float32))
    # one scale: acc * fl(s * ws0)
    ws1 = np.array([0.0123], dtype=np.float32)
    want1 = acc.astype(np.float32) * (s * ws1[0])[:, None]
    got1 = oracle.gemm_dequant(q.ravel(), s, M, K, w.ravel(), N, ws1, None, out_dt=oracle.F32).reshape(M, N)
    assert np.array_equal(got1, want1.astype(np.float32))


# ---- the canonical reduction ----
def test_canon_sum_is_a_sum(oracle):
    rng = np.random.default_rng(5)
    for n, V, L in [(4096, 8, 64), (5376, 8, 64), (100, 4, 64), (128, 8, 8), (17, 8, 64), (4096, 8, 256), (5376, 8, 256),
                    (4096, 4, 256), (16384, 8, 512), (300, 1, 128)]:
        x = rng.standard_normal(n).astype(np.float32)
        exact = math.fsum(float(v) for v in x)
        got = oracle.canon_sum(x, V, L, oracle.SUM)
        assert abs(got - exact) <= 1e-6 * math.fsum(abs(float(v)) for v in x)
        exact2 = math.fsum(float(v) * float(v) for v in x)
        got2 = oracle.canon_sum(x, V, L, oracle.SUMSQ)
        assert abs(got2 - exact2) <= 1e-6 * exact2
    # the order is the one stated: with L = 2, V = 1, lanes hold the even and the odd positions
    x = np.array([1e8, 1.0, -1e8, 1.0], dtype=np.float32)
    # lane 0: 1e8 + -1e8 = 0; lane 1: 1 + 1 = 2; total 2 (a sequential sum would give 1)
    assert oracle.canon_sum(x, 1, 2, oracle.SUM) == 2.0
    # beyond one wavefront the 64-lane groups are summed first: lane 0 (1e8) and lane 1 (1) meet inside group 0,
    # where 1e8 + 1 rounds to 1e8, and -1e8 + 1 in group 1 likewise, so the total is 0; a plain 128-lane butterfly
    # would pair lane 0 with lane 64 first and give 2
    x = np.zeros(128, dtype=np.float32)
    x[0], x[1], x[64], x[65] = 1e8, 1.0, -1e8, 1.0
    assert oracle.canon_sum(x, 1, 128, oracle.SUM) == 0.0
    assert oracle.canon_sum(x, 1, 64, oracle.SUM) == 2.0


def test_row_lanes(oracle):
    # 64 lanes below 256 chunks of 16 bytes, 256 up to 1024 chunks, 512 up to 2048
    assert [oracle.row_lanes(n, 8) for n in (8, 2040, 2048, 4096, 5376, 8192, 8200, 16384)] == [64, 64, 256, 256, 256, 256, 512, 512]
    assert [oracle.row_lanes(n, 4) for n in (1020, 1024, 4096, 4100, 8192)] == [64, 256, 256, 512, 512]


# ---- the norms: kernels/h3sycl.cpp:766-810, 1248-1274 ----
def test_rms_norm_invariants(oracle):
    rng = np.random.default_rng(6)
    M, C = 16, 1024
    x = rng.standard_normal((M, C)).astype(np.float32) * 3
    w = np.full(C, 0.5, dtype=np.float32)
    y = oracle.rms_norm_mod(x, oracle.F32, M, C, w, 1e-6).reshape(M, C)
    assert np.allclose(np.sqrt((y.astype(np.float64) ** 2).mean(axis=1)), 0.5, rtol=1e-5)
    # against a float64 restatement
    want = x / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + 1e-6) * 0.5
    assert np.abs(y - want).max() < 1e-5
    # the modulation: rows pick table rows
    rows = np.array([i % 3 for i in range(M)], dtype=np.int32)
    sc = rng.standard_normal((3, C)).astype(np.float32)
    sh = rng.standard_normal((3, C)).astype(np.float32)
    ym = oracle.rms_norm_mod(x, oracle.F32, M, C, w, 1e-6, rows, sc, sh).reshape(M, C)
    assert np.allclose(ym, y * (1 + sc[rows]) + sh[rows], atol=1e-5)


def test_layer_norm_invariants(oracle):
    rng = np.random.default_rng(7)
    M, C = 8, 2048
    x = (rng.standard_normal((M, C)) * 4 + 10).astype(np.float32)
    x[3] = 7.0
    y = oracle.layer_norm(x, oracle.F32, M, C, None, None, 1e-5).reshape(M, C)
    assert np.abs(y[3]).max() == 0.0                              # a constant row goes to zero
    ok = [r for r in range(M) if r != 3]
    assert np.abs(y[ok].mean(axis=1)).max() < 1e-5
    assert np.abs(y[ok].var(axis=1) - 1).max() < 1e-3
    w = rng.standard_normal(C).astype(np.float32)
    b = rng.standard_normal(C).astype(np.float32)
    yw = oracle.layer_norm(x, oracle.F32, M, C, w, b, 1e-5).reshape(M, C)
    assert np.array_equal(yw, (y * w + b).astype(np.float32))


# ---- rotary: kernels/h3sycl.cpp:1276-1376 ----
def test_rms_rope_invariants(oracle):
    rng = np.random.default_rng(8)
    M, H, D, rot = 5, 3, 64, 48
    stride = H * D + 16
    x = rng.standard_normal(M * stride).astype(np.float32)
    w = np.ones(D, dtype=np.float32)
    ang = rng.uniform(-10, 10, (M, rot // 2))
    cs = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32).ravel()
    y = oracle.rms_rope(x, oracle.F32, M, H, D, stride, w, 1e-5, cs, rot)
    ident = np.stack([np.ones((M, rot // 2)), np.zeros((M, rot // 2))], -1).astype(np.float32).ravel()
    n = oracle.rms_rope(x, oracle.F32, M, H, D, stride, w, 1e-5, ident, rot)     # zero angle: only the norm
    n0 = oracle.rms_rope(x, oracle.F32, M, H, D, stride, w, 1e-5, None, 0)        # rot_dim 0: only the norm
    assert np.array_equal(n, n0)
    X, Y, N0 = (a.reshape(M, stride)[:, : H * D].reshape(M, H, D) for a in (x, y, n0))
    assert np.array_equal(y.reshape(M, stride)[:, H * D:], x.reshape(M, stride)[:, H * D:])   # the gap is untouched
    rms = np.sqrt((X.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-5)
    assert np.allclose(N0, X / rms, atol=1e-5)
    h = rot // 2
    # each pair keeps its length, and the angle is the table's
    la = np.hypot(Y[..., :h], Y[..., h:rot])
    lb = np.hypot(N0[..., :h], N0[..., h:rot])
    assert np.allclose(la, lb, atol=1e-5)
    a, b = N0[..., :h], N0[..., h:rot]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    assert np.allclose(Y[..., :h], a * c - b * s, atol=1e-5)
    assert np.allclose(Y[..., h:rot], b * c + a * s, atol=1e-5)
    assert np.array_equal(Y[..., rot:], N0[..., rot:])              # features from rot_dim on: only normalized


# ---- activations: kernels/h3sycl.cpp:1395; engine/h3-core/src/audio.rs:440 ----
def test_activation_closed_forms(oracle):
    for v in np.linspace(-12, 12, 97):
        v = float(np.float32(v))
        gelu = 0.5 * v * (1 + math.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3)))
        silu = v / (1 + math.exp(-v))
        assert abs(oracle.act(v, oracle.ACT_GELU_TANH) - gelu) <= 2e-6 * max(1.0, abs(gelu))
        assert abs(oracle.act(v, oracle.ACT_SILU) - silu) <= 2e-6 * max(1.0, abs(silu))
    # GELU-tanh, not the erf form: at 1.0 they differ in the 4th digit
    assert abs(oracle.act(1.0, oracle.ACT_GELU_TANH) - 0.8411920) < 1e-6


def test_fused_chains_are_compositions(oracle):
    """norm_quant = rms_norm_mod into bf16, then the quantizer; norm_mod_act_gate = norm, modulate, act, gate_add."""
    rng = np.random.default_rng(9)
    M, C = 12, 1024
    x = oracle.to_bf16(rng.standard_normal((M, C)).astype(np.float32))
    w = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
    rows = np.zeros(M, dtype=np.int32)
    sc = (0.5 * rng.standard_normal((1, C))).astype(np.float32)
    sh = (0.5 * rng.standard_normal((1, C))).astype(np.float32)
    h = oracle.rms_norm_mod(x, oracle.BF16, M, C, w, 1e-6, rows, sc, sh)
    q, s = oracle.norm_quant(x, oracle.BF16, M, C, w, 1e-6, rows, sc, sh, oracle.F32, oracle.BF16)
    q2, s2 = oracle.quantize_rows(oracle.from_bf16(h), M, C)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    # with a rotation: quantize(rotate(h)) group by group
    q3, s3 = oracle.norm_quant(x, oracle.BF16, M, C, w, 1e-6, rows, sc, sh, oracle.F32, oracle.BF16, oracle.ROT_SYLVESTER, 128)
    hr = np.concatenate([oracle.rotate_group(g, oracle.ROT_SYLVESTER) for g in oracle.from_bf16(h).reshape(-1, 128)])
    q4, s4 = oracle.quantize_rows(hr, M, C)
    assert np.array_equal(q3, q4) and np.array_equal(s3, s4)
    # norm_mod_act_gate with act NONE, no gate and res = 0 rows equals rms_norm_mod into float32
    out = oracle.norm_mod_act_gate(x, oracle.BF16, M, C, oracle.NORM_RMS, w, None, 1e-6, rows, sc, sh, None, oracle.F32,
                                   oracle.ACT_NONE, None, oracle.BF16, oracle.F32)
    h32 = oracle.rms_norm_mod(x, oracle.BF16, M, C, w, 1e-6, rows, sc, sh, out_dt=oracle.F32)
    assert np.array_equal(out, h32)
    # and gate_add of the activation equals the fused residual
    res = oracle.to_bf16(rng.standard_normal((M, C)).astype(np.float32))
    gate = (0.5 * rng.standard_normal((1, C))).astype(np.float32)
    y = np.array([oracle.act(float(v), oracle.ACT_GELU_TANH) for v in h32], dtype=np.float32)
    want = oracle.gate_add(res, oracle.BF16, M, C, y, oracle.F32, rows, gate)
    got = oracle.norm_mod_act_gate(x, oracle.BF16, M, C, oracle.NORM_RMS, w, None, 1e-6, rows, sc, sh, gate, oracle.F32,
                                   oracle.ACT_GELU_TANH, res, oracle.BF16, oracle.BF16)
    assert np.array_equal(got, want.ravel())


# ---- swiglu -> act -> quantizer: the fused oracle is the composition of the pinned steps ----
@pytest.mark.parametrize("x_dt,h_dt", [(o.BF16, o.BF16), (o.F16, o.F16), (o.F32, o.F32), (o.F32, o.BF16)])
@pytest.mark.parametrize("rot,group", [(o.ROT_NONE, 0), (o.ROT_REGULAR, 256), (o.ROT_SYLVESTER, 128)])
def test_swiglu_quant_is_swiglu_then_quantizer(x_dt, h_dt, rot, group):
    M, C = 5, 512
    x = o.to_dt(np.random.default_rng(41).standard_normal(M * 2 * C).astype(np.float32) * 3, x_dt)
    q, s = o.swiglu_quant(x, x_dt, M, C, h_dt, rot, group)
    act = o.swiglu(x, x_dt, M, C, h_dt)
    q2, s2 = o.quantize_act(act, h_dt, M, C, rot, group)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    # the quantizer alone, unrotated, is h3o_quantize_rows on the values (the quantizer of h3o_int8_linear)
    if rot == o.ROT_NONE:
        y = o.from_dt(act, h_dt).astype(np.float32)
        q3 = np.empty(M * C, dtype=np.int8)
        s3 = np.empty(M, dtype=np.float32)
        o.lib().h3o_quantize_rows(o._p(y), M, C, o._p(q3), o._p(s3))
        assert np.array_equal(q, q3) and np.array_equal(s, s3)
    # the invariants of the quantizer hold on the rotated act
    assert np.all(np.abs(q.reshape(M, C)).max(1) == 127)


# ---- attention (kernels/h3sycl.cpp:1676-1767, 1496-1550) ----
def _attn_inputs(seed, S, H, D, dt, stride=None, spread=1.0):
    stride = H * D if stride is None else stride
    g = np.random.default_rng(seed)
    mk = lambda: o.to_dt((g.standard_normal((S, stride)) * spread).astype(np.float32), dt).ravel()  # noqa: E731
    return mk(), mk(), mk(), stride


def test_sage_quantize_invariants():
    """One scale per head per 64 rows; max |code| 127 in every nonzero block; |x - code * scale| <= scale / 2 up to
    the rounding of x * (127 / m); exact halves round away from zero; a zero block has scale 0 and codes 0."""
    S, H, D = 150, 3, 64
    x = np.random.default_rng(50).standard_normal((S, H * D)).astype(np.float32)
    x[64:128, D:2 * D] = 0.0                         # head 1, block 1: zeros
    codes, scales = o.sage_quantize(x.ravel(), o.F32, S, H, D)
    nb = 3
    c = codes.reshape(H, S, D).astype(np.int32)
    sc = scales.reshape(H, nb)
    for h in range(H):
        for b in range(nb):
            blk = x[b * 64:(b + 1) * 64, h * D:(h + 1) * D]
            cb = c[h, b * 64:(b + 1) * 64]
            if not blk.any():
                assert sc[h, b] == 0 and not cb.any()
                continue
            assert sc[h, b] == np.float32(np.float32(np.abs(blk).max()) / np.float32(127))
            assert np.abs(cb).max() == 127
            err = np.abs(blk.astype(np.float64) - cb * np.float64(sc[h, b]))
            assert err.max() <= sc[h, b] * (0.5 + 1e-4)
    # halves: x * 127 / m lands exactly on k + 0.5 for x = (k + 0.5) m / 127 with m = 127 (inv = 1)
    y = np.zeros((64, 4), np.float32)
    y[0, 0] = 127.0
    y[1, :] = [2.5, -2.5, 0.5, -0.5]
    codes, scales = o.sage_quantize(y.ravel(), o.F32, 64, 1, 4)
    assert scales[0] == 1.0
    assert list(codes.reshape(64, 4)[1]) == [3, -3, 1, -1]


def test_sage_mean_is_a_float32_sum_in_token_order():
    S, H, D = 300, 2, 64
    q, k, v, _ = _attn_inputs(51, S, H, D, o.BF16)
    _, _, _, _, _, km = o.attention(q, k, v, o.BF16, S, H, D, sage=True)
    kf = o.from_dt(k, o.BF16).reshape(S, H * D)
    want = (np.add.accumulate(kf, axis=0, dtype=np.float32)[-1] / np.float32(S)).astype(np.float32)
    assert np.array_equal(km, want)


@pytest.mark.parametrize("sage", [True, False])
def test_attention_special_cases(sage):
    H, D = 2, 64
    # one token: the softmax is 1, out = v (through half)
    q, k, v, _ = _attn_inputs(52, 1, H, D, o.F32)
    out = o.attention(q, k, v, o.F32, 1, H, D, out_dt=o.F32, sage=sage)
    out = out[0] if sage else out
    assert np.array_equal(out, o.from_dt(o.to_dt(v, o.F16), o.F16))
    # identical keys: uniform weights, out = the mean of v (within half's rounding)
    S = 96
    q, _, v, _ = _attn_inputs(53, S, H, D, o.F32)
    k = np.tile(np.random.default_rng(54).standard_normal(H * D).astype(np.float32), S)
    out = o.attention(q, k, v, o.F32, S, H, D, out_dt=o.F32, sage=sage)
    out = out[0] if sage else out
    vh = o.from_dt(o.to_dt(v, o.F16), o.F16).reshape(S, H * D).astype(np.float64)
    assert np.allclose(out.reshape(S, H * D), vh.mean(0)[None, :], rtol=2e-3, atol=2e-3)
    # one key far above the rest: out = that key's v
    q = np.ones(S * H * D, np.float32)
    k = -np.ones(S * H * D, np.float32)
    k.reshape(S, H * D)[37] = 1.0
    out = o.attention(q, k, v, o.F32, S, H, D, out_dt=o.F32, sage=sage)
    out = out[0] if sage else out
    assert np.allclose(out.reshape(S, H * D), vh[37][None, :], rtol=1e-3, atol=1e-3)


def test_attention_against_dense_softmax():
    """The 16-bit form against an independent dense formulation (numpy matmul + softmax over half values), and the
    sage form against the same formulation on its dequantized q and k - mean (the mean cancels in the softmax)."""
    S, H, D, stride = 130, 3, 64, 3 * 64 + 16
    q, k, v, _ = _attn_inputs(55, S, H, D, o.BF16, stride)
    half = lambda a: o.from_dt(o.to_dt(o.from_dt(a, o.BF16), o.F16), o.F16).reshape(S, stride)[:, :H * D].reshape(S, H, D).astype(np.float64)  # noqa: E731
    qh, kh, vh = half(q), half(k), half(v)
    sm = np.float32(1) / np.sqrt(np.float32(D))

    def dense(qq, kk, vv):
        s = np.einsum("shd,thd->hst", qq, kk) * float(sm)
        s -= s.max(-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(-1, keepdims=True)
        return np.einsum("hst,thd->shd", p, vv).reshape(S, H * D)

    out16 = o.attention(q, k, v, o.BF16, S, H, D, stride, out_dt=o.F32, sage=False)
    assert np.allclose(out16.reshape(S, H * D), dense(qh, kh, vh), rtol=1e-3, atol=1e-3)
    out, iq, ik, qs, ks, km = o.attention(q, k, v, o.BF16, S, H, D, stride, out_dt=o.F32, sage=True)
    nb = (S + 63) // 64
    deq = lambda c, s_: (c.reshape(H, S, D).astype(np.float64) * np.repeat(s_.reshape(H, nb), 64, 1)[:, :S, None]).transpose(1, 0, 2)  # noqa: E731
    assert np.allclose(out.reshape(S, H * D), dense(deq(iq, qs), deq(ik, ks), vh), rtol=1e-3, atol=1e-3)
    # and the sage result stays close to the exact attention (the quantization error of q and k)
    rel, cos = o.compare(out.astype(np.float32), dense(qh, kh, vh).astype(np.float32).ravel())
    assert rel < 0.05 and cos > 0.998


# ---- plain linear layers (kernels/h3sycl.cpp:656-739) ----
def test_linear_oracle_closed_forms():
    """An identity weight gives x back (rounded once to out's type); the bias adds per column; accumulation adds the
    previous output; scale_rows scales each row."""
    M, K = 5, 16
    x = o.to_bf16(np.random.default_rng(85).standard_normal((M, K)).astype(np.float32)).ravel()
    eye = o.to_bf16(np.eye(K, dtype=np.float32)).ravel()
    out = o.linear(x, o.BF16, M, K, eye, K, out_dt=o.BF16)
    assert np.array_equal(out, x)
    bias = np.arange(K, dtype=np.float32)
    out = o.linear(x, o.BF16, M, K, eye, K, bias, out_dt=o.F32)
    assert np.array_equal(out.reshape(M, K), o.from_dt(x, o.BF16).reshape(M, K) + bias[None, :])
    acc = o.linear(x, o.BF16, M, K, eye, K, None, out_dt=o.BF16, acc_into=x)
    assert np.array_equal(acc, o.to_bf16(2 * o.from_dt(x, o.BF16)))
    s = np.array([1, 2, 0.5, -1, 0], np.float32)
    sr = o.scale_rows(x, o.BF16, M, K, s)
    assert np.array_equal(o.from_dt(sr, o.BF16).reshape(M, K), o.from_dt(x, o.BF16).reshape(M, K) * s[:, None])
    # a general product against numpy's float64 matrix product
    w = o.to_bf16(np.random.default_rng(86).standard_normal((7, K)).astype(np.float32)).ravel()
    out = o.linear(x, o.BF16, M, K, w, 7, out_dt=o.F32)
    want = (o.from_dt(x, o.BF16).reshape(M, K).astype(np.float64) @ o.from_dt(w, o.BF16).reshape(7, K).T.astype(np.float64))
    assert np.allclose(out.reshape(M, 7), want, rtol=1e-6, atol=1e-6)


def test_attention_causal_oracle():
    """Row 0 sees only key 0 (out = v[0]); with one kv head shared by all query heads, each head is the non-causal
    attention over the prefix; the last row equals the full (non-causal) attention of the 16-bit form on f32 inputs."""
    L, Hq, Hkv, D = 40, 4, 2, 64
    g = np.random.default_rng(95)
    q = g.standard_normal((L, Hq * D)).astype(np.float32)
    k = g.standard_normal((L, Hkv * D)).astype(np.float32)
    v = g.standard_normal((L, Hkv * D)).astype(np.float32)
    out = o.attention_causal(q.ravel(), k.ravel(), v.ravel(), o.F32, L, Hq, Hkv, D).reshape(L, Hq, D)
    for h in range(Hq):
        gkv = h // (Hq // Hkv)
        assert np.allclose(out[0, h], v[0, gkv * D:(gkv + 1) * D], rtol=1e-6, atol=1e-6)
        # an independent dense formulation with the causal mask
        s = (q[:, h * D:(h + 1) * D].astype(np.float64) @ k[:, gkv * D:(gkv + 1) * D].T.astype(np.float64)) / np.sqrt(np.float32(D))
        s[np.triu_indices(L, 1)] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        assert np.allclose(out[:, h], p @ v[:, gkv * D:(gkv + 1) * D], rtol=1e-5, atol=1e-5)


# ---- the regular butterfly's association: kernels/h3sycl.cpp:433-456 ----
# A planted digit: a column of four values [a, e a, e a, e a] with e = 2^-24. Summed left to right (the two digits a
# work-item of the reference holds in registers, h3sycl.cpp:440), a + e a rounds back to a at each step, so
# t = a and the outputs are [a (1 - 2^-23)] * 3 + [-a]; summed pairwise (the digits across lanes, h3sycl.cpp:452-453),
# t = a (1 + 2^-23) exactly and the outputs are [a] * 3 + [a (-1 + 2^-23)]. Every other digit of the planted input
# sees a column [v, 0, 0, 0], whose outputs [v, v, v, -v] are exact, so the whole result is known in closed form.
def _planted_digit(g, k):
    x = np.zeros(g, dtype=np.float32)
    d = 4 ** k
    x[0] = 1.0
    x[d] = x[2 * d] = x[3 * d] = np.float32(2.0 ** -24)
    return x


def _planted_expected(g, k, left_to_right):
    nd = int(round(math.log(g, 4)))
    mid = [1 - 2.0 ** -23] * 3 + [-1.0] if left_to_right else [1.0] * 3 + [-1 + 2.0 ** -23]
    sign = [1.0, 1.0, 1.0, -1.0]
    y = np.empty(g, dtype=np.float64)
    for p in range(g):
        v = 1.0
        for j in range(nd):
            digit = (p // 4 ** j) % 4
            v *= mid[digit] if j == k else sign[digit]
        y[p] = v / math.sqrt(g)
    return y.astype(np.float32)


@pytest.mark.parametrize("g", [4, 16, 64, 256])
def test_regular_butterfly_association(oracle, g):
    """digits of stride 1 and 4 left to right, of stride 16 and 64 pairwise"""
    for k in range(int(round(math.log(g, 4)))):
        got = oracle.rotate_group(_planted_digit(g, k), oracle.ROT_REGULAR)
        want = _planted_expected(g, k, left_to_right=4 ** k < 16)
        other = _planted_expected(g, k, left_to_right=4 ** k >= 16)
        assert not np.array_equal(want, other)
        assert np.array_equal(got, want), f"g {g}, digit {k}"


def test_regular_butterfly_digit_order(oracle):
    """The low digit first (h3sycl.cpp:433-456). x[0] = 1, x[1..3] = e and x[4] = x[8] = x[12] = e, e = 2^-24: the
    first digit turns the column (0..3) into [1 - 2e] * 3 + [-1], the second then sums each column
    [1 - 2e, e, e, e] left to right to exactly 1 (and [-1, -e, -e, -e] to -1), so position r + 4 q holds
    [1 - 2e, 1 - 2e, 1 - 2e, -1 + 4e][q] for r < 3 and [-1 + 2e, -1 + 2e, -1 + 2e, 1][q] for r = 3. Taken the other
    way round, position 3 would hold -1 + 4e instead of -1 + 2e."""
    e = 2.0 ** -24
    x = np.zeros(16, dtype=np.float32)
    x[0] = 1.0
    x[[1, 2, 3, 4, 8, 12]] = np.float32(e)
    col = [1 - 2 * e, 1 - 2 * e, 1 - 2 * e, -1 + 4 * e]
    last = [-1 + 2 * e, -1 + 2 * e, -1 + 2 * e, 1.0]
    want = np.array([(col if r < 3 else last)[q] / 4 for q in range(4) for r in range(4)], dtype=np.float32)
    assert np.array_equal(oracle.rotate_group(x, oracle.ROT_REGULAR), want)


def test_convrot_codes_against_the_reference_cpu_arithmetic(oracle):
    """The g = 256 quantizer of h3s_int8_linear against engine/h3-core/src/reference.rs:52-70: each rotated value as
    the reference's CPU path forms it (a float32 sum over the dense normalized matrix in input order), its row scale
    and round_ties_even. The two orders of summation may round differently, so a code may differ by 1 - only where
    the exact value y / s lies within the two computations' error bound of a rounding boundary. The bound per
    element: the dense sum errs by at most 255 u A and the butterfly (four digits, at most four roundings each) by
    16 u A, A = sum |x_i| / 16 over the group, u = 2^-24; the scale carries the error of its row's maximum. No code
    may differ by 2 or more."""
    u = 2.0 ** -24
    M, K, g = 256, 4096, 256
    rng = np.random.default_rng(5)
    x = rng.standard_normal((M, K)).astype(np.float32) * np.where(rng.random(K) < 0.01, 20.0, 1.0).astype(np.float32)
    xb = oracle.to_bf16(x)
    X = oracle.from_bf16(xb).reshape(M, K // g, g)
    q_o, s_o = oracle.quantize_act(xb.ravel(), oracle.BF16, M, K, oracle.ROT_REGULAR, g)
    q_o = q_o.reshape(M, K).astype(np.int32)
    H = oracle.hadamard(g, oracle.ROT_REGULAR)
    acc = np.zeros_like(X)
    for i in range(g):                                          # reference.rs:57-60, in float32 without fma
        acc = (acc + X[:, :, i:i + 1] * H[i][None, None, :]).astype(np.float32)
    xr = acc.reshape(M, K)
    s_r = np.maximum(np.abs(xr).max(1) / np.float32(127), np.float32(1e-30)).astype(np.float32)   # reference.rs:67
    q_r = np.clip(np.rint(xr / s_r[:, None]), -128, 127).astype(np.int32)                          # reference.rs:68-70
    ye = (X.astype(np.float64) @ H.astype(np.float64)).reshape(M, K)
    me = np.abs(ye).max(1)
    z = ye / (me / 127)[:, None]
    A = np.abs(X.astype(np.float64)).sum(-1) / 16
    err = (255 + 16) * u * 1.01
    delta = err * np.repeat(A, g, axis=1) / (me / 127)[:, None] + np.abs(z) * (err * A.max(1) / me + 3 * u)[:, None]
    d = q_o - q_r
    assert np.abs(d).max() <= 1
    bad = d != 0
    boundary = np.minimum(q_o, q_r) + 0.5
    assert np.all(np.abs(z - boundary)[bad] <= delta[bad]), "a code differs away from a rounding boundary"
    assert np.all(np.abs(s_o / s_r - 1) <= 4 * u)
    # the comparison has teeth: the butterfly with the wrong mirror (y_a = t - 2 x_a, the matrix ones - 2 I per digit)
    # moves codes by 2 or more
    hm = np.ones((4, 4)) - 2 * np.eye(4)
    Hm = np.kron(np.kron(hm, hm), np.kron(hm, hm)) / 16
    qm, _ = oracle.quantize_rows(np.ascontiguousarray((X.astype(np.float64) @ Hm).astype(np.float32).reshape(M, K)), M, K)
    assert np.abs(qm.reshape(M, K).astype(np.int32) - q_r).max() >= 2


# ---- closed forms for the pointwise oracle functions ----
def test_swiglu_closed_form(oracle):
    """kernels/h3sycl.cpp:1394-1396: out = silu(x[:, :C]) * x[:, C:], the gate half first"""
    M, C = 9, 520
    x = (3 * np.random.default_rng(50).standard_normal((M, 2 * C))).astype(np.float32)
    g, up_ = x[:, :C].astype(np.float64), x[:, C:].astype(np.float64)
    want = g / (1 + np.exp(-g)) * up_
    got = oracle.swiglu(x.ravel(), oracle.F32, M, C, oracle.F32).reshape(M, C)
    assert np.all(np.abs(got - want) <= 4e-7 * np.abs(want) + 1e-30)
    # 16-bit in and out: within one unit in the last place of the float64 value
    xb = oracle.to_bf16(x)
    xf = oracle.from_bf16(xb).astype(np.float64).reshape(M, 2 * C)
    want16 = xf[:, :C] / (1 + np.exp(-xf[:, :C])) * xf[:, C:]
    got16 = oracle.from_bf16(oracle.swiglu(xb.ravel(), oracle.BF16, M, C, oracle.BF16)).reshape(M, C)
    assert np.all(np.abs(got16 - want16) <= 2.0 ** -8 * np.abs(want16) + 1e-30)


def test_gate_add_closed_form(oracle):
    """kernels/h3sycl.cpp:1421-1431: x[r] += other[r] * gate[rows[r]], in float32, rounded once to x's type; rows
    that are not the identity"""
    M, C, R = 7, 264, 4
    rng = np.random.default_rng(51)
    x = oracle.to_bf16(rng.standard_normal((M, C)).astype(np.float32))
    other = rng.standard_normal((M, C)).astype(np.float32)
    rows = np.array([3, 0, 2, 2, 1, 3, 0], dtype=np.int32)
    gate = rng.standard_normal((R, C)).astype(np.float32)
    want = oracle.to_bf16(oracle.from_bf16(x).reshape(M, C) + other * gate[rows])
    got = oracle.gate_add(x.ravel(), oracle.BF16, M, C, other.ravel(), oracle.F32, rows, gate.ravel())
    assert np.array_equal(got, want.ravel())
    # no gate: a plain add (ops.rs add)
    want = oracle.to_bf16(oracle.from_bf16(x).reshape(M, C) + other)
    assert np.array_equal(oracle.gate_add(x.ravel(), oracle.BF16, M, C, other.ravel(), oracle.F32), want.ravel())


@pytest.mark.parametrize("affine", [False, True])
def test_layer_norm_chain_is_a_composition(oracle, affine):
    """Config 2's chain (h3o_norm_mod_act_gate with the layer norm) equals h3o_layer_norm into float32, then
    x (1 + scale) + shift, GELU-tanh, * gate and + res in float32, rounded once to bfloat16, with [1, C] bfloat16
    tables (every row reads table row 0)."""
    M, C = 24, 4096
    rng = np.random.default_rng(52)
    x = oracle.to_bf16(rng.standard_normal((M, C)).astype(np.float32))
    res = oracle.to_bf16(rng.standard_normal((M, C)).astype(np.float32))
    sc, sh, gt = (oracle.to_bf16((0.5 * rng.standard_normal(C)).astype(np.float32)) for _ in range(3))
    w = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32) if affine else None
    b = (0.1 * rng.standard_normal(C)).astype(np.float32) if affine else None
    got = oracle.norm_mod_act_gate(x.ravel(), oracle.BF16, M, C, oracle.NORM_LAYER, w, b, 1e-5, None, sc, sh, gt,
                                   oracle.BF16, oracle.ACT_GELU_TANH, res.ravel(), oracle.BF16, oracle.BF16)
    ln = oracle.layer_norm(x.ravel(), oracle.BF16, M, C, w, b, 1e-5, oracle.F32).reshape(M, C)
    f = oracle.from_bf16
    v = (ln * (np.float32(1) + f(sc))[None]).astype(np.float32) + f(sh)[None]
    v = oracle.act_n(v, oracle.ACT_GELU_TANH).reshape(M, C)
    want = oracle.to_bf16(f(res).reshape(M, C) + (v * f(gt)[None]).astype(np.float32))
    assert np.array_equal(got, want.ravel())
    # a mis-indexed table (the shift read as the scale) is caught
    bad = oracle.norm_mod_act_gate(x.ravel(), oracle.BF16, M, C, oracle.NORM_LAYER, w, b, 1e-5, None, sh, sc, gt,
                                   oracle.BF16, oracle.ACT_GELU_TANH, res.ravel(), oracle.BF16, oracle.BF16)
    assert not np.array_equal(bad, want.ravel())


def test_rms_rope_norm_is_the_canonical_head_sum(oracle):
    """A head's norm is the canonical sum over pow2ceil(D / V) lanes, one 16-byte chunk a lane. With rot_dim 0 and a
    unit weight, feature 0 = 1 reads inv off the output. Planted (float32, V = 4, D = 128: 32 lanes): 1, 2^24, 1 in
    chunks 0, 1, 2. The butterfly adds chunks 0 and 2 first (2), then 2^24 + 2 exactly; a sequential sum loses both
    ones to ties (2^24 + 1 rounds to 2^24)."""
    D = 128
    inv = lambda s, n=D: np.float32(1.0) / np.sqrt(np.float32(np.float32(s) / np.float32(n)) + np.float32(1e-5))   # noqa: E731
    x = np.zeros(D, dtype=np.float32)
    x[0], x[4], x[8] = 1.0, 4096.0, 1.0
    w = np.ones(D, dtype=np.float32)
    y = oracle.rms_rope(x, oracle.F32, 1, 1, D, D, w, 1e-5, None, 0)
    assert oracle.canon_sum(x, 4, 32, oracle.SUMSQ) == 2.0 ** 24 + 2
    seq = np.float32(0.0)
    for v in x:
        seq = np.float32(seq + np.float32(v * v))
    assert seq == 2.0 ** 24
    assert y[0] == inv(2.0 ** 24 + 2) and y[0] != inv(seq)
    # random heads: float32 of 128 (32 lanes) and bfloat16 of 80 features (10 chunks of 8, padded to 16 lanes)
    xr = np.random.default_rng(3).standard_normal(D).astype(np.float32) * 3
    xr[0] = 1.0
    assert oracle.rms_rope(xr, oracle.F32, 1, 1, D, D, w, 1e-5, None, 0)[0] == inv(oracle.canon_sum(xr, 4, 32, oracle.SUMSQ))
    xb = oracle.to_bf16(np.random.default_rng(4).standard_normal(80).astype(np.float32) * 3)
    yb = oracle.rms_rope(xb, oracle.BF16, 1, 1, 80, 80, np.ones(80, np.float32), 1e-5, None, 0)
    xf = oracle.from_bf16(xb)
    inv_b = inv(oracle.canon_sum(xf, 8, 16, oracle.SUMSQ), 80)
    assert np.array_equal(yb, oracle.to_bf16((xf * inv_b).astype(np.float32)))


# ---- rotary with partial slots: rot_dim / 2 or D - rot_dim not a whole 16-byte vector ----
@pytest.mark.parametrize("dt", [o.F32, o.BF16])
@pytest.mark.parametrize("D,rot", [(128, 126), (128, 120), (128, 60), (128, 2), (64, 48), (128, 128)])
def test_rms_rope_partial_slots(oracle, dt, D, rot):
    """Every even rot_dim with an even remainder (kernels/h3sycl.cpp:1280-1282): the pairs (j, rot/2 + j) rotate by
    the table's angle, features from rot_dim on are only normalized, and the norm is the head's RMS."""
    rng = np.random.default_rng(53)
    M, H = 4, 3
    stride = 3 * H * D
    x = oracle.to_dt(rng.standard_normal(M * stride).astype(np.float32), dt)
    w = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    h = rot // 2
    ang = rng.uniform(-10, 10, (M, h))
    cs = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32).ravel()
    y = oracle.from_dt(oracle.rms_rope(x, dt, M, H, D, stride, w, 1e-5, cs, rot), dt).reshape(M, stride)
    X = oracle.from_dt(x, dt).reshape(M, stride).astype(np.float64)
    assert np.array_equal(y[:, H * D:], X[:, H * D:].astype(np.float32))            # the rest of the row is untouched
    Xh, Y = X[:, :H * D].reshape(M, H, D), y[:, :H * D].reshape(M, H, D).astype(np.float64)
    N = Xh / np.sqrt((Xh ** 2).mean(-1, keepdims=True) + 1e-5) * w
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    tol = 1e-5 if dt == o.F32 else 2.0 ** -7
    want = np.concatenate([N[..., :h] * c - N[..., h:rot] * s, N[..., h:rot] * c + N[..., :h] * s, N[..., rot:]], -1)
    assert np.all(np.abs(Y - want) <= tol * (1 + np.abs(want)))
