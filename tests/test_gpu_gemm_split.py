"""GPU parity of the matrix-core GEMMs whose last tiles split along K (int8: h3s_int8_gemm_dequant, h3s_int8_linear;
16-bit: h3s_linear, h3s_linear_acc), against the oracle. The split takes rows of at least 12288 bytes; a context
that sizes its grids for 4 compute units (H3S_CUS=4) gives small products the short last round it is for: 6 tiles
(4 whole, 2 in 2 parts of 48 K steps) and 5 tiles (4 whole, the fifth in 4 parts, the last ending on a half step
where K is an odd multiple of 64 bytes). The int8 parts' int32 sums are exact, so the int8 results stay bit for bit
the oracle's; the 16-bit results keep the float linear's tolerance."""
import os

import numpy as np
import pytest

from oracle import oracle as o
from helpers import assert_bits_equal, assert_close_16, new, up
from sycl_minimax_h3_amd import DType, ops

pytestmark = pytest.mark.gpu
o.set_threads(8)
DTS = {o.F32: DType.F32, o.F16: DType.F16, o.BF16: DType.BF16}


@pytest.fixture(scope="module")
def dev4():
    from sycl_minimax_h3_amd import Device

    old = os.environ.get("H3S_CUS")
    os.environ["H3S_CUS"] = "4"
    try:
        d = Device.open()
    finally:
        if old is None:
            del os.environ["H3S_CUS"]
        else:
            os.environ["H3S_CUS"] = old
    yield d
    d.close()


# (M, K, N): tiles of 256 x 256, K steps of 128 bytes
SHAPES_I8 = [(260, 12288, 600),   # 2 x 3 tiles: 4 whole, 2 in 2 parts of 48 steps
             (1100, 12352, 200)]  # 5 x 1: 4 whole, 1 in 4 parts; 96.5 steps, the half step in the last part


@pytest.mark.parametrize("act", [o.ACT_NONE, o.ACT_SILU])
@pytest.mark.parametrize("per_n,bias,out_dt", [(False, False, o.BF16), (True, True, o.BF16), (True, False, o.F32),
                                               (False, True, o.F16)])
@pytest.mark.parametrize("M,K,N", SHAPES_I8)
def test_int8_gemm_split(dev4, M, K, N, per_n, bias, out_dt, act):
    rng = np.random.default_rng(M + K + N)
    q = rng.integers(-128, 128, M * K, dtype=np.int8)
    s = rng.uniform(0.001, 0.05, M).astype(np.float32)
    w = rng.integers(-127, 128, N * K, dtype=np.int8)
    ws = rng.uniform(0.005, 0.02, N if per_n else 1).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    want = o.gemm_dequant(q, s, M, K, w, N, ws, b, act, out_dt)
    layer = ops.Int8Linear(up(dev4, w, "I8", [N, K]), up(dev4, ws, "F32", [ws.size]), up(dev4, b, "F32", [N]) if bias else None)
    out = new(dev4, DTS[out_dt], [M, N])
    ops.int8_gemm_dequant(up(dev4, q, "I8", [M, K]), up(dev4, s, "F32", [M]), layer, act, out)
    if act == o.ACT_NONE or out_dt == o.F32:
        if act == o.ACT_NONE:
            assert_bits_equal(out.to_numpy(), want, "gemm split")
        else:
            rel, _ = o.compare(out.to_numpy().ravel(), np.asarray(want, np.float32).ravel())
            assert rel < 1e-5, f"gemm split silu f32: relative L2 {rel:.2e}"
    else:
        assert_close_16(out.to_numpy(), want, out_dt, "gemm split silu", max_frac=5e-3)


@pytest.mark.parametrize("group", [0, 256])
def test_int8_linear_split(dev4, group):
    """h3s_int8_linear (the quantizer, then the GEMM with its last tiles split) against the oracle, bit for bit."""
    M, K, N = 260, 12288, 600
    rng = np.random.default_rng(77 + group)
    x = o.to_bf16((0.7 * rng.standard_normal(M * K)).astype(np.float32))
    w = rng.integers(-127, 128, N * K, dtype=np.int8)
    ws = rng.uniform(0.005, 0.02, N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    want = o.int8_linear(x, o.BF16, M, K, w, N, ws, b, o.BF16, group)
    layer = ops.Int8Linear(up(dev4, w, "I8", [N, K]), up(dev4, ws, "F32", [N]), up(dev4, b, "F32", [N]), group or None)
    out = new(dev4, "BF16", [M, N])
    layer.forward(up(dev4, x, "BF16", [M, K]), out)
    assert_bits_equal(out.to_numpy(), want, "int8_linear split")


def mats(seed, M, K, N, dt):
    g = np.random.default_rng(seed)
    x = o.to_dt(g.standard_normal((M, K)).astype(np.float32), dt).ravel()
    w = o.to_dt((g.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32), dt).ravel()
    b = g.standard_normal(N).astype(np.float32)
    return x, w, b


def close(got, want, dt, what):
    if dt == o.F32:
        rel, _ = o.compare(np.asarray(got, np.float32).ravel(), np.asarray(want, np.float32).ravel())
        assert rel < 1e-5, f"{what}: relative L2 {rel:.2e}"
    else:
        assert_close_16(got, want, dt, what, max_frac=2e-2, abs_floor=2e-5)


@pytest.mark.parametrize("dt,out_dt", [(o.BF16, o.BF16), (o.BF16, o.F32), (o.F16, o.F16)])
@pytest.mark.parametrize("M,K,N", [(260, 6144, 600), (1100, 6176, 200)])
@pytest.mark.parametrize("bias", [False, True])
def test_linear_split(dev4, dt, out_dt, M, K, N, bias):
    x, w, b = mats(200 + K, M, K, N, dt)
    want = o.linear(x, dt, M, K, w, N, b if bias else None, out_dt=out_dt)
    out = new(dev4, DTS[out_dt], [M, N])
    layer = ops.Linear(up(dev4, w, DTS[dt], [N, K]), up(dev4, b, "F32", [N]) if bias else None)
    layer.forward(up(dev4, x, DTS[dt], [M, K]), out)
    close(out.to_numpy(), want, out_dt, "linear split")


@pytest.mark.parametrize("dt", [o.BF16, o.F16])
@pytest.mark.parametrize("M,K,N", [(260, 6144, 600), (1100, 6176, 200)])
def test_linear_acc_split(dev4, dt, M, K, N):
    x, w, b = mats(210 + K, M, K, N, dt)
    prev = o.to_dt(np.random.default_rng(211).standard_normal(M * N).astype(np.float32), dt)
    want = o.linear(x, dt, M, K, w, N, b, out_dt=dt, acc_into=prev)
    out = up(dev4, prev, DTS[dt], [M, N])
    ops.Linear(up(dev4, w, DTS[dt], [N, K]), up(dev4, b, "F32", [N])).forward_acc(up(dev4, x, DTS[dt], [M, K]), out)
    close(out.to_numpy(), want, dt, "linear_acc split")
