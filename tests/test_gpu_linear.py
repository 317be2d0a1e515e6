"""GPU parity of the plain linear layers (kernels/h3sycl.cpp:656-739) through the C ABI against the oracle's float64
products: h3s_linear, h3s_linear_acc (row chunks included) and h3s_scale_rows. The reference's products are oneDNN's,
whose accumulation order is not restated: the parity tolerance (relative L2 < 1e-3, one ulp of the output type).
bfloat16 and half operands with K a multiple of 32 run on the matrix-core kernel (256 x 256 tiles: partial tiles at
every edge, K steps of 64 elements with a last half step where K is an odd multiple of 32, the long-K tile order
from K = 6144; launches of few tiles split along K: 2000 x 1024 -> 64 or 100, 8 tiles in 8 parts each); K = 200 and
float32 operands run on rocBLAS with the separate epilogue."""
import numpy as np
import pytest

from oracle import oracle as o
from helpers import assert_bits_equal, assert_close_16, new, up
from sycl_minimax_h3_amd import DType, ops

pytestmark = pytest.mark.gpu
o.set_threads(8)
DTS = {o.F32: DType.F32, o.F16: DType.F16, o.BF16: DType.BF16}


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
        # float32 accumulation: results that cancel to near zero carry the error of the terms (~1e-6 here)
        assert_close_16(got, want, dt, what, max_frac=2e-2, abs_floor=2e-5)


@pytest.mark.parametrize("dt,out_dt", [(o.BF16, o.BF16), (o.BF16, o.F32), (o.F16, o.F16), (o.F32, o.F32), (o.F32, o.BF16)])
@pytest.mark.parametrize("M,K,N", [(37, 256, 130), (300, 1024, 520), (8200, 64, 48), (1000, 2048, 700), (513, 6144, 300),
                                   (600, 200, 90), (257, 96, 256), (2000, 1024, 64), (2000, 1024, 100)])
@pytest.mark.parametrize("bias", [False, True])
def test_linear(dev, dt, out_dt, M, K, N, bias):
    x, w, b = mats(100 + K, M, K, N, dt)
    want = o.linear(x, dt, M, K, w, N, b if bias else None, out_dt=out_dt)
    out = new(dev, DTS[out_dt], [M, N])
    layer = ops.Linear(up(dev, w, DTS[dt], [N, K]), up(dev, b, "F32", [N]) if bias else None)
    layer.forward(up(dev, x, DTS[dt], [M, K]), out)
    close(out.to_numpy(), want, out_dt, "linear")


@pytest.mark.parametrize("M,K,N", [(8300, 128, 64), (700, 1024, 600), (300, 96, 260), (130, 200, 70)])
@pytest.mark.parametrize("dt", [o.BF16, o.F16, o.F32])
def test_linear_acc(dev, dt, M, K, N):
    x, w, b = mats(110, M, K, N, dt)
    prev = o.to_dt(np.random.default_rng(111).standard_normal(M * N).astype(np.float32), dt)
    want = o.linear(x, dt, M, K, w, N, b, out_dt=dt, acc_into=prev)
    out = up(dev, prev, DTS[dt], [M, N])
    ops.Linear(up(dev, w, DTS[dt], [N, K]), up(dev, b, "F32", [N])).forward_acc(up(dev, x, DTS[dt], [M, K]), out)
    close(out.to_numpy(), want, dt, "linear_acc")


@pytest.mark.parametrize("dt", [o.BF16, o.F16, o.F32])
def test_scale_rows(dev, dt):
    N, K = 77, 200
    x, w, b = mats(120, 1, K, N, dt)
    s = np.random.default_rng(121).standard_normal(N).astype(np.float32)
    want = o.scale_rows(w, dt, N, K, s)
    layer = ops.Linear(up(dev, w, DTS[dt], [N, K]), up(dev, b, "F32", [N]))
    layer.scale_outputs(up(dev, s, "F32", [N]))
    assert_bits_equal(layer.weight.to_numpy(), want, "scale_rows")
    assert np.array_equal(layer.bias.to_numpy(), (b * s).astype(np.float32))
