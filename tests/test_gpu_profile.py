"""H3S_PROFILE (kernels/h3sycl.cpp:117, 228, 1753-1760): a context opened with it set reports attention's time by
phase on each call and the int8 linear's time by pass when it is destroyed, on stderr, and computes the same results
as a context without it."""
import numpy as np
import pytest

from oracle import oracle as o
from helpers import new, up

pytestmark = pytest.mark.gpu

from sycl_minimax_h3_amd import Device, ops  # noqa: E402


def work(d):
    g = np.random.default_rng(90)
    M, K, N = 300, 256, 64
    x = o.to_bf16((0.7 * g.standard_normal(M * K)).astype(np.float32))
    w = g.integers(-127, 128, N * K).astype(np.int8)
    s = (0.01 + 0.001 * g.random(N)).astype(np.float32)
    lin = ops.Int8Linear(up(d, w, "I8", [N, K]), up(d, s, "F32", [N]))
    y = new(d, "BF16", [M, N])
    lin.forward(up(d, x, "BF16", [M, K]), y)
    S, H, D = 200, 2, 64
    q, k, v = (o.to_bf16(g.standard_normal(S * H * D).astype(np.float32)) for _ in range(3))
    qt, kt, vt = (up(d, a, "BF16", [S, H * D]) for a in (q, k, v))
    out = new(d, "F32", [S, H * D])
    ops.attention(*(ops.Rows(t, 0, H * D, S, H, D) for t in (qt, kt, vt)), out)
    return y.to_numpy(), out.to_numpy()


def test_profile_reports_and_changes_nothing(dev, monkeypatch, capfd):
    want = work(dev)
    capfd.readouterr()
    monkeypatch.setenv("H3S_PROFILE", "1")
    d = Device.open()
    try:
        got = work(d)
        err = capfd.readouterr().err
        assert "h3hip: attention (16-bit) S=200 H=2 D=64: preparation" in err and " ms, attention " in err, err
    finally:
        d.close()
    err = capfd.readouterr().err
    assert "h3hip: int8 linear, 1 row chunks: quantize" in err and "int8 GEMM" in err, err
    for a, b in zip(got, want):
        assert np.array_equal(a, b)
