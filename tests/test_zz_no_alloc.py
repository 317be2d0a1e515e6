"""h3s_int8_linear_noalloc (the int8 linear that allocates nothing: its quantized rows go into the library's fixed
device array) against h3s_int8_linear, bit for bit, through the C ABI: two calls in a row, the second smaller, so the
second reuses the array the first filled. The first call is longer than one chunk of the array (64 MiB of codes is
16384 rows of 4096 features), so the chunk loop runs. Neither call takes anything from the context's budget, nor
makes any allocation, event, stream or handle (the library's own count of them, h3s_alloc_count)."""
import numpy as np
import pytest

from oracle import oracle as o
from helpers import assert_bits_equal, new, up

pytestmark = pytest.mark.gpu

from sycl_minimax_h3_amd import Device, DType  # noqa: E402

DTS = {o.F32: DType.F32, o.BF16: DType.BF16}


@pytest.fixture(scope="module")
def ctx():
    d = Device.open()
    yield d
    d.close()


def call(dev, fn, xt, M, K, wt, N, wst, nws, bt, out, out_dt, group):
    dev.check(fn(dev.ctx, xt.ptr(), o.BF16, M, K, wt.ptr(), N, wst.ptr(), nws, bt.ptr() if bt is not None else None,
                 out.ptr(), out_dt, group))


@pytest.mark.parametrize("first,second", [((20000, 4096, 384, 256, False, False, o.BF16), (300, 1024, 128, 16, True, True, o.F32))])
def test_noalloc_matches_int8_linear(ctx, first, second):
    dev = ctx
    for i, (M, K, N, group, per_n, bias, out_dt) in enumerate((first, second)):
        print(f"noalloc call {i}: M={M} K={K} N={N} group={group}", flush=True)
        rng = np.random.default_rng(90 + i)
        x = o.to_bf16((0.7 * rng.standard_normal(M * K)).astype(np.float32))
        w = rng.integers(-127, 128, N * K, dtype=np.int8)
        ws = rng.uniform(0.005, 0.02, N if per_n else 1).astype(np.float32)
        b = rng.standard_normal(N).astype(np.float32) if bias else None
        xt, wt, wst = up(dev, x, "BF16", [M, K]), up(dev, w, "I8", [N, K]), up(dev, ws, "F32", [ws.size])
        bt = up(dev, b, "F32", [N]) if bias else None
        got, want = new(dev, DTS[out_dt], [M, N]), new(dev, DTS[out_dt], [M, N])
        used, made = dev.mem_used(), dev.api.alloc_count()
        call(dev, dev.api.int8_linear_noalloc, xt, M, K, wt, N, wst, ws.size, bt, got, out_dt, group)
        dev.wait()
        assert dev.mem_used() == used, "the allocation-free entry point took device memory"
        # no device or host allocation, event, stream or library handle was made on its path
        assert dev.api.alloc_count() == made, "the allocation-free entry point allocated"
        call(dev, dev.api.int8_linear, xt, M, K, wt, N, wst, ws.size, bt, want, out_dt, group)
        if i == 0:   # the counter sees allocations: the context's first int8 linear grows its scratch
            assert dev.api.alloc_count() > made, "h3s_int8_linear's first call on a fresh context allocated nothing"
        assert_bits_equal(got.to_numpy(), want.to_numpy(), f"noalloc call {i}")
