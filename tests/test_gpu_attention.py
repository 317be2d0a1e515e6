"""GPU parity of h3s_attention / h3s_attention_batch (kernels/h3sycl.cpp:1433-1917) against the oracle's restatement:
the int8 (SageAttention) form and the 16-bit form, through the C ABI. The reference's kernels are third-party (Intel's
ARK, oneDNN) and their rounding inside the softmax is not restated, so the bar is the parity tolerance on the result:
relative L2 below 1e-3 against the oracle's float64 softmax of the same quantized operands."""
import os

import numpy as np
import pytest

from oracle import oracle as o
from helpers import new, up

pytestmark = pytest.mark.gpu

from sycl_minimax_h3_amd import DType, Device, Error, Tensor, ops  # noqa: E402

DTS = {o.F32: DType.F32, o.F16: DType.F16, o.BF16: DType.BF16}
o.set_threads(8)


def _open_with(env):
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return Device.open()
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


@pytest.fixture(scope="module")
def dev_sage():
    """A context that takes the int8 form at every length (H3S_SAGE_MIN_S=0)."""
    d = _open_with({"H3S_SAGE_MIN_S": "0"})
    yield d
    d.close()


@pytest.fixture(scope="module")
def dev_sage4():
    """The int8 form at every length with grids sized for 4 compute units (H3S_CUS=4): k's mean then takes 32
    features a block wherever 16 would make more than 4 blocks."""
    d = _open_with({"H3S_SAGE_MIN_S": "0", "H3S_CUS": "4"})
    yield d
    d.close()


@pytest.fixture(scope="module")
def dev_16():
    """A context that keeps every call on the 16-bit form (H3S_ATTN=onednn)."""
    d = _open_with({"H3S_ATTN": "onednn"})
    yield d
    d.close()


def qkv(seed, S, H, D, dt, stride, spread=1.0):
    g = np.random.default_rng(seed)
    mk = lambda: o.to_dt((g.standard_normal((S, stride)) * spread).astype(np.float32), dt).ravel()  # noqa: E731
    return mk(), mk(), mk()


def run(d, q, k, v, dt, S, H, D, stride, out_dt):
    qt, kt, vt = (up(d, a, DTS[dt], [S, stride]) for a in (q, k, v))
    out = new(d, DTS[out_dt], [S, H * D])
    ops.attention(ops.Rows(qt, 0, stride, S, H, D), ops.Rows(kt, 0, stride, S, H, D), ops.Rows(vt, 0, stride, S, H, D), out)
    return out.to_numpy().ravel()


def check(got, want, out_dt, what):
    g, w = o.from_dt(got, out_dt).astype(np.float32), o.from_dt(want, out_dt).astype(np.float32)
    assert np.isfinite(g).all(), f"{what}: non-finite outputs"
    rel, cos = o.compare(g, w)
    assert rel < 1e-3 and cos > 0.99999, f"{what}: relative L2 {rel:.2e}, cos {cos:.7f}"


@pytest.mark.parametrize("sage", [True, False])
@pytest.mark.parametrize("dt,out_dt", [(o.BF16, o.BF16), (o.F16, o.F32), (o.F32, o.BF16)])
@pytest.mark.parametrize("S,H,D,pad", [(64, 1, 128, 0), (130, 3, 128, 16), (257, 2, 64, 0), (1000, 2, 128, 8), (77, 4, 64, 24)])
def test_attention(dev_sage, dev_16, sage, dt, out_dt, S, H, D, pad):
    stride = H * D + pad
    q, k, v = qkv(60 + S, S, H, D, dt, stride)
    want = o.attention(q, k, v, dt, S, H, D, stride, out_dt=out_dt, sage=sage)
    want = want[0] if sage else want
    got = run(dev_sage if sage else dev_16, q, k, v, dt, S, H, D, stride, out_dt)
    check(got, want, out_dt, f"{'int8' if sage else '16-bit'} S={S} H={H} D={D}")


@pytest.mark.parametrize("sage", [True, False])
@pytest.mark.parametrize("S,pad", [(1, 0), (63, 2), (65, 0), (200, 6), (129, 1)])
def test_attention_edges(dev_sage, dev_16, sage, S, pad):
    """One token, tiles cut short by one key either side of 64, and row strides that are not whole 16-byte vectors
    (the element-wise preparation)."""
    H, D = 2, 64
    stride = H * D + pad
    q, k, v = qkv(75 + S, S, H, D, o.BF16, stride)
    want = o.attention(q, k, v, o.BF16, S, H, D, stride, out_dt=o.F32, sage=sage)
    want = want[0] if sage else want
    got = run(dev_sage if sage else dev_16, q, k, v, o.BF16, S, H, D, stride, o.F32)
    check(got, want, o.F32, f"edge S={S} pad={pad}")


@pytest.mark.parametrize("sage", [True, False])
def test_attention_peaked_and_shifted(dev_sage, dev_16, sage):
    """Large score spreads (the online max moves a lot, most weights underflow) and a large common offset in k (the
    int8 form takes k's mean out)."""
    S, H, D = 300, 2, 128
    q, k, v = qkv(70, S, H, D, o.BF16, H * D, spread=4.0)
    k = o.to_dt(o.from_dt(k, o.BF16) + 3.0, o.BF16)
    want = o.attention(q, k, v, o.BF16, S, H, D, out_dt=o.F32, sage=sage)
    want = want[0] if sage else want
    got = run(dev_sage if sage else dev_16, q, k, v, o.BF16, S, H, D, H * D, o.F32)
    check(got, want, o.F32, "peaked")


@pytest.mark.parametrize("blocks", ["16", "32"])
@pytest.mark.parametrize("dt", [o.BF16, o.F16, o.F32])
@pytest.mark.parametrize("S,H,D", [(1, 2, 128), (191, 1, 64), (192, 2, 64), (384, 1, 128), (385, 2, 128),
                                   (2017, 3, 64), (5000, 1, 64)])
def test_attention_kmean(request, blocks, dt, S, H, D):
    """k's mean (h3sycl.cpp:1732-1737), seen through the output. A per-feature constant taken from k moves all of a
    query's scores alike and the softmax cancels it, so in ordinary inputs a wrong mean only shows through the
    quantization. Here each feature of k is a large power of two C_f plus or minus C_f 2^-7 in pairs of rows of
    opposite sign: the float32 sum in token order is exact and the mean is C_f, so k - mean is +-C_f 2^-7. A mean
    that misses one row then moves the output by a relative L2 of about 8e-2 (a CPU model of the scores from the
    oracle's quantizer), a missed chunk or mixed-up features by 0.15 to 1. Lengths around the 384- and 192-row
    chunks of the 16-bit and float32 inputs, and past the eight-chunk ring. blocks "32": a context sized for 4 CUs,
    where the mean takes 32 features a block (its chunks of 192 and 96 rows) for every case of 128 features or more."""
    dev_sage = request.getfixturevalue("dev_sage" if blocks == "16" else "dev_sage4")
    if blocks == "32" and (H * D) // 16 <= 4:
        pytest.skip("16 features a block already fit the 4 CUs")
    stride = H * D
    g = np.random.default_rng(S + 7 * H)
    q = o.to_dt(g.standard_normal((S, stride)).astype(np.float32), dt).ravel()
    C = 2.0 ** ((10 if dt == o.F16 else 14) + g.integers(0, 4, stride))          # C (1 +- 2^-7) exact in every type
    sgn = g.choice([-1.0, 1.0], (S // 2, stride))
    e = np.zeros((S, stride))
    e[0:2 * (S // 2):2], e[1:2 * (S // 2):2] = sgn, -sgn
    k = o.to_dt((C * (1.0 + e * 2.0 ** -7)).astype(np.float32), dt).ravel()
    v = o.to_dt(g.standard_normal((S, stride)).astype(np.float32), dt).ravel()
    want, _, _, _, _, km = o.attention(q, k, v, dt, S, H, D, stride, out_dt=o.F32, sage=True)
    assert np.array_equal(km, C.astype(np.float32)), "the oracle's mean is the constant"
    got = run(dev_sage, q, k, v, dt, S, H, D, stride, o.F32)
    check(got, want, o.F32, f"k mean S={S} H={H} D={D}")


@pytest.fixture(scope="module")
def dev_split():
    """Contexts for the pipelined kernel's split of a short last round, per form: no split (H3S_ATTN_SPLIT=1), the
    default, and the default with grids sized for 16 or 12 compute units (H3S_CUS), so that a few hundred tokens
    make full rounds and a split last one (at 12, full blocks that the XCD renumbering leaves in order)."""
    modes = {"none": {"H3S_ATTN_SPLIT": "1"}, "default": {}, "cus16": {"H3S_CUS": "16"}, "cus12": {"H3S_CUS": "12"}}
    ds = {}
    for sage in (True, False):
        form = {"H3S_SAGE_MIN_S": "0"} if sage else {"H3S_ATTN": "onednn"}
        for name, env in modes.items():
            ds[(sage, name)] = _open_with({**form, **env})
    yield ds
    for d in ds.values():
        d.close()


@pytest.mark.parametrize("sage", [True, False])
@pytest.mark.parametrize("mode", ["none", "default", "cus16", "cus12"])
@pytest.mark.parametrize("S,H", [(64, 1), (777, 3), (2000, 5)])
def test_attention_split_last_round(dev_split, sage, mode, S, H):
    """Heads of 128 features (the pipelined kernel). The grids: 64 tokens, one block of one key tile (never split);
    777 tokens x 3 heads, 12 blocks of 13 tiles (split 7 ways on 256 CUs, not at all on 16 or 12); 2000 x 5, 40 blocks
    of 32 tiles (6 ways on 256 CUs; on 16, 32 full blocks and 8 split in 2; on 12, 36 full blocks and 4 split in
    3). The split blocks' partial sums are merged by attn_merge_kernel."""
    D = 128
    stride = H * D
    q, k, v = qkv(90 + S, S, H, D, o.BF16, stride)
    want = o.attention(q, k, v, o.BF16, S, H, D, stride, out_dt=o.BF16, sage=sage)
    want = want[0] if sage else want
    got = run(dev_split[(sage, mode)], q, k, v, o.BF16, S, H, D, stride, o.BF16)
    check(got, want, o.BF16, f"{'int8' if sage else '16-bit'} {mode} S={S} H={H}")


@pytest.mark.parametrize("sage", [True, False])
@pytest.mark.parametrize("per_tile", [12.0, 30.0])
def test_attention_rising_scores(dev_sage, dev_16, sage, per_tile):
    """Scores that rise along the keys by about per_tile (base 2) every 64 keys: at 12 the weights stay inside half's
    range while the running reference lags behind the max; at 30 every tile passes the reference by more than half's
    range (the int8 kernel's overflow path: the max, the rescale, the weights again)."""
    S, H, D = 640, 2, 128
    g = np.random.default_rng(71)
    ramp = (np.arange(S, dtype=np.float32) / 64.0 * per_tile / (np.sqrt(D) * np.log2(np.e)))[:, None]
    q = o.to_dt((1.0 + 0.05 * g.standard_normal((S, H * D))).astype(np.float32), o.BF16).ravel()
    k = o.to_dt((ramp + 0.05 * g.standard_normal((S, H * D))).astype(np.float32), o.BF16).ravel()
    v = o.to_dt(g.standard_normal((S, H * D)).astype(np.float32), o.BF16).ravel()
    want = o.attention(q, k, v, o.BF16, S, H, D, out_dt=o.F32, sage=sage)
    want = want[0] if sage else want
    got = run(dev_sage if sage else dev_16, q, k, v, o.BF16, S, H, D, H * D, o.F32)
    check(got, want, o.F32, f"rising scores, {per_tile} a tile")


def test_attention_default_form_by_length(dev):
    """The default context: below 8192 tokens the 16-bit form, from 8192 on the int8 form (kernels/h3sycl.cpp:138, 1773)."""
    H, D = 1, 64
    for S, sage in ((500, False), (8200, True)):
        q, k, v = qkv(71, S, H, D, o.BF16, H * D)
        want = o.attention(q, k, v, o.BF16, S, H, D, out_dt=o.BF16, sage=sage)
        want = want[0] if sage else want
        other = o.attention(q, k, v, o.BF16, S, H, D, out_dt=o.BF16, sage=not sage)
        other = other[0] if not sage else other
        got = run(dev, q, k, v, o.BF16, S, H, D, H * D, o.BF16)
        check(got, want, o.BF16, f"default S={S}")
        # and it is measurably the form named, not the other one
        rg, _ = o.compare(o.from_dt(got, o.BF16), o.from_dt(want, o.BF16))
        ro, _ = o.compare(o.from_dt(got, o.BF16), o.from_dt(other, o.BF16))
        assert rg < ro, f"S={S}: closer to the other form ({rg:.2e} vs {ro:.2e})"


def test_attention_batch(dev_16):
    B, S, H, D = 3, 96, 2, 64
    stride = H * D
    q, k, v = qkv(72, B * S, H, D, o.BF16, stride)
    qt, kt, vt = (up(dev_16, a, "BF16", [B * S, stride]) for a in (q, k, v))
    out = new(dev_16, "BF16", [B * S, H * D])
    ops.attention_batch(ops.Rows(qt, 0, stride, B * S, H, D), ops.Rows(kt, 0, stride, B * S, H, D),
                        ops.Rows(vt, 0, stride, B * S, H, D), B, out)
    got = out.to_numpy().reshape(B, S * H * D)
    for b in range(B):
        sl = slice(b * S * stride, (b + 1) * S * stride)
        want = o.attention(q[sl], k[sl], v[sl], o.BF16, S, H, D, out_dt=o.BF16, sage=False)
        check(got[b], want, o.BF16, f"sequence {b}")


@pytest.mark.parametrize("dt", [o.F16, o.BF16, o.F32])
@pytest.mark.parametrize("L,Hq,Hkv,D", [(1, 2, 1, 128), (37, 8, 2, 128), (130, 4, 4, 64), (300, 6, 2, 128), (257, 8, 1, 64)])
def test_attention_causal(dev, dt, L, Hq, Hkv, D):
    """The text encoder's causal attention with grouped kv heads (kernels/h3sycl.cpp:873-898), q and kv in buffers of
    wider rows."""
    qs, kvs = Hq * D + 8, 2 * Hkv * D
    g = np.random.default_rng(97 + L)
    q = o.to_dt(g.standard_normal(L * qs).astype(np.float32), dt)
    kv = o.to_dt(g.standard_normal(L * kvs).astype(np.float32), dt)
    k, v = kv, kv[Hkv * D:]                                           # k and v interleaved in one buffer
    want = o.attention_causal(q, k, v, dt, L, Hq, Hkv, D, qs, kvs)
    qt, kvt = up(dev, q, DTS[dt], [L, qs]), up(dev, kv, DTS[dt], [L, kvs])
    out = new(dev, DTS[dt], [L, Hq * D])
    ops.attention_causal(ops.Rows(qt, 0, qs, L, Hq, D), ops.Rows(kvt, 0, kvs, L, Hkv, D), ops.Rows(kvt, Hkv * D, kvs, L, Hkv, D), out)
    check(out.to_numpy().ravel(), want, dt, f"causal L={L} Hq={Hq} Hkv={Hkv}")


def test_attention_refuses(dev):
    p = new(dev, "BF16", [64, 600])
    with pytest.raises(Error, match="at most 256"):
        ops.attention(ops.Rows(p, 0, 600, 64, 2, 300), ops.Rows(p, 0, 600, 64, 2, 300), ops.Rows(p, 0, 600, 64, 2, 300), p)


@pytest.mark.parametrize("sage", [True, False])
@pytest.mark.parametrize("S,H,D,pad,out_dt", [(200, 2, 256, 0, o.BF16), (130, 3, 96, 0, o.F32), (77, 2, 80, 8, o.BF16),
                                               (65, 2, 32, 0, o.F16), (150, 1, 200, 2, o.F32), (64, 2, 7, 1, o.BF16),
                                               (300, 1, 130, 0, o.BF16)])
def test_attention_head_sizes(dev_sage, dev_16, sage, S, H, D, pad, out_dt):
    """Heads of any size up to 256: 256 in its own kernel, the others zero-padded to 64, 128 or 256 features in the
    preparation and stored at their own size (odd sizes one feature at a time). The int8 form is the reference's only
    at 64 and 128 features (kernels/h3sycl.cpp:1706): on a context that asks for it at every length (dev_sage), these
    head sizes still take the 16-bit form and match the 16-bit oracle."""
    stride = H * D + pad
    q, k, v = qkv(110 + D, S, H, D, o.BF16, stride)
    assert D not in (64, 128)
    want = o.attention(q, k, v, o.BF16, S, H, D, stride, out_dt=out_dt, sage=False)
    got = run(dev_sage if sage else dev_16, q, k, v, o.BF16, S, H, D, stride, out_dt)
    check(got, want, out_dt, f"16-bit ({'a context asking for int8' if sage else 'default'}) S={S} H={H} D={D}")
    if sage:
        # and not the int8 form's result: its quantization moves the output far past the parity bar
        int8 = o.attention(q, k, v, o.BF16, S, H, D, stride, out_dt=out_dt, sage=True)[0]
        rel, _ = o.compare(o.from_dt(got, out_dt).astype(np.float32), o.from_dt(int8, out_dt).astype(np.float32))
        assert rel > 1e-3, f"S={S} D={D}: the result is the int8 form's (relative L2 {rel:.2e} from it)"


@pytest.mark.parametrize("dt", [o.BF16, o.F32])
@pytest.mark.parametrize("L,Hq,Hkv,D", [(50, 4, 2, 256), (129, 2, 1, 80), (33, 6, 3, 200), (70, 2, 2, 36)])
def test_attention_causal_head_sizes(dev, dt, L, Hq, Hkv, D):
    """The causal form at the head sizes the reference takes (D <= 256, kernels/h3sycl.cpp:877)."""
    qs, kvs = Hq * D, 2 * Hkv * D
    g = np.random.default_rng(131 + D)
    q = o.to_dt(g.standard_normal(L * qs).astype(np.float32), dt)
    kv = o.to_dt(g.standard_normal(L * kvs).astype(np.float32), dt)
    want = o.attention_causal(q, kv, kv[Hkv * D:], dt, L, Hq, Hkv, D, qs, kvs)
    qt, kvt = up(dev, q, DTS[dt], [L, qs]), up(dev, kv, DTS[dt], [L, kvs])
    out = new(dev, DTS[dt], [L, Hq * D])
    ops.attention_causal(ops.Rows(qt, 0, qs, L, Hq, D), ops.Rows(kvt, 0, kvs, L, Hkv, D), ops.Rows(kvt, Hkv * D, kvs, L, Hkv, D), out)
    check(out.to_numpy().ravel(), want, dt, f"causal L={L} Hq={Hq} Hkv={Hkv} D={D}")
