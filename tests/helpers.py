"""Helpers shared by the tests: uploads, bit comparisons of 16-bit floats, and the parity tolerance for results
through transcendental functions (relative error 1e-3, one unit in the last place on few elements)."""
import numpy as np

from oracle import oracle as o

DT = {o.F32: "F32", o.F16: "F16", o.BF16: "BF16"}


def up(dev, arr, dtype, shape):
    from sycl_minimax_h3_amd import DType, Tensor

    return Tensor.from_numpy(dev, DType[dtype] if isinstance(dtype, str) else dtype, shape, np.ascontiguousarray(arr))


def new(dev, dtype, shape):
    from sycl_minimax_h3_amd import DType, Tensor

    return Tensor.new(dev, DType[dtype] if isinstance(dtype, str) else dtype, shape)


def ordered(bits: np.ndarray, dt: int) -> np.ndarray:
    """16-bit float patterns (or float32 values) as integers in the order of the values they stand for."""
    if dt == o.F32:
        b = np.ascontiguousarray(bits, dtype=np.float32).view(np.int32).astype(np.int64)
        return np.where(b < 0, -(b & 0x7FFFFFFF), b)
    b = np.ascontiguousarray(bits, dtype=np.uint16).astype(np.int64)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def ulp_diff(a, b, dt) -> np.ndarray:
    return np.abs(ordered(a, dt) - ordered(b, dt))


def assert_bits_equal(got, want, what=""):
    got, want = np.asarray(got).ravel(), np.asarray(want).ravel()
    assert got.shape == want.shape, f"{what}: shapes {got.shape} {want.shape}"
    if got.dtype.kind == "f":   # float32 values: NaN matches NaN
        diff = (got != want) & ~(np.isnan(got) & np.isnan(want))
    else:                       # integer codes and 16-bit float patterns: the bits
        diff = got != want
    bad = np.flatnonzero(diff)
    assert bad.size == 0, f"{what}: {bad.size} of {got.size} differ, first at {bad[:8]}: got {got[bad[:8]]} want {want[bad[:8]]}"


def assert_close_16(got, want, dt, what="", max_ulp=1, max_frac=1e-3, rel_l2=1e-3, abs_floor=1e-6):
    """The parity bar for outputs through a transcendental function: at most max_ulp units in the last place apart
    (or within abs_floor, for results that cancel to near zero), on at most max_frac of the elements, and the
    relative L2 error of reference::compare below rel_l2."""
    got, want = np.asarray(got).ravel(), np.asarray(want).ravel()
    d = ulp_diff(got, want, dt)
    fg, fw = o.from_dt(got, dt), o.from_dt(want, dt)
    near = np.abs(fg.astype(np.float64) - fw.astype(np.float64)) <= abs_floor
    bad = (d > max_ulp) & ~near
    assert not bad.any(), f"{what}: {int(bad.sum())} elements more than {max_ulp} ulp apart, e.g. {fg[bad][:5]} vs {fw[bad][:5]}"
    frac = float((d > 0).mean())
    assert frac <= max_frac, f"{what}: {frac:.2e} of the elements differ (bar {max_frac})"
    rel, cos = o.compare(fg, fw)
    assert rel < rel_l2, f"{what}: relative L2 error {rel:.2e}"


def codes_close(got_q, want_q, what=""):
    """int8 codes: identical, except |delta| = 1 at an exact rounding tie (none are expected: the kernels follow the
    oracle's order), never |delta| >= 2."""
    d = np.abs(np.asarray(got_q, dtype=np.int32).ravel() - np.asarray(want_q, dtype=np.int32).ravel())
    assert d.max(initial=0) <= 1, f"{what}: a code differs by {d.max()}"
    assert int((d > 0).sum()) == 0, f"{what}: {int((d > 0).sum())} codes differ by 1"
