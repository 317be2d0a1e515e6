"""GPU parity of the step tables (engine/h3-core/src/dit.rs:155-203) through the C ABI: h3s_adaln_tables bit for bit
against the oracle's restatement of Block::tables, and h3s_rotations on the fixture's own 2,159-token layout: equal to
the correctly rounded cos / sin, and within one ulp of the C library's cosf / sinf (which Rust's f32::cos / f32::sin
call, and which are not correctly rounded everywhere)."""
import json
import os

import numpy as np
import pytest

from oracle import oracle as o
from helpers import new, up
from sycl_minimax_h3_amd import DType, Error, ops
from sycl_minimax_h3_amd.layout import Request, place, plan, step_rows

pytestmark = pytest.mark.gpu
o.set_threads(8)
HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.parametrize("R,td,m,C", [(1, 256, 3, 4096), (2, 100, 2, 100), (3, 64, 1, 64), (1, 8, 3, 128)])
def test_adaln_tables(dev, R, td, m, C):
    g = np.random.default_rng(90 + td)
    w = (0.05 * g.standard_normal((6 * m * C, td))).astype(np.float32)
    b = (0.1 * g.standard_normal(6 * m * C)).astype(np.float32)
    t = g.standard_normal((R, td)).astype(np.float32)
    want = o.adaln_tables(w.ravel(), b, t.ravel(), R, td, m, C)
    out = new(dev, "F32", [6, R * m, C])
    ops.adaln_tables(up(dev, w, "F32", [6 * m * C, td]), up(dev, b, "F32", [6 * m * C]), up(dev, t, "F32", [R, td]), m, out)
    got = out.to_numpy().ravel()
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{bad.size} differ, first {bad[:5]}: {got[bad[:5]]} vs {want[bad[:5]]}"


def fixture_request():
    gold = json.load(open(os.path.join(HERE, "golden", "layout_384x288_2s.json")))
    m = {k: int(v) for k, v in gold["metadata"].items() if k != "sigma"}
    return Request(m["text_len"], m["latent_t"], m["latent_h"], m["latent_w"], m["audio_t"])


@pytest.mark.parametrize("req", [
    fixture_request(),
    Request(10, 3, 4, 6, 5, keyframes=[(0.0, 1, None), (7.5, 2, 3)], ref_audio=(4, 0, 2)),
    Request(0, 11, 46, 64, 0),                      # no text, no audio: 11 frames of 23 x 32 patches
    Request(300, 31, 48, 80, 62, keyframes=[(120.0, 1, 1)]),
])
def test_layout_on_the_device(dev, req):
    """h3s_layout: every position bit for bit as the oracle's restatement of Layout::new (layout.rs:107-176), and
    every table row the kind's row of the step"""
    segs = plan(req)
    st = step_rows([s.kind for s in segs], 0.4, 12.0, 3.0)
    pos, rows = place(dev, req, st.row_of_kind)
    want_pos, kinds = o.layout(req.text_len, req.latent_t, req.latent_h, req.latent_w, req.audio_t, req.keyframes,
                               req.ref_audio)
    got = pos.to_numpy()
    assert got.shape == want_pos.shape
    assert np.array_equal(got.view(np.int64), want_pos.view(np.int64))
    assert np.array_equal(rows.to_numpy(), st.row_of_kind[kinds])


def test_rotations_on_the_fixture_layout(dev):
    """the fixture's positions, placed on the device by h3s_layout, then h3s_rotations (rot_dim 126 = 6 x 21)"""
    req = fixture_request()
    pos, _ = place(dev, req)
    positions = pos.to_numpy()
    S, n = positions.shape[0], 21
    inv = (1.0 / np.power(np.float32(10000.0), np.arange(n, dtype=np.float32) / np.float32(n))).astype(np.float32)
    want = o.rotations(positions, S, inv)
    cs = new(dev, "F32", [S, 3 * n, 2])
    ops.rotations(pos, up(dev, inv, "F32", [n]), cs)
    got = cs.to_numpy().ravel()
    # the device rounds float64 cos / sin of the float argument once: the correctly rounded float32 values
    ang = (positions.astype(np.float32)[:, :, None] * inv[None, None, :]).astype(np.float64)
    cr = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32).ravel()
    assert np.array_equal(got.view(np.int32), cr.view(np.int32))
    # the C library's cosf / sinf (the reference's values) are within one ulp of them, equal in all but a few
    d = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert d.max() <= 1 and (d > 0).mean() < 2e-2, f"{int((d > 0).sum())} of {d.size} differ by one ulp"


def test_step_table_errors(dev):
    t = new(dev, "F32", [1, 8])
    with pytest.raises(Error):
        ops.adaln_tables(new(dev, "F32", [6 * 3 * 4, 8]), new(dev, "F32", [5]), t, 3, new(dev, "F32", [6, 3, 4]))
