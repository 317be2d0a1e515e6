"""The host mirror of engine/h3-core/src/layout.rs against the reference's own fixture (the positions and table rows
of a real 384x288, 2 s pipeline call, kept as the compact table tests/golden/layout_384x288_2s.json), its unit tests
(layout.rs:262-312), and the step tables' oracle (dit.rs:155-203) pinned by closed forms."""
import json
import os

import numpy as np

from oracle import oracle as o
from sycl_minimax_h3_amd.layout import Keyframe, Kind, Layout, Timesteps, time_shift_sigma

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = json.load(open(os.path.join(HERE, "golden", "layout_384x288_2s.json")))


def fixture_layout():
    m = {k: int(v) for k, v in GOLD["metadata"].items() if k != "sigma"}
    return Layout.new(m["text_len"], m["latent_t"], m["latent_h"], m["latent_w"], m["audio_t"])


def test_layout_matches_the_reference():
    """layout.rs:265-281: segments, and positions within 1e-9 of the pipeline's (every axis's distinct values and
    their per-segment sums, and every 37th row)."""
    lay = fixture_layout()
    assert [(s.start, s.stop, s.kind.value) for s in lay.segments] == [tuple(x) for x in GOLD["segments"]]
    assert lay.tokens() == GOLD["tokens"]
    assert np.abs(lay.positions[::GOLD["sample_every"]] - np.array(GOLD["sample_rows"])).max() < 1e-9
    for a, b, name in GOLD["segments"]:
        for k in range(3):
            got = np.array(sorted(set(lay.positions[a:b, k].tolist())))
            want = np.array(GOLD["axis_values"][name][k])
            assert got.shape == want.shape and np.abs(got - want).max(initial=0.0) < 1e-9, (name, k)
            assert abs(lay.positions[a:b, k].sum() - GOLD["axis_sums"][name][k]) < 1e-9 * (b - a)


def test_table_rows_match_the_reference():
    """layout.rs:283-296: the first step has one timestep (0) and three table rows."""
    ts = Timesteps.new(fixture_layout(), 1.0, 12.0, 3.0)
    assert ts.values == [0.0]
    want = np.concatenate([np.full(n, r, np.int32) for r, n in GOLD["mod_rows_rle"]])
    assert np.array_equal(ts.rows, want)


def test_audio_schedule_and_curve():
    """layout.rs:298-312"""
    assert abs(time_shift_sigma(1.0, 12.0, 3.0) - 1.0) < 1e-12
    assert abs(time_shift_sigma(0.0, 12.0, 3.0)) < 1e-12
    assert time_shift_sigma(0.5, 12.0, 3.0) < 0.5
    table = np.arange(10, dtype=np.float32)
    ts = Timesteps.new(Layout.new(1, 1, 2, 2, 1), 1.0, 12.0, 3.0)
    ts.values = [0.375, 1.0]
    assert ts.embeddings(table, 2).ravel().tolist() == [3.0, 4.0, 8.0, 9.0]


def test_later_steps_and_keyframes():
    """A mid-schedule step: two timesteps (video, audio) and a keyframe conditioning block at 0.999."""
    lay = Layout.new(10, 3, 4, 6, 5, keyframes=[Keyframe(0.0, 1, None)])
    kinds = [s.kind for s in lay.segments]
    assert kinds == [Kind.TEXT, Kind.COND, Kind.AUDIO, Kind.VIDEO]
    assert lay.tokens() == 10 + 6 + 10 + 18 and lay.positions.shape == (44, 3)   # frames of 2 x 3 rows
    ts = Timesteps.new(lay, 0.5, 12.0, 3.0)
    assert len(ts.values) == 3 and ts.values == sorted(ts.values)
    cond = lay.segment(Kind.COND)
    assert ts.values[ts.rows[cond.start] // 3] == 0.999 and ts.rows[cond.start] % 3 == 0
    assert ts.rows[0] % 3 == 1 and ts.rows[lay.segment(Kind.AUDIO).start] % 3 == 2


def test_adaln_tables_oracle_closed_form():
    """With a one-hot embedding the sum is the one weight: table = b + w[:, k] exactly, which fixes the index map
    (o = mi 6 C + ci C + i into table ci, row r m + mi)."""
    R, td, m, C = 2, 5, 3, 4
    g = np.random.default_rng(80)
    w = g.standard_normal((6 * m * C, td)).astype(np.float32)
    b = g.standard_normal(6 * m * C).astype(np.float32)
    t = np.zeros((R, td), np.float32)
    t[0, 2] = 1.0
    t[1, 4] = 1.0
    out = o.adaln_tables(w.ravel(), b, t.ravel(), R, td, m, C).reshape(6, R * m, C)
    for r, k in ((0, 2), (1, 4)):
        for mi in range(m):
            for ci in range(6):
                rows = mi * 6 * C + ci * C + np.arange(C)
                assert np.array_equal(out[ci, r * m + mi], (b[rows] + w[rows, k]).astype(np.float32))
    # and a general embedding is the float32 sum in k order, within rounding of the exact dot product
    t = g.standard_normal((R, td)).astype(np.float32)
    out = o.adaln_tables(w.ravel(), b, t.ravel(), R, td, m, C).reshape(6, R * m, C)
    exact = (b[None, :] + t.astype(np.float64) @ w.T.astype(np.float64))            # [R, 6 m C]
    for r in range(R):
        for mi in range(m):
            for ci in range(6):
                rows = mi * 6 * C + ci * C + np.arange(C)
                assert np.allclose(out[ci, r * m + mi], exact[r, rows], rtol=1e-5, atol=1e-5)


def test_rotations_oracle():
    """cs = (cos, sin) of fl(pos * inv_freq) per axis in order; position 0 gives (1, 0) exactly."""
    S, n = 7, 5
    pos = np.random.default_rng(81).uniform(0, 200, (S, 3))
    pos[0] = 0.0
    inv = (1.0 / 10000.0 ** (np.arange(n) / n)).astype(np.float32)
    cs = o.rotations(pos, S, inv).reshape(S, 3, n, 2)
    ang = pos.astype(np.float32)[:, :, None] * inv[None, None, :]
    assert np.allclose(cs[..., 0], np.cos(ang.astype(np.float64)), atol=2e-7)
    assert np.allclose(cs[..., 1], np.sin(ang.astype(np.float64)), atol=2e-7)
    assert np.all(cs[0, :, :, 0] == 1.0) and np.all(cs[0, :, :, 1] == 0.0)
