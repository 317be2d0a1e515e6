"""The token layout and the step's table rows, on the CPU: the library's planner (h3s_layout_plan, host code) and the
oracle's restatement of Layout::new against the reference's own fixture (the positions and table rows of a real
384x288, 2 s pipeline call, kept as the compact table tests/golden/layout_384x288_2s.json) and against layout.rs's
unit tests (layout.rs:262-312); the step tables' oracle (dit.rs:155-203) pinned by closed forms."""
import json
import os

import numpy as np
import pytest

from oracle import oracle as o
from sycl_minimax_h3_amd.layout import Kind, Request, embeddings, plan, step_rows, time_shift_sigma, tokens

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = json.load(open(os.path.join(HERE, "golden", "layout_384x288_2s.json")))
NAMES = {"text": Kind.TEXT, "audio": Kind.AUDIO, "video": Kind.VIDEO}


def fixture_request():
    m = {k: int(v) for k, v in GOLD["metadata"].items() if k != "sigma"}
    return Request(m["text_len"], m["latent_t"], m["latent_h"], m["latent_w"], m["audio_t"])


def oracle_of(req):
    return o.layout(req.text_len, req.latent_t, req.latent_h, req.latent_w, req.audio_t, req.keyframes, req.ref_audio)


def test_plan_matches_the_reference_fixture():
    """layout.rs:265-277: three segments, 2,159 tokens"""
    segs = plan(fixture_request())
    assert [(s.start, s.stop, s.kind) for s in segs] == [(a, b, NAMES[n]) for a, b, n in GOLD["segments"]]
    assert tokens(fixture_request()) == GOLD["tokens"]


def test_oracle_positions_match_the_reference_fixture():
    """layout.rs:278-281: positions within 1e-9 of the pipeline's (every 37th row; every axis's distinct values and
    their sums per segment); the kinds follow the planner's segments"""
    pos, kinds = oracle_of(fixture_request())
    assert pos.shape == (GOLD["tokens"], 3)
    assert np.abs(pos[::GOLD["sample_every"]] - np.array(GOLD["sample_rows"])).max() < 1e-9
    for a, b, name in GOLD["segments"]:
        assert np.all(kinds[a:b] == NAMES[name])
        for k in range(3):
            got = np.array(sorted(set(pos[a:b, k].tolist())))
            want = np.array(GOLD["axis_values"][name][k])
            assert got.shape == want.shape and np.abs(got - want).max(initial=0.0) < 1e-9, (name, k)
            assert abs(pos[a:b, k].sum() - GOLD["axis_sums"][name][k]) < 1e-9 * (b - a)


def test_step_rows_match_the_reference_fixture():
    """layout.rs:283-296: the first step has one timestep (0) and three table rows"""
    segs = plan(fixture_request())
    st = step_rows([s.kind for s in segs], 1.0, 12.0, 3.0)
    assert st.values == [0.0]
    want = np.concatenate([np.full(n, r, np.int32) for r, n in GOLD["mod_rows_rle"]])
    got = np.concatenate([np.full(s.stop - s.start, st.row_of_kind[s.kind], np.int32) for s in segs])
    assert np.array_equal(got, want)


def test_audio_schedule_and_curve():
    """layout.rs:298-312"""
    assert abs(time_shift_sigma(1.0, 12.0, 3.0) - 1.0) < 1e-12
    assert abs(time_shift_sigma(0.0, 12.0, 3.0)) < 1e-12
    assert time_shift_sigma(0.5, 12.0, 3.0) < 0.5
    table = np.arange(10, dtype=np.float32)
    assert embeddings([0.375, 1.0], table, 2).ravel().tolist() == [3.0, 4.0, 8.0, 9.0]


def test_keyframes_and_references():
    """A keyframe's video block and reference voices: the planner's segments and the oracle's rows agree, and a
    mid-schedule step gives the conditioning rows their presentation timestep (0.999 for video)"""
    req = Request(10, 3, 4, 6, 5, keyframes=[(0.0, 1, None), (7.5, 2, 3)], ref_audio=(4, 0, 2))
    segs = plan(req)
    assert [s.kind for s in segs] == [Kind.TEXT, Kind.COND, Kind.COND, Kind.COND_AUDIO, Kind.REF_AUDIO, Kind.REF_AUDIO,
                                      Kind.AUDIO, Kind.VIDEO]
    frame = (4 // 2) * (6 // 2)
    assert [s.stop - s.start for s in segs] == [10, frame, 2 * frame, 6, 8, 4, 10, 3 * frame]
    pos, kinds = oracle_of(req)
    assert pos.shape[0] == segs[-1].stop
    for s in segs:
        assert np.all(kinds[s.start:s.stop] == s.kind)
    # the targets start after the text and the references: 10 + 4 + 0 + 2
    assert pos[segs[-1].start, 0] == 16.0 and pos[segs[-2].start, 0] == 16.0
    # the second reference starts after the first (and the empty one)
    assert pos[segs[5].start, 0] == 14.0
    # keyframe at frame 7.5 sits 7.5 x 5/3 after the targets' start
    assert pos[segs[2].start, 0] == 16.0 + 5.0 / 3.0 * 7.5
    st = step_rows([s.kind for s in segs], 0.5, 12.0, 3.0)
    assert len(st.values) == 4 and st.values == sorted(st.values)
    assert st.values[st.row_of_kind[Kind.COND] // 3] == 0.999 and st.row_of_kind[Kind.COND] % 3 == 0
    assert st.values[st.row_of_kind[Kind.REF_AUDIO] // 3] == 1.0 and st.row_of_kind[Kind.REF_AUDIO] % 3 == 2
    assert st.row_of_kind[Kind.TEXT] % 3 == 1 and st.row_of_kind[Kind.AUDIO] % 3 == 2


def test_plan_refuses_an_odd_latent():
    with pytest.raises(ValueError, match="even"):
        plan(Request(4, 2, 5, 6, 1))


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
