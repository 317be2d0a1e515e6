"""The token layout of one denoiser call and the AdaLN table rows of a sampler step, over the library.

The sequence of one call is [text | keyframe conditioning | reference audio | audio | video]
(engine/h3-core/src/layout.rs:1-9). The library owns it through the C ABI:
  - ``plan(req)``: its segments (start, stop, kind), from h3s_layout_plan (host code of the library, no GPU);
  - ``place(dev, req, rows)``: each token's position (time, height, width) as float64 [tokens, 3], and its table
    row as int32 [tokens], written on the device by h3s_layout. The positions feed h3s_rotations (dit.rs:188-203),
    the rows every modulated norm of the step.
What stays on the host is the few float32 numbers a step fixes (layout.rs:205-252):
  - ``step_rows(...)``: the step's distinct timesteps (1 - noise level), ascending, and the table row each kind of
    token reads: timestep index * 3 + modality (video-like 0, text 1, audio-like 2);
  - ``embeddings(...)``: each timestep's point on the model's embedding curve (linear interpolation in float32).
"""
from __future__ import annotations

import ctypes as C
import enum
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np

from . import api as _api


class Kind(enum.IntEnum):
    """A token's kind: the codes of include/h3hip.h (H3S_TOK_*), as layout.rs:21-32 lists them."""

    TEXT = 0
    COND = 1          # video rows of a keyframe
    COND_AUDIO = 2    # audio rows of a keyframe
    REF_AUDIO = 3     # audio rows of a reference voice
    AUDIO = 4
    VIDEO = 5

    @property
    def modality(self) -> int:
        """which of a timestep's three table rows the kind reads (layout.rs:35-42)"""
        return {Kind.VIDEO: 0, Kind.COND: 0, Kind.TEXT: 1}.get(self, 2)


class _Keyframe(C.Structure):
    _fields_ = [("frame_index", C.c_double), ("video_latent_t", C.c_int64), ("audio_latent_t", C.c_int64)]


@dataclass(frozen=True)
class Request:
    """What fixes a call's layout: the text length, the video latent [latent_t, latent_h, latent_w] (two latent
    pixels a token along height and width), the audio latent frames (two rows each, one per stereo channel), the
    keyframes to condition on as (frame index in pixel frames, video latent frames or None, audio latent frames or
    None), and the reference voices' audio latent frames."""

    text_len: int
    latent_t: int
    latent_h: int
    latent_w: int
    audio_t: int
    keyframes: Sequence[tuple] = field(default_factory=tuple)
    ref_audio: Sequence[int] = field(default_factory=tuple)

    def _args(self):
        kf = (_Keyframe * max(1, len(self.keyframes)))(*[
            _Keyframe(float(i), -1 if v is None else int(v), -1 if a is None else int(a)) for i, v, a in self.keyframes])
        refs = (C.c_int64 * max(1, len(self.ref_audio)))(*[int(r) for r in self.ref_audio])
        keep = (kf, refs)
        return keep, (self.text_len, self.latent_t, self.latent_h, self.latent_w, self.audio_t, C.cast(kf, C.c_void_p),
                      len(self.keyframes), C.cast(refs, C.c_void_p), len(self.ref_audio))


@dataclass(frozen=True)
class Segment:
    start: int
    stop: int
    kind: Kind


def plan(req: Request) -> list[Segment]:
    """The segments of the call's sequence, in row order (h3s_layout_plan)."""
    a = _api.load()
    keep, args = req._args()
    n = a.layout_plan(*args, None, None, None, 0)
    if n < 0:
        raise ValueError(a.error())
    starts, stops, kinds = (C.c_int64 * n)(), (C.c_int64 * n)(), (C.c_int32 * n)()
    a.layout_plan(*args, C.cast(starts, C.c_void_p), C.cast(stops, C.c_void_p), C.cast(kinds, C.c_void_p), n)
    del keep
    return [Segment(int(starts[i]), int(stops[i]), Kind(int(kinds[i]))) for i in range(n)]


def tokens(req: Request) -> int:
    segs = plan(req)
    return segs[-1].stop if segs else 0


def place(dev, req: Request, row_of_kind=None):
    """Positions float64 [tokens, 3] and, with row_of_kind (the table row of each Kind, e.g. StepRows.row_of_kind),
    table rows int32 [tokens], on dev (h3s_layout). Returns (positions, rows or None) as Tensors."""
    from .device import DType, Tensor

    n = tokens(req)
    pos = Tensor.new(dev, DType.F64, [n, 3])
    rows = Tensor.new(dev, DType.I32, [n]) if row_of_kind is not None else None
    rk = None
    if row_of_kind is not None:
        rk = (C.c_int32 * 6)(*[int(v) for v in row_of_kind])
    keep, args = req._args()
    dev.check(dev.api.layout(dev.ctx, *args, C.cast(rk, C.c_void_p) if rk is not None else None, pos.ptr(),
                             rows.ptr() if rows is not None else None, n))
    del keep
    return pos, rows


# layout.rs:17-19: the timesteps conditioning rows are presented at (almost clean video, clean audio)
VISUAL_COND_TIMESTEP = 0.999
AUDIO_COND_TIMESTEP = 1.0


def time_shift_sigma(sigma: float, from_shift: float, to_shift: float) -> float:
    """The same point of the base noise schedule under another shift (layout.rs:187-191), float64."""
    base = sigma / (from_shift + sigma * (1.0 - from_shift))
    return to_shift * base / (1.0 + (to_shift - 1.0) * base)


@dataclass
class StepRows:
    values: list              # the step's distinct timesteps, ascending (float64 values of float32 keys)
    row_of_kind: np.ndarray   # int32 [6]: the table row each Kind reads (-1 for a kind the layout does not have)
    video_index: int          # index in values of the target video's timestep (and of the target audio's)
    audio_index: int


def step_rows(kinds: Sequence[Kind], sigma_video: float, shift_video: float, shift_audio: float,
              visual_cond: float = VISUAL_COND_TIMESTEP, audio_cond: float = AUDIO_COND_TIMESTEP) -> StepRows:
    """The rows of a step for a layout whose segments have `kinds` (layout.rs:205-236). The video's noise level is
    floored at 1e-6; the audio's is the video's mapped from one schedule shift to the other. Both are computed in
    float32, as the reference computes them, because they are table keys; a conditioning kind takes the larger of
    its stream's timestep and its own presentation timestep."""
    f = np.float32
    sv = max(f(sigma_video), f(1e-6))
    base = f(sv / f(f(shift_video) + f(sv * f(f(1.0) - f(shift_video)))))
    sa = f(f(f(shift_audio) * base) / f(f(1.0) + f(f(f(shift_audio) - f(1.0)) * base)))
    t_video, t_audio = float(f(f(1.0) - sv)), float(f(f(1.0) - sa))
    stream = {Kind.TEXT: t_video, Kind.VIDEO: t_video, Kind.AUDIO: t_audio, Kind.COND: max(t_video, visual_cond),
              Kind.COND_AUDIO: max(t_audio, audio_cond), Kind.REF_AUDIO: max(t_audio, audio_cond)}
    values = sorted({t_video, t_audio, *(stream[k] for k in kinds)})
    where = {v: i for i, v in enumerate(values)}
    # a kind with no segment in the layout has no timestep among the values, and no token reads its row: -1
    row_of_kind = np.array([where[stream[k]] * 3 + k.modality if stream[k] in where else -1 for k in Kind], dtype=np.int32)
    return StepRows(values, row_of_kind, where[t_video], where[t_audio])


def embeddings(values: Sequence[float], table: np.ndarray, t_dim: int) -> np.ndarray:
    """Each timestep's point on the embedding curve, float32 [len(values), t_dim] (layout.rs:240-252): the table
    holds `grid` rows over t in [0, 1]; t is clamped, scaled by grid - 1, and read between its two rows."""
    tab = np.asarray(table, dtype=np.float32).reshape(-1, t_dim)
    grid = tab.shape[0]
    f = np.float32
    out = np.empty((len(values), t_dim), np.float32)
    for n, t in enumerate(values):
        x = f(f(min(max(f(t), f(0.0)), f(1.0))) * f(grid - 1))
        lo = min(int(np.floor(x)), grid - 2)
        frac = f(x - f(lo))
        out[n] = (tab[lo] + frac * (tab[lo + 1] - tab[lo])).astype(np.float32)
    return out
