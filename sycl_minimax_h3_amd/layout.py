"""The token sequence of one denoiser call, host side: the mirror of engine/h3-core/src/layout.rs.

Which rows are text, conditioning, audio and video (segments); where each token sits in (time, height, width) for the
position rotation (positions, float64 [tokens, 3]); and each token's AdaLN table row (Timesteps.rows, int32 [tokens],
`timestep index * 3 + modality`). The arithmetic follows the reference's order and types: float64 for the positions,
float32 where the reference computes in float32 (the timestep keys, layout.rs:216-221, and the embedding curve,
layout.rs:240-252). Device work that follows from it - the rotation table and the AdaLN tables - is ops.rotations and
ops.adaln_tables.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from enum import Enum

import numpy as np

# layout.rs:13-19
FRAME_PER_TOKEN = (1.0, 4.0, 4.0, 4.0, 4.0)
FRAME_RESCALE = 5.0 / 3.0
VISUAL_COND_TIMESTEP = 0.999
AUDIO_COND_TIMESTEP = 1.0


class Kind(Enum):
    TEXT = "text"
    COND = "cond"              # video rows of a keyframe
    COND_AUDIO = "cond_audio"  # audio rows of a keyframe
    REF_AUDIO = "ref_audio"    # audio rows of a reference
    AUDIO = "audio"
    VIDEO = "video"

    def modality(self) -> int:
        """Which of a timestep's three table rows the kind uses: video-like 0, text 1, audio-like 2 (layout.rs:37-44)."""
        if self in (Kind.VIDEO, Kind.COND):
            return 0
        if self is Kind.TEXT:
            return 1
        return 2


@dataclass
class Keyframe:
    frame_index: float
    video_latent_t: int | None = None
    audio_latent_t: int | None = None


@dataclass
class RefAudio:
    t: int

    def span(self) -> float:
        return float(self.t)


@dataclass(frozen=True)
class Segment:
    start: int
    stop: int
    kind: Kind


def _axis(dim: int, sqrt_area: float) -> list[float]:
    """dim / 2 centred coordinates along one axis, a square frame spanning 32 (layout.rs:88-93)."""
    ratio = dim / sqrt_area
    n = dim // 2
    return [(i * (ratio / n) + (1.0 - ratio) / 2.0) * 32.0 for i in range(n)]


def _video_times(n: int, origin: float) -> list[float]:
    """Time coordinates of n latent frames from origin (layout.rs:96-106)."""
    out, t = [], origin
    for k in range(n):
        out.append(t)
        t += FRAME_RESCALE * FRAME_PER_TOKEN[k % 5]
    return out


@dataclass
class Layout:
    segments: list[Segment]
    positions: np.ndarray          # float64 [tokens, 3]
    frame_rows: int

    @staticmethod
    def new(text_len: int, latent_t: int, latent_h: int, latent_w: int, audio_t: int,
            keyframes: list[Keyframe] = (), refs: list[RefAudio] = ()) -> "Layout":
        """[text | keyframe conditioning | reference audio | audio | video] (layout.rs:108-176)."""
        if latent_h % 2 or latent_w % 2 or latent_h == 0 or latent_w == 0:
            raise ValueError(f"the video latent must have even height and width, got {latent_h} x {latent_w}")
        sqrt_area = math.sqrt(float(latent_h * latent_w))
        hs, ws = _axis(latent_h, sqrt_area), _axis(latent_w, sqrt_area)
        frame = [(h, w) for h in hs for w in ws]
        w_low, w_high = ws[0], ws[-1]
        segments: list[Segment] = []
        pos: list[tuple[float, float, float]] = []
        row = 0

        def push(kind: Kind, n: int):
            nonlocal row
            segments.append(Segment(row, row + n, kind))
            row += n

        def video(vt: int, origin: float):
            for t in _video_times(vt, origin):
                pos.extend((t, h, w) for h, w in frame)

        def audio(at: int, origin: float):
            for w in (w_low, w_high):            # channel-major: the left channel's frames, then the right's
                pos.extend((origin + float(i), 0.0, w) for i in range(at))

        pos.extend((float(i), 0.0, 0.0) for i in range(text_len))
        push(Kind.TEXT, text_len)
        cursor = float(text_len) + sum((r.span() for r in refs), 0.0)
        for kf in keyframes:
            at = cursor + FRAME_RESCALE * kf.frame_index
            if kf.video_latent_t is not None:
                video(kf.video_latent_t, at)
                push(Kind.COND, kf.video_latent_t * len(frame))
            if kf.audio_latent_t is not None:
                audio(kf.audio_latent_t, at)
                push(Kind.COND_AUDIO, kf.audio_latent_t * 2)
        rc = float(text_len)
        for r in refs:
            if r.t > 0:
                audio(r.t, rc)
                push(Kind.REF_AUDIO, r.t * 2)
            rc += r.span()
        audio(audio_t, cursor)
        push(Kind.AUDIO, audio_t * 2)
        video(latent_t, cursor)
        push(Kind.VIDEO, latent_t * len(frame))
        return Layout(segments, np.array(pos, dtype=np.float64).reshape(-1, 3), len(frame))

    def tokens(self) -> int:
        return self.segments[-1].stop if self.segments else 0

    def segment(self, kind: Kind) -> Segment | None:
        return next((s for s in self.segments if s.kind is kind), None)


def time_shift_sigma(sigma: float, from_shift: float, to_shift: float) -> float:
    """The audio stream's point of the same base schedule (layout.rs:187-191)."""
    base = sigma / (from_shift + sigma * (1.0 - from_shift))
    return to_shift * base / (1.0 + (to_shift - 1.0) * base)


@dataclass
class Timesteps:
    values: list[float]            # distinct timesteps (1 - noise level), ascending
    rows: np.ndarray               # int32 [tokens]: timestep index * 3 + modality
    video_index: int
    audio_index: int

    @staticmethod
    def new(layout: Layout, sigma_video: float, shift_video: float, shift_audio: float) -> "Timesteps":
        return Timesteps.with_cond(layout, sigma_video, shift_video, shift_audio, VISUAL_COND_TIMESTEP, AUDIO_COND_TIMESTEP)

    @staticmethod
    def with_cond(layout: Layout, sigma_video: float, shift_video: float, shift_audio: float, visual_cond: float,
                  audio_cond: float) -> "Timesteps":
        """layout.rs:212-236; the keys in float32 as the reference computes them."""
        f = np.float32
        sigma_v = max(f(sigma_video), f(1e-6))
        sv = f(shift_video)
        base = f(sigma_v / f(sv + f(sigma_v * f(f(1.0) - sv))))
        sa = f(shift_audio)
        sigma_a = f(f(sa * base) / f(f(1.0) + f(f(sa - f(1.0)) * base)))
        t_v, t_a = float(f(f(1.0) - sigma_v)), float(f(f(1.0) - sigma_a))

        def of(kind: Kind) -> float:
            if kind in (Kind.TEXT, Kind.VIDEO):
                return t_v
            if kind is Kind.AUDIO:
                return t_a
            if kind is Kind.COND:
                return max(t_v, visual_cond)
            return max(t_a, audio_cond)

        values = sorted(set([t_v, t_a] + [of(s.kind) for s in layout.segments]))
        index = {v: i for i, v in enumerate(values)}
        rows = np.zeros(layout.tokens(), dtype=np.int32)
        for s in layout.segments:
            rows[s.start:s.stop] = index[of(s.kind)] * 3 + s.kind.modality()
        return Timesteps(values, rows, index[t_v], index[t_a])

    def embeddings(self, table: np.ndarray, t_dim: int) -> np.ndarray:
        """Each timestep's point on the embedding curve: `grid` rows over [0, 1], linear interpolation in float32
        (layout.rs:240-252). float32 [len(values), t_dim]."""
        table = np.asarray(table, dtype=np.float32).reshape(-1, t_dim)
        grid = table.shape[0]
        f = np.float32
        out = []
        for t in self.values:
            pos = f(min(max(f(t), f(0.0)), f(1.0)) * f(grid - 1))
            i0 = min(int(math.floor(pos)), grid - 2)
            fr = f(pos - f(i0))
            a, b = table[i0], table[i0 + 1]
            out.append((a + fr * (b - a)).astype(np.float32))
        return np.stack(out).astype(np.float32)

