"""Request geometry: from (aspect ratio, duration) to the latent token grid.

Tile plans and predictor bundles are keyed by a geometry name such as
'16x9_t37' and are valid only for the exact token grid that request
produces (the reference's rules are `miowtion/h3/geometry.py:12-169`). This
module states those rules as data:

  CanvasRule   the pixel canvas of an aspect ratio: the short edge at 768,
               the long edge from the ratio, the area capped at 768 x 1344
               (both edges shrunk by the same factor), each edge rounded to
               the nearest multiple of 32; ratios outside [1:4, 4:1] refused;
  FrameLadder  the frame counts the video VAE accepts, 17 n + 5, and their
               latent frame counts 5 n + 2 (rung n of the ladder);
  RequestRules the two plus the frame rate (24) and the token edge in pixels
               (32: VAE stride 16 times the 1x2x2 patch),

and `H3` is the rule set of the H3 model. The functions below keep the
reference's names so that callers and plan files read the same; only the
video side exists here (the audio latents play no part in the attention
path).
"""

from __future__ import annotations

import dataclasses
import math


@dataclasses.dataclass(frozen=True)
class CanvasRule:
    """The pixel canvas of an aspect ratio."""

    short_edge: int = 768
    pixel_budget: int = 768 * 1344   # fixed, whatever short edge is asked for
    multiple: int = 32
    widest: float = 4.0              # ratios in [1 / widest, widest]

    def snap(self, pixels: float) -> int:
        """Nearest multiple (Python rounding, at least one multiple)."""
        return max(self.multiple, self.multiple * int(round(float(pixels) / self.multiple)))

    def size(self, aspect_w: int, aspect_h: int, short_edge: int | None = None) -> tuple[int, int]:
        """(width, height) in pixels.

        Raises:
            ValueError: If the ratio is outside [1 / widest, widest].
        """
        edge = float(self.short_edge if short_edge is None else short_edge)
        ratio = float(aspect_w) / float(aspect_h)
        if ratio < 1.0 / self.widest or ratio > self.widest:
            raise ValueError(f'aspect {aspect_w}:{aspect_h} is outside 1:{self.widest:g} .. '
                             f'{self.widest:g}:1')
        dims = [edge * ratio, edge] if ratio >= 1.0 else [edge, edge / ratio]
        area = dims[0] * dims[1]
        if area > self.pixel_budget:
            shrink = math.sqrt(float(self.pixel_budget) / area)
            dims = [d * shrink for d in dims]
        return self.snap(dims[0]), self.snap(dims[1])


@dataclasses.dataclass(frozen=True)
class FrameLadder:
    """Rung n holds period * n + first frames and latent_step * n +
    latent_first latent frames."""

    period: int = 17
    first: int = 5
    latent_step: int = 5
    latent_first: int = 2

    def frames(self, rung: int) -> int:
        return self.period * rung + self.first

    def latent(self, rung: int) -> int:
        return self.latent_step * rung + self.latent_first

    def rung_up(self, frames: int) -> int:
        """The lowest rung with at least `frames` frames."""
        return max(0, -(-(int(frames) - self.first) // self.period))

    def rung_down(self, frames: int) -> int:
        """The highest rung with at most `frames` frames (rung 0 below it)."""
        return max(0, (int(frames) - self.first) // self.period)

    def rung_of_latent(self, latent_t: int) -> int:
        """Raises ValueError unless latent_t is latent_step * n + latent_first."""
        rung, rest = divmod(int(latent_t) - self.latent_first, self.latent_step)
        if rung < 0 or rest:
            raise ValueError(f'latent_t {latent_t} is not {self.latent_step} n + '
                             f'{self.latent_first}')
        return rung


@dataclasses.dataclass(frozen=True)
class Geometry:
    """A resolved request: canvas, frame count and the latent token grid."""

    aspect: str
    width: int
    height: int
    frame_count: int
    latent_t: int
    token_px: int = 32
    fps: int = 24

    @property
    def latent_h(self) -> int:
        return self.height // (self.token_px // 2)

    @property
    def latent_w(self) -> int:
        return self.width // (self.token_px // 2)

    @property
    def video_grid(self) -> tuple[int, int, int]:
        """Token grid (T, H, W) of the target video."""
        return self.latent_t, self.height // self.token_px, self.width // self.token_px

    @property
    def num_video_tokens(self) -> int:
        t, h, w = self.video_grid
        return t * h * w

    @property
    def duration_seconds(self) -> float:
        return self.frame_count / self.fps

    @property
    def name(self) -> str:
        """The key plans and bundles use, '<w>x<h>_t<latent_t>'."""
        return '%s_t%d' % (self.aspect.replace(':', 'x'), self.latent_t)


@dataclasses.dataclass(frozen=True)
class RequestRules:
    fps: int = 24
    canvas: CanvasRule = CanvasRule()
    ladder: FrameLadder = FrameLadder()
    token_px: int = 32

    def snap_frames(self, frames: int) -> int:
        """Requested frames snapped up onto the ladder (1 if none)."""
        return 1 if frames <= 0 else self.ladder.frames(self.ladder.rung_up(frames))

    def geometry(self, aspect: str, seconds: float, short_edge: int | None = None) -> Geometry:
        aw, ah = (int(x) for x in aspect.split(':'))
        width, height = self.canvas.size(aw, ah, short_edge)
        frames = self.snap_frames(int(round(float(seconds) * self.fps)))
        return Geometry(aspect, width, height, frames,
                        self.ladder.latent(self.ladder.rung_down(frames)), self.token_px, self.fps)

    def at_latent(self, aspect: str, latent_t: int, short_edge: int | None = None) -> Geometry:
        """The geometry of a request exactly as long as latent_t's rung."""
        frames = self.ladder.frames(self.ladder.rung_of_latent(latent_t))
        return self.geometry(aspect, frames / self.fps, short_edge)

    def reachable(self, min_seconds: float, max_seconds: float) -> list[int]:
        """latent_t of every rung whose duration lies in [min, max] seconds."""
        out, rung = [], 0
        while self.ladder.frames(rung) / self.fps <= max_seconds:
            if self.ladder.frames(rung) / self.fps >= min_seconds:
                out.append(self.ladder.latent(rung))
            rung += 1
        return out


H3 = RequestRules()
FPS = H3.fps
BASE_SHORT_EDGE = H3.canvas.short_edge
MAX_DURATION_SECONDS = 15.0


def resolve_canvas(aspect_w: int, aspect_h: int,
                   short_edge: int = BASE_SHORT_EDGE) -> tuple[int, int]:
    return H3.canvas.size(aspect_w, aspect_h, short_edge)


def align_frame_count(frame_count: int) -> int:
    return H3.snap_frames(frame_count)


def video_latent_t(frame_count: int) -> int:
    return H3.ladder.latent(H3.ladder.rung_down(frame_count))


def frame_count_from_latent_t(latent_t: int) -> int:
    return H3.ladder.frames(H3.ladder.rung_of_latent(latent_t))


def resolve_geometry(aspect: str, duration_seconds: float,
                     short_edge: int = BASE_SHORT_EDGE) -> Geometry:
    return H3.geometry(aspect, duration_seconds, short_edge)


def geometry_from_latent_t(aspect: str, latent_t: int,
                           short_edge: int = BASE_SHORT_EDGE) -> Geometry:
    return H3.at_latent(aspect, latent_t, short_edge)


def latent_t_ladder(min_seconds: float = 5.0,
                    max_seconds: float = MAX_DURATION_SECONDS) -> list[int]:
    return H3.reachable(min_seconds, max_seconds)
