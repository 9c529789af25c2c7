"""Tile permutations of a packed sequence into 128-token 3D tiles.

Host mirror of the reference's `miowtion/veda/tiling.py` (same names, same
argument meaning, same errors), built from a closed form instead of a sort:
for tile (hb, wb, tb) of a span with valid extents (vt, vh, vw) -- the box
clipped to the grid -- slot i < vt*vh*vw holds the row at local
(i // (vh*vw), (i // vw) % vh, i % vw) and every later slot is padding.
That is exactly the reference's "t, h, w row-major, then stably compacted to
the front" order (tiling.py:122-136), computed without an argsort.

The layout is built once per (spans, shape) on the host and its tensors are
moved to the device once (tiling.py:159-211 keeps the same cache contract);
gather / scatter of activations are the HIP kernels in `miowtion_amd.kernels`.
"""

from __future__ import annotations

import dataclasses
import itertools
import math
import weakref
from collections.abc import Callable, Sequence

import numpy as np
import torch

TILE_SIZE = 128


@dataclasses.dataclass(frozen=True, order=True)
class TileShape:
    """A (t, h, w) box of 128 tokens (tiling.py:43-82)."""

    t: int
    h: int
    w: int

    def __post_init__(self):
        if self.t * self.h * self.w != TILE_SIZE:
            raise ValueError(f'tile {self} does not hold {TILE_SIZE} tokens')

    def __str__(self) -> str:
        return f'{self.t}x{self.h}x{self.w}'

    @classmethod
    def parse(cls, text: str) -> 'TileShape':
        t, h, w = (int(v) for v in text.split('x'))
        return cls(t, h, w)

    def transposed(self) -> 'TileShape':
        return TileShape(self.t, self.w, self.h)

    def padded_grid(self, grid: Sequence[int]) -> tuple[int, int, int]:
        return tuple(-(-g // s) * s for g, s in zip(grid, (self.t, self.h, self.w)))

    def num_tiles(self, grid: Sequence[int]) -> int:
        tp, hp, wp = self.padded_grid(grid)
        return tp * hp * wp // TILE_SIZE

    def padding_ratio(self, grid: Sequence[int]) -> float:
        t, h, w = grid
        return self.num_tiles(grid) * TILE_SIZE / (t * h * w) - 1.0

    def aspect_spread(self) -> float:
        return max(self.t, self.h, self.w) / min(self.t, self.h, self.w)


def all_shapes() -> list[TileShape]:
    """The 36 power-of-two triples with product 128 (tiling.py:85-92)."""
    e = TILE_SIZE.bit_length() - 1
    return sorted(TileShape(2 ** i, 2 ** j, 2 ** (e - i - j))
                  for i, j in itertools.product(range(e + 1), repeat=2) if i + j <= e)


def candidate_shapes(grid: Sequence[int]) -> list[TileShape]:
    return [s for s in all_shapes() if s.t <= grid[0] and s.h <= grid[1] and s.w <= grid[2]]


def least_padding_shape(grid: Sequence[int]) -> TileShape:
    """Least padding; ties: most cubic, then lexicographic (tiling.py:101-105)."""
    return min(candidate_shapes(grid) or all_shapes(),
               key=lambda s: (s.num_tiles(grid), s.aspect_spread(), (s.t, s.h, s.w)))


@dataclasses.dataclass(frozen=True)
class TiledSpan:
    """Packed rows [start, start + T*H*W) tiled with `shape` (tiling.py:108-119)."""

    start: int
    grid: tuple[int, int, int]
    shape: TileShape

    @property
    def num_rows(self) -> int:
        t, h, w = self.grid
        return t * h * w


def span_tiles(span: TiledSpan) -> torch.Tensor:
    """[n_tiles, 128] packed row ids of one span, -1 on padding.

    Tile order is (h-block, w-block, t-block), outer to inner; the real rows
    of a tile are its clipped box in t, h, w row-major order, as a prefix.
    """
    T, H, W = span.grid
    st, sh, sw = span.shape.t, span.shape.h, span.shape.w
    nt, nh, nw = -(-T // st), -(-H // sh), -(-W // sw)
    hb, wb, tb = np.meshgrid(np.arange(nh), np.arange(nw), np.arange(nt), indexing='ij')
    hb, wb, tb = hb.reshape(-1, 1), wb.reshape(-1, 1), tb.reshape(-1, 1)
    vt = np.minimum(st, T - tb * st)
    vh = np.minimum(sh, H - hb * sh)
    vw = np.minimum(sw, W - wb * sw)
    i = np.arange(TILE_SIZE)[None, :]
    lt, lh, lw = i // (vh * vw), (i // vw) % vh, i % vw
    rows = span.start + ((tb * st + lt) * H + (hb * sh + lh)) * W + (wb * sw + lw)
    rows = np.where(i < vt * vh * vw, rows, -1)
    return torch.from_numpy(rows.astype(np.int64))


def contiguous_span_tiles(span: TiledSpan) -> torch.Tensor:
    """The span cut in sequence order (tiling.py:139-156)."""
    n = -(-span.num_rows // TILE_SIZE)
    i = np.arange(n * TILE_SIZE)
    rows = np.where(i < span.num_rows, span.start + i, -1)
    return torch.from_numpy(rows.astype(np.int64).reshape(n, TILE_SIZE))


@dataclasses.dataclass
class TileLayout:
    """One permutation of the packed sequence and its derived constants
    (tiling.py:159-211; same attributes, all on `device`)."""

    perm: torch.Tensor
    valid_count: torch.Tensor
    n_video_tiles: int
    n_ref_tiles: int
    n_global_tiles: int
    ref_tokens: int
    target_tokens: int
    used: int
    seq_len: int
    gather_index: torch.Tensor
    scatter_index: torch.Tensor
    pad_slots: torch.Tensor
    partial_tiles: torch.Tensor
    kv_ok: torch.Tensor
    full_tile: torch.Tensor
    slot_valid: torch.Tensor

    @property
    def n_tiles(self) -> int:
        return self.n_video_tiles + self.n_global_tiles

    @property
    def num_slots(self) -> int:
        return self.n_tiles * TILE_SIZE


# Small tensors derived from a layout (per-tile log counts, an identity
# index), keyed by the layout object's identity and dropped when it is
# collected. The layout itself carries only the reference's fields, so a
# layout built by the reference's own builder works here unchanged (its
# dataclass is unhashable, hence the identity key).
_DERIVED: dict[int, dict[str, torch.Tensor]] = {}


def layout_cached(layout, key: str, build: Callable[[], torch.Tensor]) -> torch.Tensor:
    """The tensor `build()` for this layout object, built on first use and
    kept until the layout is garbage collected."""
    entry = _DERIVED.get(id(layout))
    if entry is None:
        entry = _DERIVED[id(layout)] = {}
        weakref.finalize(layout, _DERIVED.pop, id(layout), None)
    hit = entry.get(key)
    if hit is None:
        hit = entry[key] = build()
    return hit


def build_tile_layout(spans: Sequence[TiledSpan], used: int, seq_len: int,
                      device: torch.device | str = 'cpu',
                      tiler: Callable[[TiledSpan], torch.Tensor] = span_tiles) -> TileLayout:
    """Permutation of tiled spans (refs first, target last) followed by the
    remaining real rows of [0, used) chunked by 128 (tiling.py:214-275).

    Raises:
        ValueError: If spans overlap, are out of order or exceed `used`.
    """
    if not spans:
        raise ValueError('at least the target span must be tiled')
    covered = np.zeros(used, dtype=bool)
    parts = []
    prev_stop = 0
    for span in spans:
        if span.start < prev_stop or span.start + span.num_rows > used:
            raise ValueError(f'span {span} overlaps or exceeds used={used}')
        prev_stop = span.start + span.num_rows
        covered[span.start:prev_stop] = True
        parts.append(tiler(span).numpy())
    video = np.concatenate(parts).reshape(-1)
    glob = np.flatnonzero(~covered)
    n_global = -(-glob.size // TILE_SIZE)
    gtiles = np.full(n_global * TILE_SIZE, -1, dtype=np.int64)
    gtiles[:glob.size] = glob
    perm = np.concatenate([video, gtiles])
    vc = (perm.reshape(-1, TILE_SIZE) >= 0).sum(1).astype(np.int32)

    def dev(a) -> torch.Tensor:
        return torch.from_numpy(np.ascontiguousarray(a)).to(device)

    return TileLayout(
        perm=dev(perm), valid_count=dev(vc),
        n_video_tiles=video.size // TILE_SIZE,
        n_ref_tiles=sum(p.shape[0] for p in parts[:-1]),
        n_global_tiles=n_global,
        ref_tokens=sum(s.num_rows for s in spans[:-1]),
        target_tokens=spans[-1].num_rows, used=used, seq_len=seq_len,
        gather_index=dev(np.maximum(perm, 0)),
        scatter_index=dev(np.where(perm < 0, seq_len, perm)),
        pad_slots=dev(np.flatnonzero(perm < 0).astype(np.int64)),
        partial_tiles=dev(np.flatnonzero((vc > 0) & (vc < TILE_SIZE)).astype(np.int64)),
        kv_ok=dev(vc > 0), full_tile=dev(vc == TILE_SIZE),
        slot_valid=dev((perm >= 0).astype(np.int32)))


def _heads(x: torch.Tensor, heads: torch.Tensor | None) -> torch.Tensor:
    if heads is None:
        return torch.arange(x.shape[1], device=x.device)
    return heads


def gather_tiles(x: torch.Tensor, layout: TileLayout, heads: torch.Tensor | None) -> torch.Tensor:
    """[S, H, D] -> [N, H', D] in tile order, padding slots zero
    (tiling.py:278-297); the HIP gather kernel."""
    from miowtion_amd import ops
    return ops.gather(x, layout.gather_index, layout.slot_valid, layout.valid_count,
                      _heads(x, heads), True, False, False)[0]


def scatter_tiles_(out: torch.Tensor, tiled: torch.Tensor, layout: TileLayout,
                   heads: torch.Tensor | None) -> None:
    """Writes tile-ordered rows back into out[S + 1, H, D] (tiling.py:300-312);
    padding slots are dropped instead of landing in row S."""
    from miowtion_amd import ops
    if out.shape[0] != layout.seq_len + 1:
        raise ValueError(f'scatter buffer needs {layout.seq_len + 1} rows')
    ops.scatter_(out, tiled, layout.scatter_index, layout.slot_valid, _heads(out, heads))
