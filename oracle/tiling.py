"""Oracle: 3D tile permutation of a packed sequence (CPU torch, test-only).

Restates `miowtion/veda/tiling.py` of the reference:
  * tile shapes and padding          -> tiling.py:43-105
  * span_tiles (argsort compaction)  -> tiling.py:122-136
  * contiguous_span_tiles            -> tiling.py:139-156
  * build_tile_layout                -> tiling.py:214-275
  * gather_tiles / scatter_tiles_    -> tiling.py:278-312
The permutation is produced the way the reference produces it (a padded grid
of row ids, a block transpose, a stable sort of padding to the back), so it
is an independent statement from the closed form the product uses.
"""

from __future__ import annotations

import dataclasses
import math

import torch

TILE = 128


@dataclasses.dataclass(frozen=True, order=True)
class Shape:
    t: int
    h: int
    w: int

    def __post_init__(self):
        if self.t * self.h * self.w != TILE:
            raise ValueError(f'{self} is not a {TILE}-token tile')

    @staticmethod
    def parse(text: str) -> 'Shape':
        t, h, w = (int(v) for v in text.split('x'))
        return Shape(t, h, w)

    def padded(self, grid):
        # tiling.py:67-69: every extent rounded up to a multiple of the shape.
        return tuple(math.ceil(g / s) * s for g, s in zip(grid, (self.t, self.h, self.w)))

    def count(self, grid) -> int:
        tp, hp, wp = self.padded(grid)
        return tp * hp * wp // TILE

    def spread(self) -> float:
        return max(self.t, self.h, self.w) / min(self.t, self.h, self.w)


def shape_menu() -> list[Shape]:
    """tiling.py:85-92 -- every power-of-two (t, h, w) with product 128."""
    out = []
    for a in range(8):
        for b in range(8 - a):
            out.append(Shape(2 ** a, 2 ** b, 2 ** (7 - a - b)))
    return sorted(out)


def least_padding(grid) -> Shape:
    """tiling.py:95-105: fewest tiles, then most cubic, then lexicographic."""
    fits = [s for s in shape_menu() if s.t <= grid[0] and s.h <= grid[1] and s.w <= grid[2]]
    return min(fits or shape_menu(), key=lambda s: (s.count(grid), s.spread(), (s.t, s.h, s.w)))


@dataclasses.dataclass(frozen=True)
class Span:
    start: int
    grid: tuple
    shape: Shape

    @property
    def rows(self) -> int:
        return self.grid[0] * self.grid[1] * self.grid[2]


def span_tiles(span: Span) -> torch.Tensor:
    """[n_tiles, 128] row ids, -1 on padding (tiling.py:122-136).

    Tiles are ordered h-block, w-block, t-block (outer to inner); a tile's
    rows are t, h, w row-major and then its real rows are moved, stably, to
    the front.
    """
    T, Hh, W = span.grid
    st, sh, sw = span.shape.t, span.shape.h, span.shape.w
    tp, hp, wp = span.shape.padded(span.grid)
    ids = torch.full((tp, hp, wp), -1, dtype=torch.long)
    ids[:T, :Hh, :W] = span.start + torch.arange(T * Hh * W).view(T, Hh, W)
    blocks = ids.view(tp // st, st, hp // sh, sh, wp // sw, sw)
    # (t-block, t, h-block, h, w-block, w) -> (h-block, w-block, t-block, t, h, w)
    blocks = blocks.permute(2, 4, 0, 1, 3, 5).reshape(-1, TILE)
    pad_last = torch.argsort((blocks < 0).to(torch.int8), dim=1, stable=True)
    return torch.gather(blocks, 1, pad_last)


def contiguous_span_tiles(span: Span) -> torch.Tensor:
    """tiling.py:139-156: the span cut in sequence order, padding at the end."""
    n = math.ceil(span.rows / TILE)
    flat = torch.full((n * TILE,), -1, dtype=torch.long)
    flat[:span.rows] = span.start + torch.arange(span.rows)
    return flat.view(n, TILE)


@dataclasses.dataclass
class Layout:
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
        return self.n_tiles * TILE


def build_layout(spans, used: int, seq_len: int, tiler=span_tiles) -> Layout:
    """tiling.py:214-275: video tiles of every span (refs first, target last),
    then the uncovered real rows of [0, used) chunked by 128 in order."""
    if not spans:
        raise ValueError('at least the target span must be tiled')
    covered = torch.zeros(used, dtype=torch.bool)
    parts, stop = [], 0
    for sp in spans:
        if sp.start < stop or sp.start + sp.rows > used:
            raise ValueError(f'span {sp} overlaps or exceeds used={used}')
        stop = sp.start + sp.rows
        covered[sp.start:stop] = True
        parts.append(tiler(sp))
    video = torch.cat(parts)
    glob = torch.nonzero(~covered).view(-1)
    n_glob = math.ceil(glob.numel() / TILE)
    gt = torch.full((n_glob * TILE,), -1, dtype=torch.long)
    gt[:glob.numel()] = glob
    perm = torch.cat([video.view(-1), gt])
    vc = (perm.view(-1, TILE) >= 0).sum(1).to(torch.int32)
    return Layout(
        perm=perm, valid_count=vc, n_video_tiles=video.shape[0],
        n_ref_tiles=sum(p.shape[0] for p in parts[:-1]), n_global_tiles=n_glob,
        ref_tokens=sum(s.rows for s in spans[:-1]), target_tokens=spans[-1].rows,
        used=used, seq_len=seq_len,
        gather_index=perm.clamp(min=0),
        scatter_index=torch.where(perm < 0, torch.full_like(perm, seq_len), perm),
        pad_slots=torch.nonzero(perm < 0).view(-1),
        partial_tiles=torch.nonzero((vc > 0) & (vc < TILE)).view(-1),
        kv_ok=vc > 0, full_tile=vc == TILE,
        slot_valid=(perm >= 0).to(torch.int32))


def gather_tiles(x: torch.Tensor, lay: Layout, heads) -> torch.Tensor:
    """tiling.py:278-297: [S, H, D] -> [N, H', D], padding slots zero."""
    if heads is None:
        out = x.index_select(0, lay.gather_index)
    else:
        out = x[lay.gather_index[:, None], heads[None, :]]
    if lay.pad_slots.numel():
        out.index_fill_(0, lay.pad_slots, 0)
    return out


def scatter_tiles_(out: torch.Tensor, tiled: torch.Tensor, lay: Layout, heads) -> None:
    """tiling.py:300-312: [N, H', D] back into out[S + 1, H, D]."""
    if out.shape[0] != lay.seq_len + 1:
        raise ValueError(f'scatter buffer needs {lay.seq_len + 1} rows')
    if heads is None:
        out.index_copy_(0, lay.scatter_index, tiled)
    else:
        out[lay.scatter_index[:, None], heads[None, :]] = tiled


def gather_lse(lse: torch.Tensor, lay: Layout, heads) -> torch.Tensor:
    """`miowtion/veda/attention.py:299-305`: [S, H] -> [N, H'], 0 on padding."""
    out = lse[lay.gather_index[:, None], heads[None, :]]
    if lay.pad_slots.numel():
        out.index_fill_(0, lay.pad_slots, 0.0)
    return out
