"""Block masks from tile scores: equal-cost budgets, Bresenham rounding,
forced diagonal, top-k on the GPU.

Host mirror of `miowtion/veda/mask.py` (rules 1-7 of its docstring, :1-22).
The budget arithmetic stays on the host in Python floats / fp64, exactly as
the reference computes it (mask.py:61-93), because the kept counts depend on
its rounding; the per-row top-k, the block mask and the index lists run as
HIP kernels (`veda::select_topk`, `veda::dense_block_mask`,
`veda::index_lists`).

Tie order of the top-k: higher score first, lower column first on exactly
equal scores. `torch.topk` (the reference) returns the same result whenever
the scores at the cut are distinct; its order among exact ties is
backend-defined.
"""

from __future__ import annotations

import dataclasses
import functools
import math

import numpy as np
import torch

from miowtion_amd import ops
from miowtion_amd import tiling


@dataclasses.dataclass(frozen=True)
class Budget:
    """Keep budget of one column block: a ratio or an absolute tile count
    (mask.py:38-65)."""

    ratio: float | None = None
    tiles: float | None = None

    def __post_init__(self):
        if (self.ratio is None) == (self.tiles is None):
            raise ValueError('set exactly one of ratio / tiles')
        value = self.ratio if self.tiles is None else self.tiles
        if value <= 0:
            raise ValueError(f'budget must be positive: {self}')

    @property
    def keeps_all(self) -> bool:
        return self.ratio is not None and self.ratio >= 1.0

    def per_row(self, real_tokens: int, n_tiles: int) -> float:
        """ratio * n_ideal * n_ideal / n_tiles, evaluated left to right."""
        if self.tiles is not None:
            return float(self.tiles)
        n_ideal = math.ceil(real_tokens / tiling.TILE_SIZE)
        return self.ratio * n_ideal * n_ideal / n_tiles


def split_budget(budget: float, n_cols: int) -> tuple[int, int, float]:
    """(k_lo, k_hi, frac), 1 <= k_lo <= k_hi <= n_cols (mask.py:68-76).

    frac is rounded to 12 decimals so that e.g. 2.3 - 2 is 0.3 exactly.
    """
    if budget >= n_cols:
        return n_cols, n_cols, 0.0
    k_lo = min(max(1, math.floor(budget)), n_cols)
    frac = round(min(max(budget - k_lo, 0.0), 1.0), 12)
    return k_lo, min(k_lo + 1, n_cols), frac


@functools.lru_cache(maxsize=256)
def _bresenham(n_rows: int, frac: float, device: str) -> torch.Tensor:
    r = np.arange(n_rows + 1, dtype=np.float64) * frac
    ramp = np.floor(r)
    extra = ramp[1:] > ramp[:-1]
    return torch.from_numpy(extra).to(device)


def bresenham_extra(n_rows: int, frac: float, device: torch.device | str) -> torch.Tensor:
    """[n_rows] bool: row r keeps k_hi iff floor((r+1) f) > floor(r f), fp64
    (mask.py:79-93). Cached per device and shared read-only."""
    return _bresenham(n_rows, float(frac), str(torch.device(device)))


@dataclasses.dataclass(frozen=True)
class ColumnBlock:
    start: int
    stop: int
    budget: Budget
    real_tokens: int


def column_blocks(layout: tiling.TileLayout, target_budget: Budget,
                  ref_budget: Budget | None = None) -> list[ColumnBlock]:
    """Target block, preceded by a reference block when references are tiled
    (mask.py:106-120)."""
    target = ColumnBlock(layout.n_ref_tiles, layout.n_video_tiles, target_budget,
                         layout.target_tokens)
    if layout.n_ref_tiles == 0:
        return [target]
    if ref_budget is None:
        raise ValueError('tiled references need their own budget')
    return [ColumnBlock(0, layout.n_ref_tiles, ref_budget, layout.ref_tokens), target]


@dataclasses.dataclass
class Selection:
    """index [H', R, K] int64 global key tile ids; keep [H', R, K] bool."""

    index: torch.Tensor
    keep: torch.Tensor


@torch.no_grad()
def select_video_blocks(scores: torch.Tensor, layout: tiling.TileLayout,
                        blocks: list[ColumnBlock], rows: torch.Tensor | None = None,
                        rule: str = 'topk') -> Selection:
    """Top-k over the video quadrant of `scores` (mask.py:200-285, rule 'topk').

    Args:
        scores: [H', R, >= n_video] fp32 block scores of query tiles `rows`.
        layout: Tile layout.
        blocks: Column blocks from column_blocks().
        rows: [R] int64 video query tile ids; None means all n_video tiles.

    Raises:
        ValueError: On a rule other than 'topk', or scores not restricted to
            `rows`.
        NotImplementedError: For CPU tensors (the kernels are GPU-only).
    """
    if rule != 'topk':
        raise ValueError(f"rule must be 'topk' (the threshold rule is a Sol ablation): {rule!r}")
    heads = scores.shape[0]
    n_video = layout.n_video_tiles
    device = scores.device
    if rows is None:
        rows = torch.arange(n_video, device=device)
    num_rows = rows.numel()
    if scores.shape[1] != num_rows:
        raise ValueError(f'scores has {scores.shape[1]} query rows but rows has {num_rows}; '
                         'index the query axis by `rows` before calling')
    widths = []
    for block in blocks:
        n_cols = block.stop - block.start
        if block.budget.keeps_all:
            widths.append(n_cols)
        else:
            widths.append(split_budget(block.budget.per_row(block.real_tokens, n_cols), n_cols)[1])
    k_total = sum(widths)
    index = torch.empty(heads, num_rows, k_total, dtype=torch.int64, device=device)
    keep = torch.empty(heads, num_rows, k_total, dtype=torch.bool, device=device)
    scores32 = scores if scores.dtype == torch.float32 else scores.float()
    if scores32.stride(-1) != 1:
        scores32 = scores32.contiguous()
    rows = rows.to(device=device, dtype=torch.int64).contiguous()
    col0 = 0
    for block, width in zip(blocks, widths):
        n_cols = block.stop - block.start
        if block.budget.keeps_all:
            index[:, :, col0:col0 + width] = torch.arange(block.start, block.stop, device=device)
            keep[:, :, col0:col0 + width] = layout.kv_ok[block.start:block.stop]
        else:
            budget = block.budget.per_row(block.real_tokens, n_cols)
            k_lo, k_hi, frac = split_budget(budget, n_cols)
            extra = bresenham_extra(n_video, frac, device)
            ops.select_topk(scores32, block.start, n_cols, layout.kv_ok, rows, k_lo, k_hi,
                            extra, index, keep, col0)
        col0 += width
    return Selection(index, keep)


@torch.no_grad()
def dense_block_mask(selection: Selection, layout: tiling.TileLayout,
                     global_rows: bool = True) -> torch.Tensor:
    """[H', n_tiles (or R), n_tiles] bool block mask (mask.py:288-317)."""
    return ops.dense_block_mask(selection.index, selection.keep, layout.kv_ok,
                                layout.n_video_tiles, global_rows)


def kept_tiles_per_row(selection: Selection) -> torch.Tensor:
    """[H', n_video] number of selected video tiles (mask.py:320-322)."""
    return selection.keep.sum(-1)
