"""Oracle: equal-cost budgets, Bresenham rounding, top-k selection, block
masks and full / partial index lists (CPU torch, test-only).

Restates:
  * Budget.per_row / split_budget / bresenham  -> `miowtion/veda/mask.py:38-93`
  * column_blocks                              -> `miowtion/veda/mask.py:106-120`
  * select_video_blocks (rule 'topk')          -> `miowtion/veda/mask.py:200-285`
  * dense_block_mask                           -> `miowtion/veda/mask.py:288-317`
  * _pack_lists / index_lists                  -> `miowtion/kernels/fa4.py:266-296`

Tie order: equal scores are taken lower column first (a stable descending
sort). `torch.topk`, which the reference calls, agrees whenever the scores
at the cut are distinct; on exact ties its order is backend-defined.
"""

from __future__ import annotations

import dataclasses
import math

import torch

from oracle.tiling import TILE, Layout


@dataclasses.dataclass(frozen=True)
class Budget:
    ratio: float | None = None
    tiles: float | None = None

    @property
    def keeps_all(self) -> bool:
        return self.ratio is not None and self.ratio >= 1.0

    def per_row(self, real_tokens: int, n_tiles: int) -> float:
        # mask.py:61-65 -- Python float arithmetic, left to right.
        if self.tiles is not None:
            return float(self.tiles)
        ideal = math.ceil(real_tokens / TILE)
        return self.ratio * ideal * ideal / n_tiles


def split_budget(budget: float, n_cols: int):
    """mask.py:68-76 -> (k_lo, k_hi, frac)."""
    if budget >= n_cols:
        return n_cols, n_cols, 0.0
    k_lo = min(max(1, math.floor(budget)), n_cols)
    frac = round(min(max(budget - k_lo, 0.0), 1.0), 12)
    return k_lo, min(k_lo + 1, n_cols), frac


def bresenham(n_rows: int, frac: float) -> torch.Tensor:
    """mask.py:79-93: row r keeps k_hi iff floor((r+1) f) > floor(r f), fp64."""
    ramp = torch.floor(torch.arange(n_rows + 1, dtype=torch.float64) * frac)
    return ramp[1:] > ramp[:-1]


@dataclasses.dataclass(frozen=True)
class ColumnBlock:
    start: int
    stop: int
    budget: Budget
    real_tokens: int


def column_blocks(lay: Layout, target: Budget, ref: Budget | None = None):
    tb = ColumnBlock(lay.n_ref_tiles, lay.n_video_tiles, target, lay.target_tokens)
    if lay.n_ref_tiles == 0:
        return [tb]
    if ref is None:
        raise ValueError('tiled references need their own budget')
    return [ColumnBlock(0, lay.n_ref_tiles, ref, lay.ref_tokens), tb]


def _stable_topk(s: torch.Tensor, k: int):
    vals, idx = torch.sort(s, dim=-1, descending=True, stable=True)
    return vals[..., :k], idx[..., :k]


def select_video_blocks(scores: torch.Tensor, lay: Layout, blocks, rows=None):
    """mask.py:200-285 (rule 'topk'). Returns (index int64, keep bool)."""
    heads = scores.shape[0]
    if rows is None:
        rows = torch.arange(lay.n_video_tiles)
    R = rows.numel()
    if scores.shape[1] != R:
        raise ValueError('scores must already be restricted to rows')
    idx_parts, keep_parts = [], []
    for b in blocks:
        n_cols = b.stop - b.start
        if b.budget.keeps_all:
            idx_parts.append(torch.arange(b.start, b.stop).expand(heads, R, n_cols))
            keep_parts.append(lay.kv_ok[b.start:b.stop].expand(heads, R, n_cols))
            continue
        s = scores[:, :, b.start:b.stop].float().clone()
        s[:, :, ~lay.kv_ok[b.start:b.stop]] = float('-inf')
        for ri, r in enumerate(rows.tolist()):
            if b.start <= r < b.stop:
                s[:, ri, r - b.start] = float('inf')
        k_lo, k_hi, frac = split_budget(b.budget.per_row(b.real_tokens, n_cols), n_cols)
        vals, idx = _stable_topk(s, k_hi)
        allowed = k_lo + bresenham(lay.n_video_tiles, frac)[rows].long()
        keep = (torch.arange(k_hi)[None, None, :] < allowed[None, :, None]) & (vals > float('-inf'))
        idx_parts.append(idx + b.start)
        keep_parts.append(keep)
    return torch.cat(idx_parts, -1), torch.cat(keep_parts, -1)


def dense_block_mask(index, keep, lay: Layout, global_rows: bool = True):
    """mask.py:288-317 -> [H', n or R, n] bool."""
    heads, R, _ = index.shape
    n, nv = lay.n_tiles, lay.n_video_tiles
    if global_rows and R != nv:
        raise ValueError('global_rows needs a selection of all video rows')
    m = torch.zeros(heads, n if global_rows else R, n, dtype=torch.bool)
    m[:, :R].scatter_(2, index, keep)
    m[:, :, nv:] = lay.kv_ok[nv:]
    if global_rows:
        m[:, nv:, :] = lay.kv_ok
    return m


def pack_lists(member: torch.Tensor):
    """fa4.py:266-272: members ascending, then non-members ascending."""
    heads, R, C = member.shape
    order = torch.argsort((~member).to(torch.int8), dim=-1, stable=True)
    idx = torch.arange(C).expand(heads, R, C)
    return (member.sum(-1)[None].to(torch.int32),
            torch.gather(idx, -1, order)[None].to(torch.int32).contiguous())


def index_lists(block_mask: torch.Tensor, lay: Layout, transpose: bool = False):
    """fa4.py:275-296 -> (part_cnt, part_idx, full_cnt, full_idx); transpose:
    the Q-direction lists (rows = key tiles, split by the row's fullness)."""
    m = block_mask & lay.kv_ok
    full = lay.full_tile
    if transpose:
        m = m.transpose(1, 2)
        full = full[:, None]
    fc, fi = pack_lists(m & full)
    pc, pi = pack_lists(m & ~full)
    return pc, pi, fc, fi
