"""Teacher block heat (host mirror of miowtion/veda/heatmap.py:1-110).

heat[i, j] with reduce='max' is the largest true attention probability in
the 128x128 block (query tile i, key tile j); with reduce='sum' it is the
block's total attention mass. Both come from the dense teacher's LSE and are
computed by the `veda::block_heat` HIP kernel.
"""

from __future__ import annotations

import torch

from miowtion_amd import kernels
from miowtion_amd import tiling


def teacher_heat(q: torch.Tensor, k: torch.Tensor, lse: torch.Tensor,
                 layout: tiling.TileLayout, q_tiles: torch.Tensor,
                 reduce: str = 'max') -> torch.Tensor:
    """[H', R, n_tiles] fp32 heat of query tiles `q_tiles` (tile-ordered q, k
    [N, H', D] bf16, lse [N, H'] fp32 with 0 on padding)."""
    if reduce not in ('max', 'sum'):
        raise ValueError(f"reduce must be 'max' or 'sum': {reduce!r}")
    return kernels.teacher_heat(q, k, lse, layout, q_tiles, reduce)
