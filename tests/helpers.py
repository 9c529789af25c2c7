"""Shared builders of the parity tests: the BASELINE geometries, seeded
synthetic q / k / v, and product / oracle layout pairs.

Synthetic inputs follow the reference's GPU tests
(`tests/gpu/test_kernels_gpu.py:26-29`): torch.randn on a seeded CPU
generator, cast to bf16, then moved to the device.
"""

from __future__ import annotations

import torch

from miowtion_amd import tiling as pt
from oracle import tiling as ot

# name -> (spans [(start, grid)], used, seq_len, shape)
CONFIGS = {
    'C1': ([(0, (4, 16, 16))], 1024, 1024, '2x8x8'),
    'C2': ([(0, (37, 30, 52))], 57720, 57728, '1x8x16'),
    'C3a': ([(0, (37, 52, 30))], 57720, 57728, '1x8x16'),
    'C3b': ([(0, (37, 52, 30))], 57720, 57728, '4x4x8'),
    'C5': ([(2048, (102, 30, 52))], 161168, 161216, '1x8x16'),
}


def product_layout(spans, used, seq_len, shape, device='cpu', contiguous=False):
    sh = pt.TileShape.parse(shape)
    tsp = [pt.TiledSpan(s, tuple(g), sh) for s, g in spans]
    tiler = pt.contiguous_span_tiles if contiguous else pt.span_tiles
    return pt.build_tile_layout(tsp, used, seq_len, device, tiler=tiler)


def oracle_layout(spans, used, seq_len, shape, contiguous=False):
    sh = ot.Shape.parse(shape)
    osp = [ot.Span(s, tuple(g), sh) for s, g in spans]
    tiler = ot.contiguous_span_tiles if contiguous else ot.span_tiles
    return ot.build_layout(osp, used, seq_len, tiler=tiler)


def small_layout(grid=(8, 12, 20), shape='4x8x4', text=300, extra=32):
    """The reference GPU tests' layout (test_kernels_gpu.py:20-23): a target
    span after some text rows, padded grid -> partial tiles."""
    start = text + 60
    used = start + grid[0] * grid[1] * grid[2]
    return [(start, grid)], used, used + extra, shape


def qkv(seq_len, heads=4, dim=128, seed=0, n=3):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(seq_len, heads, dim, generator=g).to(torch.bfloat16) for _ in range(n)]


