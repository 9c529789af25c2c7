"""Pins the oracle's tile permutation (oracle/tiling.py) against the
reference's own known answers (tests/unit/test_veda_tiling_plan.py of the
reference), invariants, and a brute-force box enumeration."""

import itertools

import pytest
import torch

from oracle import tiling as ot

_GRID = (37, 24, 42)


def test_known_answers_shape_menu_and_padding():
    # reference tests/unit/test_veda_tiling_plan.py:13-20
    assert len(ot.shape_menu()) == 36
    assert ot.Shape(1, 8, 16).count(_GRID) == 333
    assert ot.Shape(8, 4, 4).count(_GRID) == 330
    assert ot.Shape(8, 4, 4).padded(_GRID) == (40, 24, 44)
    assert ot.least_padding((1, 64, 112)).t == 1
    with pytest.raises(ValueError):
        ot.Shape(2, 2, 2)


def test_known_answers_baseline_geometries():
    # Tile counts of the BASELINE configs from the closed form tiling.py:67-73.
    assert ot.Shape(2, 8, 8).count((4, 16, 16)) == 8             # C1
    assert ot.Shape(1, 8, 16).count((37, 30, 52)) == 592         # C2
    assert ot.Shape(1, 8, 16).padded((37, 30, 52)) == (37, 32, 64)
    assert ot.Shape(1, 8, 16).count((37, 52, 30)) == 518         # C3
    assert ot.Shape(4, 4, 8).count((37, 52, 30)) == 520
    assert ot.Shape(1, 8, 16).count((102, 30, 52)) == 1632       # C5


def _brute_tiles(span):
    """Each tile as its box clipped to the grid, rows t,h,w row-major, padding
    last; tiles ordered h-block, w-block, t-block (tiling.py:122-127)."""
    T, H, W = span.grid
    s = span.shape
    nt, nh, nw = -(-T // s.t), -(-H // s.h), -(-W // s.w)
    out = []
    for hb, wb, tb in itertools.product(range(nh), range(nw), range(nt)):
        rows = []
        for lt, lh, lw in itertools.product(range(s.t), range(s.h), range(s.w)):
            t, h, w = tb * s.t + lt, hb * s.h + lh, wb * s.w + lw
            if t < T and h < H and w < W:
                rows.append(span.start + (t * H + h) * W + w)
        out.append(rows + [-1] * (128 - len(rows)))
    return torch.tensor(out, dtype=torch.long)


@pytest.mark.parametrize('grid,shape', [((4, 16, 16), '2x8x8'), ((7, 6, 10), '4x8x4'),
                                        ((5, 9, 13), '8x2x8'), ((3, 30, 20), '1x8x16'),
                                        ((37, 12, 10), '4x4x8'), ((6, 6, 12), '2x4x16')])
def test_span_tiles_equals_brute_force_boxes(grid, shape):
    span = ot.Span(17, grid, ot.Shape.parse(shape))
    assert torch.equal(ot.span_tiles(span), _brute_tiles(span))


def test_tile_contents_are_3d_boxes():
    # reference tests/unit/test_veda_tiling_plan.py:52-61
    tiles = ot.span_tiles(ot.Span(0, (4, 8, 16), ot.Shape(2, 4, 16)))
    t, h, _ = torch.unravel_index(tiles[0], (4, 8, 16))
    assert set(t.tolist()) == {0, 1} and set(h.tolist()) == {0, 1, 2, 3}
    t, h, _ = torch.unravel_index(tiles[1], (4, 8, 16))
    assert set(t.tolist()) == {2, 3} and set(h.tolist()) == {0, 1, 2, 3}


def _layout(shape='4x8x4', text=100, cond=None):
    spans, start = [], text
    if cond is not None:
        spans.append(ot.Span(start, cond, ot.least_padding(cond)))
        start += cond[0] * cond[1] * cond[2]
    target = ot.Span(start + 50, (7, 6, 10), ot.Shape.parse(shape))
    used = target.start + target.rows
    return ot.build_layout(spans + [target], used, used + 30)


def test_bijection_prefix_and_global_order():
    lay = _layout('8x2x8')
    real = lay.perm[lay.perm >= 0]
    assert torch.equal(real.sort().values, torch.arange(lay.used))
    tiles = lay.perm.view(-1, 128)
    for tile, count in zip(tiles, lay.valid_count):
        assert (tile[:count] >= 0).all() and (tile[count:] < 0).all()
    assert (lay.valid_count[lay.partial_tiles] < 128).all()
    lay = _layout(cond=(1, 6, 10))
    assert lay.n_ref_tiles == ot.least_padding((1, 6, 10)).count((1, 6, 10))
    video = lay.perm[:lay.n_video_tiles * 128]
    glob = lay.perm[lay.n_video_tiles * 128:]
    assert (glob[glob >= 0] < 100 + 60 + 50).all()
    assert (video[video >= 0] >= 100).all()
    assert lay.ref_tokens == 60 and lay.target_tokens == 420
    # global rows are the uncovered real rows, in sequence order
    g = glob[glob >= 0]
    assert torch.equal(g, g.sort().values)


def test_contiguous_known_answers():
    # reference tests/unit/test_veda_tiling_plan.py:140-177
    tiles = ot.contiguous_span_tiles(ot.Span(7, (8, 4, 8), ot.Shape.parse('4x4x8')))
    assert torch.equal(tiles, (7 + torch.arange(256)).view(-1, 128))
    tiles = ot.contiguous_span_tiles(ot.Span(0, (3, 4, 8), ot.Shape.parse('4x4x8')))
    assert tiles.shape == (1, 128) and torch.equal(tiles[0, :96], torch.arange(96))
    assert bool((tiles[0, 96:] == -1).all())
    span = ot.Span(0, (4, 4, 8), ot.Shape.parse('2x8x8'))
    lay = ot.build_layout([span], 128, 128, tiler=ot.contiguous_span_tiles)
    assert torch.equal(lay.perm, torch.arange(128))
    assert not torch.equal(ot.build_layout([span], 128, 128).perm, torch.arange(128))
    # C2 under the contiguous tiler: 451 tiles, the last holding 120 rows
    c = ot.contiguous_span_tiles(ot.Span(0, (37, 30, 52), ot.Shape(1, 8, 16)))
    assert c.shape[0] == 451 and int((c[-1] >= 0).sum()) == 120


def test_derived_index_tensors():
    lay = _layout('2x8x8')
    pad = lay.perm < 0
    assert torch.equal(lay.gather_index[pad], torch.zeros(int(pad.sum()), dtype=torch.long))
    assert (lay.scatter_index[pad] == lay.seq_len).all()
    assert torch.equal(lay.slot_valid.bool(), ~pad)
    assert torch.equal(lay.kv_ok, lay.valid_count > 0)
    assert torch.equal(lay.full_tile, lay.valid_count == 128)


def test_gather_scatter_roundtrip():
    # reference tests/unit/test_veda_tiling_plan.py:75-87
    lay = _layout('2x8x8')
    x = torch.randn(lay.seq_len, 4, 8)
    heads = torch.tensor([1, 3])
    tiled = ot.gather_tiles(x, lay, heads)
    assert tiled.shape == (lay.num_slots, 2, 8) and (tiled[lay.pad_slots] == 0).all()
    out = torch.zeros(lay.seq_len + 1, 4, 8)
    ot.scatter_tiles_(out, tiled, lay, heads)
    real = lay.perm[lay.perm >= 0]
    assert torch.equal(out[real][:, heads], x[real][:, heads])
    assert (out[:lay.seq_len, 0] == 0).all()
