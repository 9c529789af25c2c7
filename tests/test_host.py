"""CPU tests of the product's host logic: the closed-form permutation, the
budgets, plans and students' guards, against the (pinned) oracle."""

import json
import pathlib

import pytest
import torch

from miowtion_amd import attention as pa
from miowtion_amd import mask as pm
from miowtion_amd import plan as pp
from miowtion_amd import tiling as pt
from oracle import mask as om
from oracle import tiling as ot
from tests import helpers


@pytest.mark.parametrize('name', sorted(helpers.CONFIGS))
def test_layout_bit_exact_at_baseline_geometries(name):
    spans, used, seq_len, shape = helpers.CONFIGS[name]
    got = helpers.product_layout(spans, used, seq_len, shape)
    want = helpers.oracle_layout(spans, used, seq_len, shape)
    for field in ('perm', 'valid_count', 'gather_index', 'scatter_index', 'pad_slots',
                  'partial_tiles', 'kv_ok', 'full_tile', 'slot_valid'):
        a, b = getattr(got, field), getattr(want, field)
        assert a.dtype == b.dtype, field
        assert torch.equal(a, b), field
    for field in ('n_video_tiles', 'n_ref_tiles', 'n_global_tiles', 'ref_tokens',
                  'target_tokens', 'used', 'seq_len'):
        assert getattr(got, field) == getattr(want, field), field


def test_baseline_tile_counts():
    lay = helpers.product_layout(*helpers.CONFIGS['C2'])
    assert lay.n_tiles == 592 and lay.num_slots == 75776
    assert int((lay.valid_count == 128).sum()) == 333
    assert int(lay.valid_count.min()) == 24
    lay = helpers.product_layout(*helpers.CONFIGS['C5'])
    assert (lay.n_video_tiles, lay.n_global_tiles) == (1632, 16)
    assert lay.num_slots == 210944
    lay = helpers.product_layout(*helpers.CONFIGS['C3b'])
    assert lay.n_tiles == 520 and int(lay.full_tile.sum()) == 351


@pytest.mark.parametrize('seed', range(20))
def test_layout_bit_exact_random_spans(seed):
    g = torch.Generator().manual_seed(seed)
    shapes = pt.all_shapes()
    r = lambda lo, hi: int(torch.randint(lo, hi, (1,), generator=g))
    n_spans = r(1, 4)
    spans, start = [], r(0, 300)
    for _ in range(n_spans):
        grid = (r(1, 9), r(1, 40), r(1, 40))
        spans.append((start, grid))
        start += grid[0] * grid[1] * grid[2] + r(0, 200)
    used = start
    seq_len = used + r(0, 64)
    shape = str(shapes[r(0, len(shapes))])
    for contiguous in (False, True):
        # condition spans take their own least-padding shape in the product;
        # here every span uses `shape`, which both sides support
        got = helpers.product_layout(spans, used, seq_len, shape, contiguous=contiguous)
        want = helpers.oracle_layout(spans, used, seq_len, shape, contiguous=contiguous)
        assert torch.equal(got.perm, want.perm)
        assert got.n_ref_tiles == want.n_ref_tiles
        assert torch.equal(got.valid_count, want.valid_count)


def test_shape_menu_matches_oracle():
    assert [str(s) for s in pt.all_shapes()] == [f'{s.t}x{s.h}x{s.w}' for s in ot.shape_menu()]
    for grid in ((37, 24, 42), (1, 64, 112), (37, 30, 52), (5, 3, 2), (102, 52, 30)):
        a, b = pt.least_padding_shape(grid), ot.least_padding(grid)
        assert (a.t, a.h, a.w) == (b.t, b.h, b.w)


@pytest.mark.parametrize('budget', [0.3, 1.0, 2.3, 3.75, 5.5, 34.358277027027027, 63.99, 70.0])
def test_budget_arithmetic_matches_oracle(budget):
    assert pm.split_budget(budget, 64) == om.split_budget(budget, 64)
    _, _, frac = pm.split_budget(budget, 64)
    assert torch.equal(pm.bresenham_extra(700, frac, 'cpu'), om.bresenham(700, frac))


def test_equal_cost_per_row_matches_oracle():
    for ratio, tokens, n in ((0.1, 57720, 592), (0.2, 57720, 518), (0.2, 57720, 520),
                             (0.05, 159120, 1632), (0.1, 37296, 330), (0.5, 1024, 8)):
        assert pm.Budget(ratio=ratio).per_row(tokens, n) == om.Budget(ratio=ratio).per_row(tokens, n)
    with pytest.raises(ValueError):
        pm.Budget()
    with pytest.raises(ValueError):
        pm.Budget(ratio=-1.0)


def test_plan_groups_limits_and_json(tmp_path):
    # reference tests/unit/test_veda_tiling_plan.py:90-102
    shapes = [pt.TileShape(4, 8, 4), pt.TileShape(8, 8, 2), pt.TileShape(2, 8, 8)]
    with pytest.raises(ValueError):
        pp.TilePlan('g', (37, 30, 52), shapes, [[0, 1, 2, 0]])
    plan = pp.TilePlan('g', (37, 30, 52), shapes, [[0, 1, 1, 0], [2, 2, 2, 2]])
    groups = plan.head_groups(0, 'cpu')
    assert [g.heads.tolist() for g in groups] == [[0, 3], [1, 2]]
    path = tmp_path / 'p.json'
    plan.save(str(path))
    assert pp.TilePlan.load(str(path)).to_json() == plan.to_json()


def test_released_plan_fixture_loads():
    path = pathlib.Path(__file__).parent / 'golden' / 'plan_16x9_t37.json'
    plan = pp.TilePlan.load(str(path))
    assert plan.grid == (37, 24, 42)
    for layer in range(plan.num_layers):
        assert len(plan.layer_shapes(layer)) <= 2
        heads = torch.cat([g.heads for g in plan.head_groups(layer, 'cpu')])
        assert torch.equal(heads.sort().values, torch.arange(len(plan.head_shape[layer])))


def test_products_refuse_cpu_tensors_and_students_refuse_cpu_clips():
    from miowtion_amd import kernels
    lay = helpers.product_layout(*helpers.small_layout())
    x = torch.zeros(lay.seq_len, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        kernels.gather_tiles(x, lay, None)
    layout = pa.PackedLayout((pa.VideoSpan(0, (4, 16, 16)),), 1024, 1024)
    clip = pa.ClipTiling(layout, pa.VedaConfig(), 'cpu')
    plan = pp.TilePlan.uniform('c1', (4, 16, 16), pt.TileShape(2, 8, 8), 1, 8)
    with pytest.raises(RuntimeError, match='refusing to fall back'):
        pa.SparseStudent(clip, plan, None)
    with pytest.raises(RuntimeError, match='refusing to fall back'):
        pa.OracleStudent(clip, plan)


def test_select_rejects_threshold_rule():
    lay = helpers.product_layout(*helpers.small_layout())
    with pytest.raises(ValueError, match='topk'):
        pm.select_video_blocks(torch.zeros(1, lay.n_video_tiles, lay.n_tiles), lay,
                               pm.column_blocks(lay, pm.Budget(ratio=0.3)), rule='threshold')


def test_chunk_heads_bound():
    lay = helpers.product_layout(*helpers.CONFIGS['C2'])
    assert pa._chunk_heads(lay, 256 * 2 ** 20) == 13
    assert pa._chunk_heads(lay, pa.DEFAULT_COLLECT_BYTES) >= 48
