"""Host tests of the on-disk formats feeding the path: the request geometry
rules, the plan table (miowtion/veda/plan.py:36-188) and the predictor
bundle (miowtion/veda/bundle.py:48-359).

Pinned by reference data: every plan file the reference ships records the
token grid of its geometry (tests/golden/plan_grids.json, written from
those files by tests/golden/make_plan_fixture.py), which the geometry rules
must reproduce; the released 9x16 plans are the transposes the mirroring
rule produces. The e4m3 path is pinned by torch's own e4m3 conversion (the
library routine the reference calls) and by the per-head amax / 448 rule.
"""

import json
import os
import stat
import pathlib

import pytest
import torch

from miowtion_amd import bundle
from miowtion_amd import geometry
from miowtion_amd import mask as pm
from miowtion_amd import plan as pplan
from miowtion_amd import predictor as pp
from miowtion_amd import tiling as pt

GOLDEN = pathlib.Path(__file__).resolve().parent / 'golden'


def _grids():
    return json.loads((GOLDEN / 'plan_grids.json').read_text())


def test_geometry_rules_reproduce_every_shipped_plan_grid():
    checked = 0
    for name, rec in _grids().items():
        geo = rec['geometry']
        if geo.startswith('wan_'):  # Wan geometries are not H3 requests
            continue
        aspect, t = geo.split('_t')
        g = geometry.geometry_from_latent_t(aspect.replace('x', ':'), int(t))
        assert g.name == geo, name
        assert list(g.video_grid) == rec['grid'], (name, g.video_grid, rec['grid'])
        checked += 1
    assert checked == 17


def test_geometry_known_answers():
    g = geometry.resolve_geometry('16:9', 5.0)
    # 5 s -> 120 frames -> snapped to 124 = 17 * 7 + 5 -> latent_t 37
    assert (g.frame_count, g.latent_t, g.width, g.height) == (124, 37, 1344, 768)
    assert g.video_grid == (37, 24, 42) and g.num_video_tokens == 37 * 24 * 42
    assert geometry.align_frame_count(5) == 5 and geometry.align_frame_count(6) == 22
    assert geometry.video_latent_t(5) == 2 and geometry.video_latent_t(22) == 7
    assert geometry.frame_count_from_latent_t(102) == 345
    with pytest.raises(ValueError):
        geometry.frame_count_from_latent_t(100)
    with pytest.raises(ValueError):
        geometry.resolve_canvas(5, 1)
    assert geometry.latent_t_ladder(5.0, 15.0) == [37, 42, 47, 52, 57, 62, 67, 72, 77, 82, 87,
                                                   92, 97, 102]


def _plan(name, grid, shapes=('1x8x16', '2x8x8'), layers=2, heads=4):
    return pplan.TilePlan(name, tuple(grid), [pt.TileShape.parse(s) for s in shapes],
                          [[i % len(shapes) for i in range(heads)] for _ in range(layers)])


def test_plan_table_selection_rules():
    table = pplan.PlanTable([_plan('16x9_t37', (37, 24, 42)), _plan('16x9_t72', (72, 24, 42)),
                             _plan('16x9_t102', (102, 24, 42))])
    g = lambda a, t: geometry.geometry_from_latent_t(a, t)
    assert table.select(g('16:9', 37)).geometry == '16x9_t37'          # exact
    assert table.select(g('16:9', 52)).geometry == '16x9_t37'          # nearest latent_t
    assert table.select(g('16:9', 87)).geometry == '16x9_t72'          # 15 vs 15: shorter wins
    assert table.select(g('16:9', 97)).geometry == '16x9_t102'
    # no 9:16 plan: the mirrored aspect's nearest plan, as is or transposed,
    # whichever pads the 9:16 grid least
    pick = table.select(g('9:16', 42))
    grid = g('9:16', 42).video_grid
    base = table.plans['16x9_t37']
    pad = lambda p: sum(s.num_tiles(grid) for s in p.shapes)
    assert pad(pick) == min(pad(base), pad(base.transposed()))
    with pytest.raises(KeyError):
        table.select(g('1:1', 37))


def test_mirrored_plans_match_the_released_transposes():
    grids = _grids()
    for t in (37, 72, 102):
        src = grids[f'released/16x9_t{t}.json']
        plan = pplan.TilePlan(src['geometry'], tuple(src['grid']),
                              [pt.TileShape.parse(s) for s in src['shapes']], [[0] * 56] * 50)
        m = plan.mirrored()
        want = grids[f'released/9x16_t{t}.json']
        assert m.geometry == want['geometry'] and list(m.grid) == want['grid']
        assert [str(s) for s in m.shapes] == [str(pt.TileShape.parse(s).transposed())
                                              for s in src['shapes']]
        assert m.provenance['mirrored_from'] == src['geometry']


def test_released_plan_fixture_loads_into_the_table():
    plan = pplan.TilePlan.load(str(GOLDEN / 'plan_16x9_t37.json'))
    table = pplan.PlanTable([plan])
    assert table.select(geometry.geometry_from_latent_t('16:9', 42)) is plan
    groups = plan.head_groups(0, 'cpu')
    assert sum(g.heads.numel() for g in groups) == 56 and len(groups) <= 2


def _weights(layers=2, heads=4, d=128, rank=0, count=False, seed=0):
    g = torch.Generator().manual_seed(seed)
    out = {}
    for i in range(layers):
        out[f'layers.{i}.proj_q'] = torch.randn(heads, 3 * d, d, generator=g) * 0.02
        out[f'layers.{i}.proj_k'] = torch.randn(heads, 3 * d, d, generator=g) * 0.02
        if rank:
            out[f'layers.{i}.so_q'] = torch.randn(heads, d, rank, generator=g) * 0.02
            out[f'layers.{i}.so_k'] = torch.randn(heads, d, rank, generator=g) * 0.02
        if count:
            out[f'layers.{i}.count_gain'] = 1 + 0.1 * torch.randn(heads, generator=g)
    return out


def _table():
    return pplan.PlanTable([pplan.TilePlan.load(str(GOLDEN / 'plan_16x9_t37.json'))])


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16, torch.float8_e4m3fn])
@pytest.mark.parametrize('extras', [(0, False), (16, True)])
def test_bundle_round_trip(tmp_path, dtype, extras):
    rank, count = extras
    w = _weights(rank=rank, count=count)
    path = str(tmp_path / 'b.safetensors')
    bundle.save(path, {'predictor.' + k: v for k, v in w.items()}, _table(), num_layers=2,
                num_heads=4, head_dim=128, keep_tiles=12.5, source='ckpt/x', source_weights='ema',
                step=7, dtype=dtype, second_order_rank=rank, count_term=count)
    meta = bundle.read_metadata(path)
    assert meta['format'] == 'miowtion-veda-predictor-v1'
    assert meta['target_budget_kind'] == 'tiles' and float(meta['target_budget_value']) == 12.5
    assert 'keep_ratio' not in meta and meta['step'] == '7' and meta['source_weights'] == 'ema'
    b = bundle.load(path)
    assert b.target_budget == pm.Budget(tiles=12.5) and b.keep_ratio is None
    assert b.ref_budget is None and not b.tile_conditions
    assert set(b.plans.plans) == {'16x9_t37'}
    layer = b.predictor.layers[1]
    assert layer.second_order_rank == rank and (layer.count_gain is not None) == count
    ref = w['layers.1.proj_q']
    if dtype is torch.float8_e4m3fn:
        # per-head amax onto 448, torch's e4m3 rounding, decoded to bf16
        amax = ref.abs().amax(dim=(1, 2))
        scale = (amax / 448).clamp(min=torch.finfo(torch.float32).tiny)
        vals = (ref / scale[:, None, None]).to(torch.float8_e4m3fn)
        assert torch.equal(layer.proj_q.values, vals) and torch.equal(layer.proj_q.scale, scale)
        want = (vals.float() * scale[:, None, None]).to(torch.bfloat16)
        assert torch.equal(bundle.state_dict(b.predictor)['layers.1.proj_q'], want)
        flat = bundle.load(path, keep_fp8=False).predictor.layers[1].proj_q
        assert flat.scale is None and torch.equal(flat.values, want)
    else:
        assert layer.proj_q.values.dtype == dtype
        assert torch.equal(layer.proj_q.values, ref.to(dtype))
    if count:
        g = w['layers.1.count_gain']
        if dtype is torch.float8_e4m3fn:
            s = (g.abs().amax() / 448)  # one scale for a 1-D tensor
            g = ((g / s).to(torch.float8_e4m3fn).float() * s).to(torch.bfloat16)
        torch.testing.assert_close(layer.count_gain, g.to(dtype if dtype != torch.float8_e4m3fn
                                                          else torch.bfloat16).float(),
                                   rtol=0, atol=0)


def test_bundle_budgets_and_errors(tmp_path):
    w = _weights()
    path = str(tmp_path / 'b.safetensors')
    kw = dict(num_layers=2, num_heads=4, head_dim=128, source='s', source_weights='live', step=1)
    bundle.save(path, w, _table(), keep_ratio=0.1, ref_keep_ratio=0.3, tile_conditions=True, **kw)
    b = bundle.load(path)
    assert b.target_budget == pm.Budget(ratio=0.1) and b.keep_ratio == 0.1
    assert b.ref_budget == pm.Budget(ratio=0.3) and b.tile_conditions
    assert bundle.read_metadata(path)['keep_ratio'] == '0.1'
    with pytest.raises(ValueError, match='exactly one'):
        bundle.save(path, w, _table(), keep_ratio=0.1, keep_tiles=3.0, **kw)
    with pytest.raises(ValueError, match='requires tile_conditions'):
        bundle.save(path, w, _table(), keep_ratio=0.1, ref_keep_ratio=0.3, **kw)
    with pytest.raises(ValueError, match='requires a reference budget'):
        bundle.save(path, w, _table(), keep_ratio=0.1, tile_conditions=True, **kw)
    with pytest.raises(ValueError, match='mix prefixed'):
        bundle.save(path, {'predictor.layers.0.proj_q': w['layers.0.proj_q'],
                           'layers.0.proj_k': w['layers.0.proj_k']}, _table(), keep_ratio=0.1,
                    **kw)
    with pytest.raises(ValueError, match='plans'):
        bundle.save(path, w, pplan.PlanTable([]), keep_ratio=0.1, **kw)
    with pytest.raises(ValueError, match='storage dtype'):
        bundle.save(path, w, _table(), keep_ratio=0.1, dtype=torch.float16, **kw)
    # the metadata's predictor must match the weights exactly
    bad = str(tmp_path / 'bad.safetensors')
    bundle.save(bad, w, _table(), keep_ratio=0.1, **{**kw, 'num_layers': 3})
    with pytest.raises(ValueError, match='do not match'):
        bundle.load(bad)
    from safetensors.torch import save_file
    save_file({'x': torch.zeros(1)}, bad, metadata={'format': 'other'})
    with pytest.raises(ValueError, match='not a miowtion-veda-predictor-v1'):
        bundle.load(bad)
    # an e4m3 tensor without its scale is refused
    q, s = bundle.quantize_fp8(w['layers.0.proj_q'])
    save_file({'layers.0.proj_q': q}, bad,
              metadata={**bundle.read_metadata(path), 'dtype': 'float8_e4m3fn',
                        'num_layers': '1'})
    with pytest.raises(ValueError, match='scale'):
        bundle.load(bad)


def test_random_bundle_uses_least_padding_uniform_plans():
    geos = [geometry.geometry_from_latent_t('16:9', 37), geometry.geometry_from_latent_t('1:1', 72)]
    b = bundle.random_bundle(2, 4, 128, geos, keep_ratio=0.1, seed=3)
    for g in geos:
        plan = b.plans.select(g)
        assert plan.geometry == g.name and plan.shapes == [pt.least_padding_shape(g.video_grid)]
        assert plan.head_shape == [[0] * 4, [0] * 4]
    assert isinstance(b.predictor, pp.TileScorePredictor) and b.keep_ratio == 0.1


def test_bundle_metadata_is_the_reference_format(tmp_path):
    """Every metadata key and value a 'miowtion-veda-predictor-v1' writer
    puts in the file (the format of miowtion/veda/bundle.py:215-235): the
    strings, the sorted plans JSON and the legacy keep_ratio."""
    w = _weights(layers=1)
    path = str(tmp_path / 'b.safetensors')
    table = _table()
    bundle.save(path, w, table, num_layers=1, num_heads=4, head_dim=128, keep_ratio=0.25,
                ref_keep_tiles=7.0, tile_conditions=True, source='ckpt/run', source_weights='live',
                step=12, dtype=torch.bfloat16, second_order_rank=0, count_term=False)
    meta = bundle.read_metadata(path)
    want_plans = json.dumps({name: p.to_json() for name, p in sorted(table.plans.items())})
    assert meta == {
        'format': 'miowtion-veda-predictor-v1', 'num_layers': '1', 'num_heads': '4',
        'head_dim': '128', 'dtype': 'bfloat16', 'tile_conditions': 'true', 'source': 'ckpt/run',
        'source_weights': 'live', 'step': '12', 'second_order_rank': '0', 'count_term': '0',
        'plans': want_plans, 'target_budget_kind': 'ratio', 'target_budget_value': '0.25',
        'ref_budget_kind': 'tiles', 'ref_budget_value': '7.0', 'keep_ratio': '0.25'}
    # the tensors: bare state-dict names, stored in the requested dtype
    from safetensors import safe_open
    with safe_open(path, framework='pt', device='cpu') as f:
        assert sorted(f.keys()) == ['layers.0.proj_k', 'layers.0.proj_q']
        assert f.get_tensor('layers.0.proj_q').dtype == torch.bfloat16


def test_plan_json_round_trips_the_released_file_unchanged(tmp_path):
    raw = json.loads((GOLDEN / 'plan_16x9_t37.json').read_text())
    plan = pplan.TilePlan.from_json(raw)
    assert plan.to_json() == raw
    out = tmp_path / 'p.json'
    plan.save(str(out))
    assert json.loads(out.read_text()) == raw
    assert [p.name for p in tmp_path.iterdir()] == ['p.json']   # no temporary left behind
    # the mode open(path, 'w') gives, as the reference's writer (0666 less the umask)
    umask = os.umask(0)
    os.umask(umask)
    assert stat.S_IMODE(out.stat().st_mode) == 0o666 & ~umask
    with pytest.raises(ValueError, match='at most 2'):
        pplan.TilePlan('g', (1, 8, 16), [pt.TileShape.parse(s) for s in ('1x8x16', '2x8x8',
                                                                             '4x4x8')],
                       [[0, 1, 2]])
