"""GPU parity of the top-k selection, the block mask and the full / partial
lists: bit-exact against the oracle (which equals torch.topk on distinct
scores and follows the stable order on ties)."""

import math
import types

import pytest
import torch

from miowtion_amd import kernels
from miowtion_amd import mask as pm
from miowtion_amd import ops
from oracle import mask as om
from oracle import tiling as ot
from tests import helpers

pytestmark = pytest.mark.gpu


def _spec_with_cond():
    # condition span (tiled with its least-padding shape in the reference's
    # ClipTiling) + target: two column blocks with their own budgets
    return [(90, (1, 16, 32)), (90 + 512 + 40, (16, 8, 16))], 90 + 512 + 40 + 2048, 90 + 512 + 40 + 2048, '4x8x4'


def _layouts(spec):
    return helpers.product_layout(*spec, device='cuda'), helpers.oracle_layout(*spec)


def _run(scores, lay, olay, p_blocks, o_blocks, rows=None):
    sel = pm.select_video_blocks(scores.cuda(), lay, p_blocks, None if rows is None else rows.cuda())
    ri, rk = om.select_video_blocks(scores, olay, o_blocks, rows)
    assert torch.equal(sel.index.cpu(), ri)
    assert torch.equal(sel.keep.cpu(), rk)
    return sel, ri, rk


@pytest.mark.parametrize('seed', range(3))
def test_select_bit_exact_two_blocks(seed):
    lay, olay = _layouts(_spec_with_cond())
    nv = lay.n_video_tiles
    g = torch.Generator().manual_seed(seed)
    scores = torch.randn(3, nv, lay.n_tiles, generator=g)
    pb = pm.column_blocks(lay, pm.Budget(ratio=0.25), pm.Budget(tiles=2.5))
    ob = om.column_blocks(olay, om.Budget(ratio=0.25), om.Budget(tiles=2.5))
    sel, ri, rk = _run(scores, lay, olay, pb, ob)
    mask = pm.dense_block_mask(sel, lay).cpu()
    assert torch.equal(mask, om.dense_block_mask(ri, rk, olay))
    rows = torch.tensor([0, lay.n_ref_tiles - 1, lay.n_ref_tiles, nv - 1])
    sel, ri, rk = _run(scores[:, rows], lay, olay, pb, ob, rows)
    sub = pm.dense_block_mask(sel, lay, global_rows=False).cpu()
    assert torch.equal(sub, om.dense_block_mask(ri, rk, olay, global_rows=False))


def test_select_ties_follow_the_stable_order():
    lay, olay = _layouts(_spec_with_cond())
    nv = lay.n_video_tiles
    scores = torch.randint(0, 4, (3, nv, lay.n_tiles), generator=torch.Generator().manual_seed(0)).float()
    scores[0, :, 5] = -0.0
    scores[0, :, 6] = 0.0
    pb = pm.column_blocks(lay, pm.Budget(ratio=0.25), pm.Budget(tiles=2))
    ob = om.column_blocks(olay, om.Budget(ratio=0.25), om.Budget(tiles=2))
    _run(scores, lay, olay, pb, ob)


def test_select_nan_scores_rank_first_and_are_never_kept():
    """torch.topk / torch.sort rank every NaN, of either sign, above +inf, and
    the reference keeps an entry only where `val > -inf`, which is False for
    NaN (mask.py:251-284): NaN columns take the first positions of the index
    and are never kept. The oracle follows torch.sort (pinned against
    torch.topk in test_oracle_mask.py); the kernel must match it bit for
    bit. Rows with more NaNs than k_hi, NaN on the own-tile diagonal (the
    diagonal is forced to +inf) and NaN on empty tiles (forced to -inf) are
    all covered."""
    lay, olay = _layouts(_spec_with_cond())
    nv = lay.n_video_tiles
    g = torch.Generator().manual_seed(5)
    scores = torch.randn(3, nv, lay.n_tiles, generator=g)
    pick = torch.rand(scores.shape, generator=g)
    nan = torch.tensor(float('nan'))
    scores = torch.where(pick < 0.05, nan, scores)
    scores = torch.where((pick >= 0.05) & (pick < 0.08), -nan, scores)
    scores = torch.where((pick >= 0.08) & (pick < 0.09), torch.tensor(float('inf')), scores)
    scores = torch.where((pick >= 0.09) & (pick < 0.10), torch.tensor(float('-inf')), scores)
    assert torch.signbit(scores[(pick >= 0.05) & (pick < 0.08)]).all()
    scores[1, 3] = nan                       # a row of NaN only
    scores[2, 4] = -nan
    rows = torch.arange(nv)
    scores[0, rows, rows] = nan              # NaN on every diagonal
    pb = pm.column_blocks(lay, pm.Budget(ratio=0.25), pm.Budget(tiles=2.5))
    ob = om.column_blocks(olay, om.Budget(ratio=0.25), om.Budget(tiles=2.5))
    sel, ri, rk = _run(scores, lay, olay, pb, ob)
    flat_s = scores.gather(-1, ri)
    # the own tile is forced to +inf, so its NaN score does not count; NaN
    # columns rank ahead of it and can push it past the row's budget
    own = ri == torch.arange(nv)[None, :, None]
    assert not rk[torch.isnan(flat_s) & ~own].any()
    mask = pm.dense_block_mask(sel, lay).cpu()
    assert torch.equal(mask, om.dense_block_mask(ri, rk, olay))


def test_select_keep_all_and_budget_above_columns():
    lay, olay = _layouts(helpers.small_layout())
    scores = torch.rand(2, lay.n_video_tiles, lay.n_tiles, generator=torch.Generator().manual_seed(3))
    for b in (1.0, 0.999):
        _run(scores, lay, olay, pm.column_blocks(lay, pm.Budget(ratio=b)),
             om.column_blocks(olay, om.Budget(ratio=b)))
    _run(scores, lay, olay, pm.column_blocks(lay, pm.Budget(tiles=1000)),
         om.column_blocks(olay, om.Budget(tiles=1000)))


def test_index_lists_bit_exact():
    lay, olay = _layouts(helpers.small_layout())
    g = torch.Generator().manual_seed(5)
    mask = torch.rand(4, lay.n_tiles, lay.n_tiles, generator=g) < 0.4
    got = kernels.index_lists(mask.cuda(), lay)
    want = om.index_lists(mask, olay)
    for a, b in zip(got, want):
        assert a.dtype == b.dtype and torch.equal(a.cpu(), b)


@pytest.mark.parametrize('n,offset', [(592, 0), (592, 1), (100, 0), (37, 0), (4096, 0),
                                      (4097, 0), (4160, 0)])
def test_index_lists_every_load_width(n, offset):
    """Random masks and column tables whose row length and alignment select
    each load width of the list kernel (16-, 4- and 1-byte loads; a column
    table 1 byte off its allocation), and rows past the LDS-staged length
    (4096 columns): bit-exact against the oracle, counts included."""
    g = torch.Generator().manual_seed(n + offset)
    mask = torch.rand(2, 3, n, generator=g) < 0.3
    mask[1, 2] = False                      # an empty row
    mask[0, 1] = True                       # a row of all columns
    kv_ok = torch.rand(n + offset, generator=g) < 0.9
    full = torch.rand(n + offset, generator=g) < 0.5
    kv_ok, full = kv_ok[offset:], full[offset:]
    kv_gpu = torch.zeros(n + offset, dtype=torch.bool, device='cuda')
    full_gpu = torch.zeros(n + offset, dtype=torch.bool, device='cuda')
    kv_gpu[offset:] = kv_ok.cuda()
    full_gpu[offset:] = full.cuda()
    got = ops.index_lists(mask.cuda(), kv_gpu[offset:], full_gpu[offset:])
    want = om.index_lists(mask, types.SimpleNamespace(kv_ok=kv_ok, full_tile=full))
    for a, b in zip(got, want):
        assert a.dtype == b.dtype and torch.equal(a.cpu(), b)


@pytest.mark.parametrize('name,ratio', [('C2', 0.1), ('C3b', 0.2)])
def test_selection_and_lists_at_full_size(name, ratio):
    """48 heads of uniform random scores at the BASELINE geometry: top-k,
    block mask and lists bit-exact; kept blocks per head = the equal-cost
    budget (C2: 20,340, C3: 40,680)."""
    lay, olay = _layouts(helpers.CONFIGS[name])
    n = lay.n_tiles
    scores = torch.rand(48, n, n, generator=torch.Generator().manual_seed(11))
    pb = pm.column_blocks(lay, pm.Budget(ratio=ratio))
    ob = om.column_blocks(olay, om.Budget(ratio=ratio))
    sel, ri, rk = _run(scores, lay, olay, pb, ob)
    mask = pm.dense_block_mask(sel, lay)
    want_mask = om.dense_block_mask(ri, rk, olay)
    assert torch.equal(mask.cpu(), want_mask)
    expected = {'C2': 20340, 'C3b': 40680}[name]
    assert (mask.sum((1, 2)).cpu() == expected).all()
    got = kernels.index_lists(mask, lay)
    for a, b in zip(got, om.index_lists(want_mask, olay)):
        assert torch.equal(a.cpu(), b)


def test_select_at_the_largest_column_count():
    """2048 key tiles (FA4's per-side cap; the top-k kernel's score rows then
    take its largest LDS size, 4 waves x 2048 columns x 8 bytes = 64 KB), with
    ties and -inf rows mixed in: bit-exact against the oracle."""
    spec = ([(0, (32, 62, 120))], 32 * 62 * 120, 32 * 62 * 120, '1x8x16')
    lay, olay = _layouts(spec)
    assert lay.n_tiles == 2048
    g = torch.Generator().manual_seed(21)
    scores = torch.rand(2, lay.n_video_tiles, lay.n_tiles, generator=g)
    scores[0, ::7] = torch.randint(0, 3, (scores[0, ::7].shape), generator=g).float()  # ties
    scores[1, 5] = float('-inf')  # only the forced diagonal survives
    _run(scores, lay, olay, pm.column_blocks(lay, pm.Budget(ratio=0.1)),
         om.column_blocks(olay, om.Budget(ratio=0.1)))


@pytest.mark.parametrize('thw,n_tiles', [((4, 64, 512), 1024), ((5, 40, 656), 1025),
                                         ((11, 80, 160), 1100)])
def test_select_around_the_key_list_sizes(thw, n_tiles):
    """The top-k sorts each lane's keys in registers, 16 of them up to 1,024
    columns and 32 above: the largest 16-key case, the smallest 32-key case
    and a ragged one, with ties, bit-exact against the oracle."""
    t, h, w = thw
    spec = ([(0, thw)], t * h * w, t * h * w, '1x8x16')
    lay, olay = _layouts(spec)
    assert lay.n_tiles == n_tiles
    g = torch.Generator().manual_seed(n_tiles)
    scores = torch.rand(2, lay.n_video_tiles, lay.n_tiles, generator=g)
    scores[1, ::5] = torch.randint(0, 4, (scores[1, ::5].shape), generator=g).float()  # ties
    _run(scores, lay, olay, pm.column_blocks(lay, pm.Budget(ratio=0.1)),
         om.column_blocks(olay, om.Budget(ratio=0.1)))
