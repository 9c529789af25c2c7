"""Pins the oracle's budgets, Bresenham rounding, selection, block mask and
index lists (oracle/mask.py) against the reference's known answers
(tests/unit/test_veda_predictor_mask.py, tests/unit/test_kernels_fa4.py),
`torch.topk` on distinct scores, and the selection rules."""

import math

import pytest
import torch

from oracle import mask as om
from oracle import tiling as ot


def _layout(target_grid=(7, 6, 10), shape='8x4x4', cond=None, text=90):
    spans, start = [], text
    if cond is not None:
        spans.append(ot.Span(start, cond, ot.least_padding(cond)))
        start += math.prod(cond)
    target = ot.Span(start + 40, target_grid, ot.Shape.parse(shape))
    used = target.start + target.rows
    return ot.build_layout(spans + [target], used, used)


@pytest.mark.parametrize('budget', [1.0, 2.3, 3.75, 5.5])
def test_bresenham_mean_equals_budget(budget):
    # reference test_veda_predictor_mask.py:65-72
    k_lo, _, frac = om.split_budget(budget, 64)
    extra = om.bresenham(400, frac)
    mean = (k_lo + extra.double()).mean().item()
    assert 0 <= budget - mean < 1.0 / 400


def test_equal_cost_budget_known_answers():
    # reference test_veda_predictor_mask.py:75-80
    assert om.Budget(ratio=0.1).per_row(37296, 330) == pytest.approx(0.1 * 292 ** 2 / 330)
    assert om.Budget(tiles=7).per_row(37296, 330) == 7.0
    assert om.Budget(ratio=1.0).keeps_all
    # 2.3 - 2 rounds to 0.3 exactly (mask.py:73-75)
    assert om.split_budget(2.3, 64) == (2, 3, 0.3)
    assert om.split_budget(70.0, 64) == (64, 64, 0.0)
    assert om.split_budget(0.4, 64)[0] == 1


def test_budget_known_answers_baseline_configs():
    # C1: 1024 tokens, 8 tiles, ratio 0.5 -> 4 per row
    assert om.split_budget(om.Budget(ratio=0.5).per_row(1024, 8), 8) == (4, 5, 0.0)
    # C2: n_ideal 451, 592 tiles, ratio 0.1
    b = om.Budget(ratio=0.1).per_row(57720, 592)
    k_lo, k_hi, frac = om.split_budget(b, 592)
    assert (k_lo, k_hi, frac) == (34, 35, 0.358277027027)
    extra = om.bresenham(592, frac)
    assert int(extra.sum()) == 212 and k_lo * 592 + int(extra.sum()) == 20340
    # C3: equal cost across the two shapes, ratio 0.2 on 57720 tokens
    for n in (518, 520):
        k_lo, _, frac = om.split_budget(om.Budget(ratio=0.2).per_row(57720, n), n)
        assert k_lo * n + int(om.bresenham(n, frac).sum()) == 40680
    # C5: target 159120 tokens, 1632 video tiles, ratio 0.05
    b = om.Budget(ratio=0.05).per_row(159120, 1632)
    k_lo, _, frac = om.split_budget(b, 1632)
    assert k_lo == 47 and int(om.bresenham(1632, frac).sum()) == 672
    assert k_lo * 1632 + 672 == 77376


def test_selection_rules():
    # reference test_veda_predictor_mask.py:83-104
    lay = _layout(target_grid=(16, 8, 16), shape='4x8x4')
    nv = lay.n_video_tiles
    scores = torch.randn(2, lay.n_tiles, lay.n_tiles, generator=torch.Generator().manual_seed(0))
    blocks = om.column_blocks(lay, om.Budget(ratio=0.3))
    index, keep = om.select_video_blocks(scores[:, :nv], lay, blocks)
    kept = keep.sum(-1).float()
    budget = blocks[0].budget.per_row(lay.target_tokens, nv)
    assert 0 <= budget - kept.double().mean().item() < 1.0 / nv
    mask = om.dense_block_mask(index, keep, lay)
    diag = torch.arange(nv)
    assert mask[:, diag, diag].all()
    assert torch.equal(mask[:, :nv, :nv].sum(-1).float(), kept)
    assert mask[:, :, nv:].all() and mask[:, nv:, :].all()
    s = scores[:, :nv, :nv].clone()
    s[:, diag, diag] = float('inf')
    top1 = s.topk(2, -1).indices[..., 1]
    assert torch.gather(mask[:, :nv], 2, top1[..., None]).all()


def test_segmented_blocks_have_independent_budgets():
    # reference test_veda_predictor_mask.py:107-124
    lay = _layout(target_grid=(16, 8, 16), cond=(1, 16, 32))
    n_ref, nv = lay.n_ref_tiles, lay.n_video_tiles
    blocks = om.column_blocks(lay, om.Budget(ratio=0.25), om.Budget(tiles=1))
    assert [(b.start, b.stop) for b in blocks] == [(0, n_ref), (n_ref, nv)]
    scores = torch.randn(1, nv, lay.n_tiles, generator=torch.Generator().manual_seed(1))
    mask = om.dense_block_mask(*om.select_video_blocks(scores, lay, blocks), lay)[0]
    assert (mask[:nv, :n_ref].sum(-1) == 1).all()
    assert mask[torch.arange(n_ref), torch.arange(n_ref)].all()
    t = torch.arange(n_ref, nv)
    assert mask[t, t].all()
    with pytest.raises(ValueError):
        om.column_blocks(lay, om.Budget(ratio=0.25))


@pytest.mark.parametrize('nan', [False, True])
@pytest.mark.parametrize('seed', range(4))
def test_selection_equals_torch_topk_on_distinct_scores(seed, nan):
    """The reference's selection is torch.topk; with distinct scores the
    oracle's stable order must give identical indices and keep flags. With
    `nan`, a third of the rows hold one NaN (either sign, so the order stays
    defined): torch.topk ranks it above +inf and `val > -inf` never keeps
    it; the oracle must agree."""
    lay = _layout(target_grid=(16, 8, 16), cond=(1, 16, 32))
    nv = lay.n_video_tiles
    g = torch.Generator().manual_seed(seed)
    scores = torch.rand(3, nv, lay.n_tiles, generator=g)
    assert scores.unique().numel() == scores.numel()
    if nan:
        hit = torch.rand(3, nv, generator=g) < 0.33
        col = torch.randint(0, lay.n_tiles, (3, nv), generator=g)
        sign = torch.where(torch.rand(3, nv, generator=g) < 0.5, -1.0, 1.0)
        val = torch.copysign(torch.full((3, nv), float('nan')), sign)
        scores.scatter_(-1, col[..., None], torch.where(hit, val, scores.gather(-1, col[..., None])[..., 0])[..., None])
        assert torch.isnan(scores).sum() == hit.sum()
    blocks = om.column_blocks(lay, om.Budget(ratio=0.25), om.Budget(tiles=2.5))
    index, keep = om.select_video_blocks(scores, lay, blocks)
    # the same selection written with torch.topk (mask.py:251-284)
    parts_i, parts_k = [], []
    rows = torch.arange(nv)
    for b in blocks:
        n_cols = b.stop - b.start
        s = scores[:, :, b.start:b.stop].clone()
        s.masked_fill_(~lay.kv_ok[None, None, b.start:b.stop], float('-inf'))
        own = (rows >= b.start) & (rows < b.stop)
        col = (rows - b.start).clamp(0, n_cols - 1)[None, :, None].expand(3, nv, 1)
        s.scatter_(-1, col, torch.where(own[None, :, None], float('inf'), s.gather(-1, col)))
        k_lo, k_hi, frac = om.split_budget(b.budget.per_row(b.real_tokens, n_cols), n_cols)
        vals, idx = torch.topk(s, k_hi, dim=-1, sorted=True)
        allowed = k_lo + om.bresenham(nv, frac).long()
        parts_k.append((torch.arange(k_hi)[None, None] < allowed[None, :, None]) & (vals > float('-inf')))
        parts_i.append(idx + b.start)
    assert torch.equal(index, torch.cat(parts_i, -1))
    assert torch.equal(keep, torch.cat(parts_k, -1))


def test_row_subset_follows_tile_ids():
    # reference test_veda_predictor_mask.py:127-150
    lay = _layout(target_grid=(16, 8, 16))
    blocks = om.column_blocks(lay, om.Budget(ratio=0.3))
    scores = torch.randn(2, lay.n_video_tiles, lay.n_tiles, generator=torch.Generator().manual_seed(2))
    fi, fk = om.select_video_blocks(scores, lay, blocks)
    rows = torch.tensor([1, 5, lay.n_video_tiles - 1])
    si, sk = om.select_video_blocks(scores[:, rows], lay, blocks, rows)
    assert torch.equal(si, fi[:, rows]) and torch.equal(sk, fk[:, rows])
    sub = om.dense_block_mask(si, sk, lay, global_rows=False)
    assert torch.equal(sub, om.dense_block_mask(fi, fk, lay)[:, rows])
    with pytest.raises(ValueError):
        om.dense_block_mask(si, sk, lay)


def _rebuild(cnt, idx, shape):
    out = torch.zeros(shape, dtype=torch.bool)
    for h in range(shape[0]):
        for i in range(shape[1]):
            out[h, i, idx[0, h, i, :cnt[0, h, i]].long()] = True
    return out


def test_index_lists_rebuild_the_mask():
    # reference tests/unit/test_kernels_fa4.py:13-46
    target = ot.Span(130, (7, 6, 10), ot.Shape.parse('8x4x4'))
    used = target.start + target.rows
    lay = ot.build_layout([target], used, used)
    assert lay.partial_tiles.numel() > 0
    scores = torch.randn(3, lay.n_tiles, lay.n_tiles, generator=torch.Generator().manual_seed(0))
    blocks = om.column_blocks(lay, om.Budget(ratio=0.5))
    mask = om.dense_block_mask(*om.select_video_blocks(scores[:, :lay.n_video_tiles], lay, blocks), lay)
    pc, pi, fc, fi = om.index_lists(mask, lay)
    full = _rebuild(fc, fi, mask.shape)
    part = _rebuild(pc, pi, mask.shape)
    assert not (full & part).any()
    assert torch.equal(full, mask & lay.full_tile)
    assert torch.equal(full | part, mask & lay.kv_ok)
    for h in range(mask.shape[0]):
        for i in range(mask.shape[1]):
            for cnt, idx in ((fc, fi), (pc, pi)):
                row = idx[0, h, i]
                members, rest = row[:cnt[0, h, i]], row[cnt[0, h, i]:]
                assert torch.equal(members, members.sort().values)
                assert torch.equal(rest, rest.sort().values)
                assert torch.equal(row.sort().values, torch.arange(mask.shape[2], dtype=torch.int32))
