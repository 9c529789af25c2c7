"""The layout-level API driven with a layout that carries only the
reference's fields.

The reference's `TileLayout` (miowtion/veda/tiling.py:159-211) is a plain
dataclass of 16 attributes plus the `n_tiles` and `num_slots` properties; a
caller that builds it with the reference's own `build_tile_layout` hands that
object to the kernel wrappers. `RefTileLayout` below is exactly that shape,
filled from a product layout, and every entry point of `miowtion_amd.kernels`
(and `TileScorePredictor.scores`, predictor.py:387-410) runs through it
against the oracle: nothing may read an attribute the reference's layout
does not have.
"""

import dataclasses
import math

import pytest
import torch

from miowtion_amd import kernels
from miowtion_amd import mask as pm
from miowtion_amd import predictor as pp
from miowtion_amd import tiling as pt
from oracle import attention as oa
from oracle import mask as om
from oracle import predictor as op
from oracle import tiling as ot
from tests import helpers

# the attributes of miowtion/veda/tiling.py:197-212, in their order
REFERENCE_FIELDS = ('perm', 'valid_count', 'n_video_tiles', 'n_ref_tiles', 'n_global_tiles',
                    'ref_tokens', 'target_tokens', 'used', 'seq_len', 'gather_index',
                    'scatter_index', 'pad_slots', 'partial_tiles', 'kv_ok', 'full_tile',
                    'slot_valid')


@dataclasses.dataclass
class RefTileLayout:
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
        return self.n_tiles * 128


def test_product_layout_has_exactly_the_reference_fields():
    assert tuple(f.name for f in dataclasses.fields(pt.TileLayout)) == REFERENCE_FIELDS
    assert tuple(f.name for f in dataclasses.fields(RefTileLayout)) == REFERENCE_FIELDS


def test_layout_cache_is_dropped_with_the_layout():
    import gc
    spec = helpers.small_layout()
    lay = RefTileLayout(**{f: getattr(helpers.product_layout(*spec), f) for f in REFERENCE_FIELDS})
    key = id(lay)
    a = pt.layout_cached(lay, 'x', lambda: torch.arange(3))
    assert pt.layout_cached(lay, 'x', lambda: torch.arange(5)) is a
    del lay
    gc.collect()
    assert key not in pt._DERIVED


def _case(heads=4, seed=3):
    spec = helpers.small_layout()
    prod = helpers.product_layout(*spec, device='cuda')
    lay = RefTileLayout(**{f: getattr(prod, f) for f in REFERENCE_FIELDS})
    olay = helpers.oracle_layout(*spec)
    q, k, v = helpers.qkv(lay.seq_len, heads, 128, seed=seed)
    return lay, olay, q, k, v


def _bar(got, want, abs_tol=2e-2, rel_tol=1e-2):
    d = got.cpu().float() - want.float()
    assert d.abs().max().item() <= abs_tol, d.abs().max().item()
    assert (d.norm() / want.float().norm()).item() <= rel_tol


def _mask(olay, heads, seed, density=0.35):
    n = olay.n_tiles
    g = torch.Generator().manual_seed(seed)
    m = torch.rand(heads, n, n, generator=g) < density
    return (m | torch.eye(n, dtype=torch.bool)[None]) & olay.kv_ok[None, None, :]


@pytest.mark.gpu
def test_gather_pool_scatter_and_lse():
    lay, olay, q, _, _ = _case()
    heads = torch.tensor([2, 0, 3])
    hc = heads.cuda()
    ref_rows = ot.gather_tiles(q, olay, heads)
    assert torch.equal(kernels.gather_tiles(q.cuda(), lay, hc).cpu(), ref_rows)
    rows, feats, sq, var = kernels.gather_and_pool(q.cuda(), lay, hc, second=True)
    assert torch.equal(rows.cpu(), ref_rows)
    ref_feats = op.pool_tiles(ref_rows, olay)
    assert torch.equal(feats.cpu()[..., 128:], ref_feats[..., 128:])
    torch.testing.assert_close(feats.cpu()[..., :128], ref_feats[..., :128], rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(sq.cpu(), op.pool_tiles(ref_rows, olay, 'raw'), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(var.cpu(), op.pool_tiles(ref_rows, olay, 'central'),
                               rtol=1e-4, atol=1e-5)
    # first-order pooling (packed max / min, its own summation order of the
    # mean) against the second-moment form's features
    for first in (kernels.pool_seq(q.cuda(), lay, hc)[0], kernels.pool_tiles(rows, lay)):
        assert torch.equal(first[..., 128:], feats[..., 128:])
        torch.testing.assert_close(first[..., :128], feats[..., :128], rtol=1e-5, atol=1e-6)
    assert torch.equal(kernels.pool_tiles(rows, lay, 'raw'), sq)
    assert torch.equal(kernels.pool_tiles(rows, lay, 'central'), var)
    out = torch.zeros(lay.seq_len + 1, *q.shape[1:], dtype=q.dtype, device='cuda')
    kernels.scatter_tiles_(out, rows, lay, hc)
    out_ref = torch.zeros(lay.seq_len + 1, *q.shape[1:], dtype=q.dtype)
    ot.scatter_tiles_(out_ref, ref_rows, olay, heads)
    assert torch.equal(out[:lay.seq_len].cpu(), out_ref[:lay.seq_len])
    lse = torch.randn(lay.seq_len, 4, generator=torch.Generator().manual_seed(5))
    assert torch.equal(kernels.gather_lse(lse.cuda(), lay, hc).cpu(), ot.gather_lse(lse, olay, heads))


@pytest.mark.gpu
def test_selection_lists_attention_and_gradients():
    lay, olay, q, k, v = _case()
    hs = torch.arange(4)
    qt, kt, vt = (ot.gather_tiles(t, olay, hs) for t in (q, k, v))
    scores = torch.rand(4, olay.n_video_tiles, olay.n_video_tiles,
                        generator=torch.Generator().manual_seed(8))
    sel = pm.select_video_blocks(scores.cuda(), lay, pm.column_blocks(lay, pm.Budget(ratio=0.3)))
    idx, keep = om.select_video_blocks(scores, olay, om.column_blocks(olay, om.Budget(ratio=0.3)))
    assert torch.equal(sel.index.cpu(), idx) and torch.equal(sel.keep.cpu(), keep)
    mask = pm.dense_block_mask(sel, lay)
    assert torch.equal(mask.cpu(), om.dense_block_mask(idx, keep, olay))
    for transpose in (False, True):
        for a, b in zip(kernels.index_lists(mask, lay, transpose),
                        om.index_lists(mask.cpu(), olay, transpose)):
            assert torch.equal(a.cpu(), b)
    ts = [t.cuda().requires_grad_(True) for t in (qt, kt, vt)]
    out, lse = kernels.block_sparse_attention(*ts, mask, lay, return_lse=True)
    ref, ref_lse = oa.block_sparse_attention(qt, kt, vt, mask.cpu(), olay.valid_count,
                                             return_lse=True)
    _bar(out.detach(), ref)
    fin = torch.isfinite(ref_lse)
    assert torch.equal(torch.isfinite(lse.detach().cpu()), fin)
    assert (lse.detach().cpu()[fin] - ref_lse[fin]).abs().max() <= 2e-2
    dout = torch.randn(qt.shape, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    out.backward(dout.cuda())
    want = oa.block_sparse_attention_grads(qt, kt, vt, mask.cpu(), olay.valid_count, dout.float())
    for t, w in zip(ts, want):
        _bar(t.grad, w, abs_tol=3e-2)
    # the sequence-order forward (gather of q, attention, scatter in one kernel)
    lists = kernels.index_lists(mask, lay)
    got = torch.zeros(lay.seq_len + 1, 4, 128, dtype=torch.bfloat16, device='cuda')
    kernels.block_sparse_attention_seq_(got, q.cuda(), kt.cuda(), vt.cuda(), lists, lay, None)
    back = torch.zeros(lay.seq_len + 1, 4, 128, dtype=torch.bfloat16)
    ot.scatter_tiles_(back, ref, olay, None)
    _bar(got[:lay.seq_len], back[:lay.seq_len])


@pytest.mark.gpu
def test_heat_dense_and_compensation():
    lay, olay, q, k, v = _case(seed=11)
    hs = torch.arange(4)
    ref_dense, lse = oa.dense_attention(q, k, v, lay.used, return_lse=True)
    dense, dense_lse = kernels.dense_attention(q.cuda(), k.cuda(), v.cuda(), lay.used,
                                               return_lse=True)
    _bar(dense, ref_dense)
    assert (dense_lse.cpu() - lse).abs().max() <= 2e-2
    qt, kt, vt = (ot.gather_tiles(t, olay, hs) for t in (q, k, v))
    lse_t = ot.gather_lse(lse, olay, hs)
    rows = torch.arange(0, olay.n_tiles, 2)
    heat = kernels.teacher_heat(qt.cuda(), kt.cuda(), lse_t.cuda(), lay, rows.cuda(), 'sum')
    want = oa.teacher_heat(qt, kt, lse_t, olay, rows, 'sum', score_dtype=torch.float32)
    torch.testing.assert_close(heat.cpu(), want, rtol=1e-4, atol=1e-7)
    fused, flse, _ = kernels.dense_heat(qt.cuda(), kt.cuda(), lay, rows.cuda(), 'sum')
    torch.testing.assert_close(fused.cpu(), want, rtol=1e-4, atol=1e-7)
    mask = _mask(olay, 4, 12)
    kc, vc = kernels.tile_summaries(kt.cuda(), vt.cuda(), lay)
    okc, ovc = oa.tile_summaries(kt, vt, olay.valid_count, torch.float32)
    torch.testing.assert_close(kc.cpu().float(), okc, rtol=8e-3, atol=1e-6)
    torch.testing.assert_close(vc.cpu().float(), ovc, rtol=8e-3, atol=1e-5)
    o, ol = kernels.block_sparse_attention(qt.cuda(), kt.cuda(), vt.cuda(), mask.cuda(), lay,
                                           return_lse=True)
    comp = kernels.zero_order_compensation(o, ol, qt.cuda(), kt.cuda(), vt.cuda(), mask.cuda(), lay)
    want = oa.zero_order_compensation(o.cpu(), ol.cpu(), qt, kt, vt, mask, olay.valid_count,
                                      torch.bfloat16)
    _bar(comp, want)
    one = kernels.compensated_attention(qt.cuda(), kt.cuda(), vt.cuda(), mask.cuda(), lay)
    o_ref, l_ref = oa.block_sparse_attention(qt, kt, vt, mask, olay.valid_count, return_lse=True)
    _bar(one, oa.zero_order_compensation(o_ref, l_ref, qt, kt, vt, mask, olay.valid_count))


@pytest.mark.gpu
def test_predictor_scores():
    lay, olay, q, k, _ = _case(seed=13)
    heads = torch.tensor([1, 3])
    g = torch.Generator().manual_seed(14)
    layer = pp.LayerPredictor.random(4, 128, std=0.02, generator=g, device='cuda',
                                     second_order_rank=8, count_term=True, fp8=True)
    pred = pp.TileScorePredictor([layer])
    qt = kernels.gather_tiles(q.cuda(), lay, heads.cuda())
    kt = kernels.gather_tiles(k.cuda(), lay, heads.cuda())
    got = pred.scores(0, qt, kt, lay, heads.cuda()).cpu()
    oq, ok = ot.gather_tiles(q, olay, heads), ot.gather_tiles(k, olay, heads)

    def w(pw):
        return op.dequantize_fp8(pw.values.cpu(), pw.scale.cpu())

    want = op.logits(op.pool_tiles(oq, olay), op.pool_tiles(ok, olay), w(layer.proj_q),
                     w(layer.proj_k), heads, gain=layer.count_gain.cpu(),
                     log_count=torch.log(olay.valid_count.clamp(min=1).float()),
                     sq_q=op.pool_tiles(oq, olay, 'raw'), var_k=op.pool_tiles(ok, olay, 'central'),
                     so_q=w(layer.so_q), so_k=w(layer.so_k))
    assert (got - want).abs().max() <= 1e-4 * want.abs().max() + 1e-6
    assert math.isfinite(got.abs().max().item())
