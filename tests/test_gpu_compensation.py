"""GPU parity of the zero-order compensation (`kernels.zero_order_compensation`,
`kernels.compensated_attention`) against the oracle's restatement of
miowtion/veda/attention.py:591-689.

The kernel rounds the tile summaries to bf16, as the reference's own kernel
does (compensation_triton.py:80-99, its one deliberate numeric difference);
it is compared with the oracle on bf16 summaries tightly and with the fp32
torch form to the attention bar (max-abs 2e-2, rel-L2 1e-2). The exactness
case (every dropped tile holds one key) is compared with dense attention.
"""

import pytest
import torch

from miowtion_amd import attention as pa
from miowtion_amd import kernels
from miowtion_amd import mask as pm
from miowtion_amd import plan as pplan
from miowtion_amd import predictor as pp
from miowtion_amd import tiling as pt
from oracle import attention as oa
from oracle import tiling as ot
from tests import helpers

pytestmark = pytest.mark.gpu


def _bar(got, want):
    d = got.float() - want.float()
    assert d.abs().max().item() <= 2e-2, d.abs().max().item()
    assert (d.norm() / want.float().norm()).item() <= 1e-2


def _case(seed=0, heads=4, density=0.4):
    spec = helpers.small_layout()
    lay = helpers.product_layout(*spec, device='cuda')
    olay = helpers.oracle_layout(*spec)
    q, k, v = helpers.qkv(lay.seq_len, heads, 128, seed=seed)
    hs = torch.arange(heads)
    qt, kt, vt = (ot.gather_tiles(t, olay, hs) for t in (q, k, v))
    n = olay.n_tiles
    g = torch.Generator().manual_seed(seed)
    mask = torch.rand(heads, n, n, generator=g) < density
    mask |= torch.eye(n, dtype=torch.bool)[None]
    mask &= olay.kv_ok[None, None, :]
    return lay, olay, qt, kt, vt, mask


def test_summaries_match_oracle():
    lay, olay, qt, kt, vt, mask = _case()
    kc, vc = kernels.tile_summaries(kt.cuda(), vt.cuda(), lay)
    okc, ovc = oa.tile_summaries(kt, vt, olay.valid_count, torch.float32)
    # fp32 sums in a different order, then one bf16 rounding
    torch.testing.assert_close(kc.cpu().float(), okc, rtol=8e-3, atol=1e-6)
    torch.testing.assert_close(vc.cpu().float(), ovc, rtol=8e-3, atol=1e-5)


def test_compensation_matches_oracle():
    lay, olay, qt, kt, vt, mask = _case()
    o, lse = kernels.block_sparse_attention(qt.cuda(), kt.cuda(), vt.cuda(), mask.cuda(), lay,
                                            return_lse=True)
    got = kernels.zero_order_compensation(o, lse, qt.cuda(), kt.cuda(), vt.cuda(), mask.cuda(),
                                          lay).cpu()
    o_c, lse_c = o.cpu(), lse.cpu()
    want16 = oa.zero_order_compensation(o_c, lse_c, qt, kt, vt, mask, olay.valid_count,
                                        torch.bfloat16)
    want32 = oa.zero_order_compensation(o_c, lse_c, qt, kt, vt, mask, olay.valid_count)
    torch.testing.assert_close(got.float(), want16.float(), rtol=1e-2, atol=4e-3)
    _bar(got, want32)
    # the term is present: the output moved away from o_kept
    assert (got.float() - o_c.float()).abs().max() > 5e-2
    # the one-pass form (kept = mask & kv_ok) keeps o_kept in fp32: the same
    # result up to that bf16 rounding
    both = kernels.compensated_attention(qt.cuda(), kt.cuda(), vt.cuda(), mask.cuda(), lay).cpu()
    torch.testing.assert_close(both.float(), got.float(), rtol=1e-2, atol=4e-3)
    _bar(both, want32)


def test_narrow_tiles_and_zero_rows_match_oracle():
    """Query tiles whose only non-zero rows are their first 32 take the
    narrow compensation (waves 0 and 1 split the real rows' virtual keys,
    waves 2 and 3 sum the dropped tiles' V sums and weights, which every
    all-zero row scales by its own exp2(-lse_kept)); other all-zero
    groups take the product-free step. Here rows 32..127 of three full
    tiles are zero (one of them keeps nothing), a 24-row tile too, and
    every all-zero row gets its own o_kept and lse_kept, so the per-row
    scaling is checked. Every row against the oracle on bf16 summaries."""
    lay, olay, qt, kt, vt, mask = _case(2)
    full = [int(t) for t in torch.nonzero(olay.valid_count == 128).flatten()[:4]]
    qt = qt.clone()
    for t in full[:3]:
        qt[t * 128 + 32:(t + 1) * 128] = 0
    qt[full[3] * 128 + 24:(full[3] + 1) * 128] = 0
    mask[:, full[2]] = False
    g = torch.Generator().manual_seed(5)
    o = torch.randn(qt.shape, generator=g).to(torch.bfloat16)
    lse = torch.randn(qt.shape[1], qt.shape[0], generator=g) * 2 + 3
    lse[0, full[0] * 128 + 40] = float('-inf')  # a zero row that kept nothing
    got = kernels.zero_order_compensation(o.cuda(), lse.cuda(), qt.cuda(), kt.cuda(), vt.cuda(),
                                          mask.cuda(), lay).cpu()
    want16 = oa.zero_order_compensation(o, lse, qt, kt, vt, mask, olay.valid_count,
                                        torch.bfloat16)
    torch.testing.assert_close(got.float(), want16.float(), rtol=1e-2, atol=4e-3)
    rows = torch.cat([torch.arange(t * 128, (t + 1) * 128) for t in full])
    torch.testing.assert_close(got.float()[rows], want16.float()[rows], rtol=1e-2, atol=4e-3)
    assert (got.float()[rows] - o.float()[rows]).abs().max() > 5e-2


def test_exact_when_dropped_tiles_hold_one_key():
    lay, olay, qt, kt, vt, mask = _case(1)
    n = olay.n_tiles
    k_same = kt.clone().view(n, 128, *kt.shape[1:])
    real = (torch.arange(128)[None, :] < olay.valid_count[:, None])
    k_same[:] = torch.where(real[:, :, None, None], k_same[:, :1], torch.zeros((), dtype=kt.dtype))
    k_same = k_same.view_as(kt)
    got = kernels.compensated_attention(qt.cuda(), k_same.cuda(), vt.cuda(), mask.cuda(),
                                        lay).cpu()
    full = oa.block_sparse_attention(qt, k_same, vt, torch.ones_like(mask), olay.valid_count)
    _bar(got, full)


def test_one_pass_row_that_kept_nothing():
    """A query tile whose mask row is empty: the one-pass kernel gives the
    reference's num / (1 + den) at reference 0 (attention.py:640-650)."""
    lay, olay, qt, kt, vt, mask = _case(3)
    m = mask.clone()
    m[0, 1] = False
    m[2, 0] = False
    got = kernels.compensated_attention(qt.cuda(), kt.cuda(), vt.cuda(), m.cuda(), lay).cpu()
    o, lse = oa.block_sparse_attention(qt, kt, vt, m & olay.kv_ok, olay.valid_count,
                                       return_lse=True)
    assert torch.isinf(lse[0, 128:256]).all()
    want = oa.zero_order_compensation(o, lse, qt, kt, vt, m & olay.kv_ok, olay.valid_count,
                                      torch.bfloat16)
    _bar(got, want.float())
    _bar(got[128:256, 0], want[128:256, 0].float())


def test_nothing_dropped_returns_o_kept():
    lay, olay, qt, kt, vt, mask = _case(2)
    allm = olay.kv_ok[None, None, :].expand_as(mask).clone().cuda()
    o, lse = kernels.block_sparse_attention(qt.cuda(), kt.cuda(), vt.cuda(), allm, lay,
                                            return_lse=True)
    got = kernels.zero_order_compensation(o, lse, qt.cuda(), kt.cuda(), vt.cuda(), allm, lay)
    assert torch.equal(got, o)


def test_rejects_bad_shapes():
    lay, olay, qt, kt, vt, mask = _case()
    o = qt.cuda()
    lse = torch.zeros(4, qt.shape[0], device='cuda')
    with pytest.raises(ValueError, match='block_mask'):
        kernels.zero_order_compensation(o, lse, qt.cuda(), kt.cuda(), vt.cuda(),
                                        mask[:, :-1].cuda(), lay)
    with pytest.raises(ValueError, match='lse_kept'):
        kernels.zero_order_compensation(o, lse[:, :-1], qt.cuda(), kt.cuda(), vt.cuda(),
                                        mask.cuda(), lay)


def test_sparse_student_with_compensation():
    spec = helpers.small_layout(grid=(4, 16, 16), shape='2x8x8', text=0, extra=0)
    spans, used, seq_len, shape = spec
    H = 4
    layout = pa.PackedLayout((pa.VideoSpan(spans[0][0], spans[0][1]),), used, seq_len)
    cfg = pa.VedaConfig(target_budget=pm.Budget(ratio=0.3), zero_order_compensation=True)
    clip = pa.ClipTiling(layout, cfg, 'cuda')
    plan = pplan.TilePlan('c', spans[0][1], [pt.TileShape.parse(shape)], [[0] * H])
    pred = pp.TileScorePredictor([pp.LayerPredictor.random(
        H, 128, std=0.02, generator=torch.Generator().manual_seed(4), device='cuda')])
    student = pa.SparseStudent(clip, plan, pred)
    q, k, v = helpers.qkv(seq_len, H, 128, seed=6)
    out = student(q.cuda(), k.cuda(), v.cuda(), 0).cpu()
    part = student.last['parts'][0]
    olay = helpers.oracle_layout(*spec)
    hs = torch.arange(H)
    qt, kt, vt = (ot.gather_tiles(t, olay, hs) for t in (q, k, v))
    sel = part['selection']
    mask = pm.dense_block_mask(sel, clip.get(pt.TileShape.parse(shape))).cpu()
    mask &= olay.kv_ok[None, None, :]
    o, lse = oa.block_sparse_attention(qt, kt, vt, mask, olay.valid_count, return_lse=True)
    comp = oa.zero_order_compensation(o, lse, qt, kt, vt, mask, olay.valid_count)
    want = torch.zeros(seq_len + 1, H, 128, dtype=comp.dtype)
    ot.scatter_tiles_(want, comp, olay, None)
    _bar(out[:used], want[:used])


def test_config2_sampled_query_tiles():
    """BASELINE config 2 geometry, 2 heads, keep 0.1: the compensation of
    every query tile on the GPU against the oracle on a sample of tiles."""
    spans, used, seq_len, shape = helpers.CONFIGS['C2']
    lay = helpers.product_layout(spans, used, seq_len, shape, device='cuda')
    H = 2
    print(f'C2 compensation: {lay.n_tiles} tiles, {H} heads', flush=True)
    g = torch.Generator(device='cuda').manual_seed(2)
    q, k, v = (torch.randn(seq_len, H, 128, generator=g, device='cuda').to(torch.bfloat16)
               for _ in range(3))
    qt, kt, vt = (kernels.gather_tiles(t, lay, None) for t in (q, k, v))
    scores = torch.rand(H, lay.n_tiles, lay.n_tiles, generator=g, device='cuda')
    sel = pm.select_video_blocks(scores, lay, pm.column_blocks(lay, pm.Budget(ratio=0.1)))
    mask = pm.dense_block_mask(sel, lay) & lay.kv_ok[None, None, :]
    o, lse = kernels.block_sparse_attention(qt, kt, vt, mask, lay, return_lse=True)
    got = kernels.zero_order_compensation(o, lse, qt, kt, vt, mask, lay)
    tiles = torch.arange(0, lay.n_tiles, 53)
    rows = (tiles[:, None] * 128 + torch.arange(128)[None, :]).reshape(-1)
    kt_c, vt_c = kt.cpu(), vt.cpu()
    want = oa.zero_order_compensation(o.cpu()[rows], lse.cpu()[:, rows], qt.cpu()[rows], kt_c,
                                      vt_c, mask.cpu()[:, tiles], lay.valid_count.cpu(),
                                      torch.bfloat16)
    torch.testing.assert_close(got.cpu()[rows].float(), want.float(), rtol=1e-2, atol=4e-3)
    # the one-pass form on the same inputs
    one = kernels.compensated_attention(qt, kt, vt, mask, lay)
    torch.testing.assert_close(one.cpu()[rows].float(), want.float(), rtol=1e-2, atol=8e-3)
