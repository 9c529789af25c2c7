"""GPU parity of the teacher's fused dense pass in tile order
(`kernels.dense_heat`: one pass gives the row LSE, the block heat and, with
v, the dense output).

Oracle: the reference semantics restated in oracle/attention.py -- dense
attention with LSE (miowtion/h3/attention.py:18-102) gathered to tile order,
and the block heat from that LSE (miowtion/veda/heatmap.py:36-110). 'sum' is
compared with fp32 scores to 1e-4 relative (BASELINE config 5's bar); 'max'
against the bf16-rounded row max the reference takes (the max commutes with
the rounding, block_heat_triton.py:131-133) to 2e-3. At full config-5 size
the size-independent identity sum_j heat_sum[i, j] = valid_count[i] (every
real row's probabilities over all keys sum to 1) is checked, and the fused
heat is compared with the two-pass kernels (dense LSE, then the heat kernel).
"""

import pytest
import torch

from miowtion_amd import kernels
from miowtion_amd import ops
from oracle import attention as oa
from oracle import tiling as ot
from tests import helpers

pytestmark = pytest.mark.gpu


def _case(heads=4, seed=0):
    spec = helpers.small_layout()
    lay = helpers.product_layout(*spec, device='cuda')
    olay = helpers.oracle_layout(*spec)
    q, k, v = helpers.qkv(lay.seq_len, heads, 128, seed=seed)
    _, lse = oa.dense_attention(q, k, v, lay.used, return_lse=True)
    hs = torch.arange(heads)
    qt, kt, vt = (ot.gather_tiles(t, olay, hs) for t in (q, k, v))
    lse_t = ot.gather_lse(lse, olay, hs)
    return lay, olay, qt, kt, vt, lse_t


def _rows_valid(olay, rows):
    vc = olay.valid_count[rows]
    return (torch.arange(128)[None, :] < vc[:, None]).reshape(-1)


@pytest.mark.parametrize('reduce', ['sum', 'max'])
@pytest.mark.parametrize('with_v', [False, True])
def test_dense_heat_matches_oracle(reduce, with_v):
    lay, olay, qt, kt, vt, lse_t = _case()
    # video tiles, a partial tile, the first and last global tiles
    rows = torch.cat([torch.arange(0, olay.n_video_tiles, 2),
                      torch.tensor([olay.n_tiles - 1, olay.n_video_tiles])]).unique()
    heat, lse, out = kernels.dense_heat(qt.cuda(), kt.cuda(), lay, rows.cuda(), reduce,
                                        v=vt.cuda() if with_v else None)
    heat, lse = heat.cpu(), lse.cpu()
    if reduce == 'sum':
        ref = oa.teacher_heat(qt, kt, lse_t, olay, rows, 'sum', score_dtype=torch.float32)
        torch.testing.assert_close(heat, ref, rtol=1e-4, atol=1e-7)
        torch.testing.assert_close(heat.sum(-1), olay.valid_count[rows].float().expand(4, -1),
                                   rtol=1e-4, atol=1e-4)
    else:
        ref = oa.teacher_heat(qt, kt, lse_t, olay, rows, 'max', score_dtype=torch.bfloat16)
        torch.testing.assert_close(heat, ref, rtol=2e-3, atol=1e-7)
    # LSE of the real rows equals the dense teacher's, gathered to tile order
    sel = (rows[:, None] * 128 + torch.arange(128)[None, :]).reshape(-1)
    real = _rows_valid(olay, rows)
    want = lse_t[sel].t()  # [H', R * 128]
    torch.testing.assert_close(lse[:, real], want[:, real], rtol=0, atol=2e-4)
    if with_v:
        mask = torch.ones(4, rows.numel(), olay.n_tiles, dtype=torch.bool)
        ref_o = oa.block_sparse_attention(qt[sel], kt, vt, mask, olay.valid_count)
        d = (out.cpu().float() - ref_o.float())
        assert d.abs().max().item() <= 2e-2
        assert (d.norm() / ref_o.float().norm()).item() <= 1e-2
    else:
        assert out is None


def test_dense_heat_sum_with_a_late_score_jump():
    """'sum' keeps a row's reference while the step sums stay in range: a key
    tile late in the walk whose scores jump far past every earlier one (K
    scaled by 30: ~130 log2 units above the running max, so its
    probabilities would overflow) makes those steps raise the reference, and
    the LSE and heat still match the oracle on tile-ordered data."""
    lay, olay, qt, kt, vt, _ = _case()
    j = olay.n_video_tiles - 3
    kt = kt.clone()
    kt[j * 128:(j + 1) * 128] = (kt[j * 128:(j + 1) * 128].float() * 30).to(kt.dtype)
    full = torch.ones(4, olay.n_tiles, olay.n_tiles, dtype=torch.bool)
    _, ref_lse = oa.block_sparse_attention(qt, kt, vt, full, olay.valid_count, return_lse=True)
    rows = torch.arange(0, olay.n_video_tiles)
    heat, lse, _ = kernels.dense_heat(qt.cuda(), kt.cuda(), lay, rows.cuda(), 'sum')
    heat, lse = heat.cpu(), lse.cpu()
    sel = (rows[:, None] * 128 + torch.arange(128)[None, :]).reshape(-1)
    real = _rows_valid(olay, rows)
    want = ref_lse[:, sel]
    torch.testing.assert_close(lse[:, real], want[:, real], rtol=0, atol=2e-4)
    ref = oa.teacher_heat(qt, kt, ref_lse.t().contiguous(), olay, rows, 'sum',
                          score_dtype=torch.float32)
    torch.testing.assert_close(heat, ref, rtol=1e-4, atol=1e-7)
    # the scaled tile takes most of the mass of many rows
    assert (heat[:, :, j] > 0.5 * olay.valid_count[rows].float()).float().mean() > 0.1


def test_dense_heat_head_chunks_and_empty_key_tile_are_exact():
    """Heads are independent: a workspace that forces one head per chunk
    gives the same bits. A key tile with no real row (valid count zeroed
    here) gets zero heat and no LSE mass."""
    lay, olay, qt, kt, vt, lse_t = _case()
    rows = torch.arange(olay.n_video_tiles).cuda()
    vc = lay.valid_count.clone()
    vc[3] = 0
    q, k = qt.cuda(), kt.cuda()
    for reduce in ('sum', 'max'):
        full = ops.dense_heat(q, k, None, vc, rows, reduce)
        small = ops.dense_heat(q, k, None, vc, rows, reduce, workspace_bytes=1)
        assert torch.equal(full[0], small[0]) and torch.equal(full[1], small[1])
        assert torch.equal(full[0][:, :, 3], torch.zeros_like(full[0][:, :, 3]))
    heat = full[0] if reduce == 'sum' else ops.dense_heat(q, k, None, vc, rows, 'sum')[0]
    want = vc[rows.long()].float()
    torch.testing.assert_close(heat.sum(-1), want.expand(4, -1), rtol=1e-4, atol=1e-4)


def test_dense_heat_rejects_bad_arguments():
    lay, olay, qt, kt, vt, lse_t = _case()
    rows = torch.arange(4).cuda()
    with pytest.raises(ValueError, match='reduce'):
        kernels.dense_heat(qt.cuda(), kt.cuda(), lay, rows, 'mean')
    with pytest.raises(ValueError, match='q_tiles'):
        kernels.dense_heat(qt.cuda(), kt.cuda(), lay, torch.tensor([lay.n_tiles]).cuda(), 'sum')
    with pytest.raises(NotImplementedError):
        kernels.dense_heat(qt, kt, lay, rows.cpu(), 'sum')


def test_dense_heat_config5_row_mass_and_two_pass_agreement():
    """BASELINE config 5 geometry (2,048 global rows + 102x30x52 video,
    (1,8,16) tiles), 2 heads: the fused heat of all video query tiles
    satisfies the row-mass identity, and matches the two-pass kernels
    (dense LSE, heat kernel) on a sample of query tiles."""
    spans, used, seq_len, shape = helpers.CONFIGS['C5']
    lay = helpers.product_layout(spans, used, seq_len, shape, device='cuda')
    H = 2
    print(f'C5 dense_heat: {lay.n_tiles} tiles, {H} heads', flush=True)
    g = torch.Generator(device='cuda').manual_seed(5)
    q, k, v = (torch.randn(seq_len, H, 128, generator=g, device='cuda').to(torch.bfloat16)
               for _ in range(3))
    for t in (q, k, v):
        t[used:] = 0
    qt, kt = (kernels.gather_tiles(t, lay, None) for t in (q, k))
    rows = torch.arange(lay.n_video_tiles, device='cuda')
    heat, lse, _ = kernels.dense_heat(qt, kt, lay, rows, 'sum')
    want = lay.valid_count[rows].float()
    torch.testing.assert_close(heat.sum(-1), want.expand(H, -1), rtol=2e-4, atol=2e-3)
    _, lse_d = kernels.dense_attention(q, k, v, used, return_lse=True)
    lse_t = kernels.gather_lse(lse_d, lay, torch.arange(H, device='cuda'))
    sample = rows[::97]
    ref = kernels.teacher_heat(qt, kt, lse_t, lay, sample, 'sum')
    torch.testing.assert_close(heat[:, ::97], ref, rtol=1e-4, atol=1e-7)
