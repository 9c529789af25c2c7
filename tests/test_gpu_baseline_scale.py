"""Parity at the BASELINE configurations' full sizes, sampled.

Every check runs the product at the real size (all 48 heads, the real
geometry) and compares a sample -- two heads, a few query tiles -- with the
CPU oracle, so the oracle's cost stays a few seconds per test:

  * dense forward + LSE at C2 (57,720 rows) and C5 (161,168 rows, 2,048 of
    them global), the reference's own bar (tests/gpu/test_kernels_gpu.py:
    32-41: out to 2e-2, LSE to rtol = atol = 1e-3);
  * the C3 layer (37x52x30, 48 heads, a seeded per-head choice of (1,8,16) or
    (4,4,8), keep 0.2) through SparseStudent: block lists bit-exact for every
    head on the kernel's logits, sampled query tiles of both groups against
    the oracle output;
  * the C5 chain (fused teacher pass -> heat -> top-k at 0.05 -> sparse)
    through OracleStudent: the tile-order LSE and the heat of sampled tiles
    against the oracle, the selection bit-exact for every head on the
    kernel's heat, and sampled output tiles, a global (dense) query tile
    among them.
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
from oracle import mask as om
from oracle import tiling as ot
from tests import helpers
from tests.test_gpu_attention import _close

pytestmark = pytest.mark.gpu

H = 48
SAMPLE_HEADS = [0, 47]


def _qkv_cuda(seq_len, seed, used=None):
    g = torch.Generator(device='cuda').manual_seed(seed)
    out = [torch.randn(seq_len, H, 128, generator=g, device='cuda').to(torch.bfloat16)
           for _ in range(3)]
    if used is not None:
        for t in out:
            t[used:] = 0
    return out


def _tile_rows(tiles):
    tiles = torch.as_tensor(tiles)
    return (tiles[:, None] * 128 + torch.arange(128)[None, :]).reshape(-1)


@pytest.mark.parametrize('name', ['C2', 'C5'])
def test_dense_forward_and_lse_at_full_size(name):
    spans, used, seq_len, _ = helpers.CONFIGS[name]
    print(f'{name} dense: {seq_len} rows ({used} real), {H} heads', flush=True)
    q, k, v = _qkv_cuda(seq_len, seed=11)
    out, lse = kernels.dense_attention(q, k, v, used, return_lse=True)
    assert (out[used:] == 0).all() and (lse[used:] == 0).all()
    mid = used // 2
    rows = torch.cat([torch.arange(0, 128), torch.arange(mid, mid + 64),
                      torch.arange(used - 128, seq_len)])
    if name == 'C5':        # the global rows end at 2,048; video rows follow
        rows = torch.cat([rows, torch.arange(2048 - 64, 2048 + 64)])
    hs = SAMPLE_HEADS
    qc, kc, vc = (t[:, hs].cpu() for t in (q, k, v))
    ref, ref_lse = oa.dense_attention(qc, kc, vc, used, return_lse=True, rows=rows)
    got = out[rows.cuda()][:, hs].cpu()
    got_lse = lse[rows.cuda()][:, hs].cpu()
    torch.testing.assert_close(got.float(), ref.float(), rtol=2e-2, atol=2e-2)
    _close(got, ref)
    torch.testing.assert_close(got_lse, ref_lse, rtol=1e-3, atol=1e-3)


def test_config3_layer_at_full_size():
    """BASELINE C3: 37x52x30, 48 heads, per-head seeded (1,8,16) / (4,4,8),
    keep 0.2, the whole SparseStudent layer."""
    spans, used, seq_len, _ = helpers.CONFIGS['C3a']
    grid = spans[0][1]
    shapes = [pt.TileShape(1, 8, 16), pt.TileShape(4, 4, 8)]
    choice = torch.randint(0, 2, (H,), generator=torch.Generator().manual_seed(3)).tolist()
    assert len(set(choice)) == 2
    layout = pa.PackedLayout((pa.VideoSpan(0, grid),), used, seq_len)
    clip = pa.ClipTiling(layout, pa.VedaConfig(target_budget=pm.Budget(ratio=0.2)), 'cuda')
    plan = pplan.TilePlan('c3', grid, shapes, [choice])
    pred = pp.TileScorePredictor([pp.LayerPredictor.random(
        H, 128, std=0.02, generator=torch.Generator().manual_seed(5), device='cuda')])
    student = pa.SparseStudent(clip, plan, pred)
    q, k, v = _qkv_cuda(seq_len, seed=13, used=used)
    print(f'C3 layer: {seq_len} rows, {H} heads, choice {sum(choice)} x (4,4,8)', flush=True)
    out = student(q, k, v, 0)
    torch.cuda.synchronize()
    assert (out[used:] == 0).all()
    parts = student.last['parts']
    assert len(parts) == 2
    for part in parts:
        heads = part['heads'].cpu()
        shape = shapes[choice[int(heads[0])]]
        assert all(shapes[choice[h]] == shape for h in heads.tolist())
        olay = helpers.oracle_layout(spans, used, seq_len, str(shape))
        logits = part['logits'].cpu()
        idx, keep = om.select_video_blocks(logits[:, :olay.n_video_tiles], olay,
                                           om.column_blocks(olay, om.Budget(ratio=0.2)))
        assert torch.equal(part['selection'].index.cpu(), idx)
        assert torch.equal(part['selection'].keep.cpu(), keep)
        mask = om.dense_block_mask(idx, keep, olay)
        for a, b in zip(part['lists'], om.index_lists(mask, olay)):
            assert torch.equal(a.cpu(), b)
        # 40,680 kept blocks per head at keep 0.2 for both shapes (equal cost)
        assert int((mask & olay.kv_ok[None, None, :]).sum()) == 40680 * heads.numel()
        # every query tile of the group's first head; the first, a padded
        # (partial) and the last tile of its last head
        partial = int(olay.partial_tiles[len(olay.partial_tiles) // 2])
        for hs, tiles in ((heads[[0]], torch.arange(olay.n_tiles)),
                          (heads[[-1]], torch.tensor([0, partial, olay.n_tiles - 1]))):
            rows = _tile_rows(tiles)
            print(f'C3 group {shape}: head {int(hs[0])}, {tiles.numel()} query tiles against the '
                  'oracle', flush=True)
            qt = ot.gather_tiles(q[:, hs.cuda()].cpu(), olay, None)[rows]
            kt = ot.gather_tiles(k[:, hs.cuda()].cpu(), olay, None)
            vt = ot.gather_tiles(v[:, hs.cuda()].cpu(), olay, None)
            hpos = [heads.tolist().index(h) for h in hs.tolist()]
            ref = oa.block_sparse_attention(qt, kt, vt, mask[hpos][:, tiles], olay.valid_count)
            real = olay.slot_valid[rows].bool()
            seq_rows = olay.perm[rows][real]
            got = out[seq_rows.cuda()][:, hs.cuda()].cpu()
            _close(got, ref[real])


def test_config5_oracle_chain_at_full_size():
    """BASELINE C5: 2,048 global rows then 102x30x52 video, (1,8,16), 48
    heads, keep 0.05, through OracleStudent (fused teacher pass)."""
    spans, used, seq_len, shape = helpers.CONFIGS['C5']
    grid = spans[0][1]
    layout = pa.PackedLayout((pa.VideoSpan(spans[0][0], grid),), used, seq_len)
    clip = pa.ClipTiling(layout, pa.VedaConfig(target_budget=pm.Budget(ratio=0.05)), 'cuda')
    plan = pplan.TilePlan.uniform('c5', grid, pt.TileShape.parse(shape), 1, H)
    student = pa.OracleStudent(clip, plan, target='mass')
    q, k, v = _qkv_cuda(seq_len, seed=17, used=used)
    print(f'C5 chain: {seq_len} rows, {H} heads', flush=True)
    out = student(q, k, v, 0)
    torch.cuda.synchronize()
    assert (out[used:] == 0).all()
    (part,) = student.last['parts']
    olay = helpers.oracle_layout(spans, used, seq_len, shape)
    n_video = olay.n_video_tiles
    assert olay.n_tiles - n_video == 16
    heat = part['heat'].cpu()
    assert heat.shape == (H, n_video, olay.n_tiles)
    # selection bit-exact for every head on the kernel's heat
    rows_all = torch.arange(n_video)
    idx, keep = om.select_video_blocks(heat[:, :, :n_video], olay,
                                       om.column_blocks(olay, om.Budget(ratio=0.05)), rows_all)
    assert torch.equal(part['selection'].index.cpu(), idx)
    assert torch.equal(part['selection'].keep.cpu(), keep)
    mask = om.dense_block_mask(idx, keep, olay)
    assert int(mask[:, :n_video, :n_video].sum()) == 77376 * H
    # the oracle on two heads: dense LSE of the sampled rows, their heat, and
    # the output of sampled query tiles (the last one global: every key tile)
    hs = SAMPLE_HEADS
    qc, kc, vc = (t[:, hs].cpu() for t in (q, k, v))
    tiles = torch.tensor([0, 700, n_video - 1, olay.n_tiles - 1])
    rows = _tile_rows(tiles)
    real = olay.slot_valid[rows].bool()
    seq_rows = olay.perm[rows][real]
    _, ref_lse = oa.dense_attention(qc, kc, vc, used, return_lse=True, rows=seq_rows)
    got_lse = part['lse_tiles'].cpu()                       # [H, n_video * 128]
    vid = tiles < n_video
    vrows = _tile_rows(tiles[vid])
    vreal = olay.slot_valid[vrows].bool()
    torch.testing.assert_close(got_lse[hs][:, vrows[vreal]].T, ref_lse[:int(vreal.sum())],
                               rtol=1e-3, atol=1e-3)
    lse_full = torch.zeros(seq_len, len(hs))
    lse_full[seq_rows] = ref_lse
    qt, kt, vt = (ot.gather_tiles(t, olay, None) for t in (qc, kc, vc))
    ref_heat = oa.teacher_heat(qt, kt, ot.gather_lse(lse_full, olay, torch.arange(len(hs))),
                               olay, tiles[vid], 'sum')
    torch.testing.assert_close(heat[hs][:, tiles[vid]], ref_heat, rtol=2e-3, atol=1e-6)
    ref = oa.block_sparse_attention(qt[rows], kt, vt, mask[hs][:, tiles], olay.valid_count)
    got = out[seq_rows.cuda()][:, hs].cpu()
    _close(got, ref[real])
