"""GPU parity of the block-sparse and dense attention forwards against the
fp32 masked-dense oracle. Bar: on real rows, output
max-abs <= 2e-2 and rel-L2 <= 1e-2 (bf16 I/O); LSE to the same max-abs."""

import pytest
import torch

from miowtion_amd import kernels
from miowtion_amd import mask as pm
from oracle import attention as oa
from oracle import mask as om
from oracle import tiling as ot
from tests import helpers

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
REL_L2 = 1e-2


def _close(got, want, rows=None):
    got, want = got.float().cpu(), want.float().cpu()
    if rows is not None:
        got, want = got[rows], want[rows]
    fin = torch.isfinite(want)
    assert torch.equal(torch.isfinite(got), fin)
    assert torch.equal(got[~fin], want[~fin])
    err = (got[fin] - want[fin]).abs().max().item() if fin.any() else 0.0
    rel = ((got[fin] - want[fin]).norm() / want[fin].norm().clamp(min=1e-30)).item()
    assert err <= MAX_ABS, f'max-abs {err}'
    assert rel <= REL_L2, f'rel-L2 {rel}'
    return err, rel


def _case(spec, heads=4, ratio=0.3, seed=0):
    lay = helpers.product_layout(*spec, device='cuda')
    olay = helpers.oracle_layout(*spec)
    q, k, v = helpers.qkv(lay.seq_len, heads, 128, seed=seed)
    qt, kt, vt = (ot.gather_tiles(t, olay, None) for t in (q, k, v))
    scores = torch.randn(heads, lay.n_tiles, lay.n_tiles, generator=torch.Generator().manual_seed(seed + 1))
    idx, keep = om.select_video_blocks(scores[:, :lay.n_video_tiles], olay,
                                       om.column_blocks(olay, om.Budget(ratio=ratio)))
    mask = om.dense_block_mask(idx, keep, olay)
    return lay, olay, qt, kt, vt, mask


def test_sparse_matches_oracle_with_partial_tiles():
    # reference tests/gpu/test_kernels_gpu.py:95-112
    lay, olay, qt, kt, vt, mask = _case(helpers.small_layout())
    assert olay.partial_tiles.numel() > 0
    out, lse = kernels.block_sparse_attention(qt.cuda(), kt.cuda(), vt.cuda(), mask.cuda(), lay,
                                              return_lse=True)
    ref, ref_lse = oa.block_sparse_attention(qt, kt, vt, mask, olay.valid_count, return_lse=True)
    real = olay.slot_valid.bool()
    _close(out, ref, real)
    _close(lse.T, ref_lse.T, real)


def test_non_finite_values_stay_in_the_query_tiles_that_keep_them():
    """An Inf in V reaches only the query tiles that keep its key tile, as in
    the reference (whose rows there become Inf, or NaN where p underflows to
    0, through P.V). The kernel does not reload a step's key rows past a
    sub-block's valid count, so those slot rows hold V rows of tiles that
    the same query tile kept in earlier steps; multiplied by p = 0 they can
    only turn an element the reference makes Inf into NaN, never make a
    finite element non-finite. Checked with Inf in ragged tiles (16 and 32
    valid keys, whose halves share steps) and in a full tile: the finite
    mask equals the oracle's element for element, and the finite elements
    meet the usual bar."""
    spec = helpers.small_layout(grid=(5, 12, 20), shape='2x8x8')
    lay, olay, qt, kt, vt, mask = _case(spec, heads=2, ratio=0.5, seed=7)
    vc = olay.valid_count
    ragged = [int(t) for t in torch.nonzero((vc > 0) & (vc <= 32)).flatten()[:2]]
    full = int(torch.nonzero(vc == 128).flatten()[0])
    vinf = vt.clone()
    expect = torch.ones(qt.shape, dtype=torch.bool)           # finite elements
    for t, d in zip(ragged + [full], (3, 70, 127)):
        vinf[t * 128 + int(vc[t]) - 1, 0, d] = float('inf')
        # rows of every query tile that keeps tile t, head 0, column d
        expect.view(-1, 128, 2, 128)[mask[0, :, t], :, 0, d] = False
    out = kernels.block_sparse_attention(qt.cuda(), kt.cuda(), vinf.cuda(), mask.cuda(), lay).cpu()
    # the oracle's masked-dense product multiplies every masked key too (0 x
    # Inf would poison every row), so its values come from the finite V: a
    # value row changes nothing but its own column of the rows that keep it
    ref = oa.block_sparse_attention(qt, kt, vt, mask, olay.valid_count)
    real = olay.slot_valid.bool()
    got, fin, want = out.float()[real], expect[real], ref.float()[real]
    assert (~fin).any() and fin.any()
    assert torch.equal(torch.isfinite(got), fin)
    assert (got[fin] - want[fin]).abs().max().item() <= MAX_ABS


def test_keep_all_sparse_equals_dense_kernel_and_oracle():
    # reference tests/gpu/test_kernels_gpu.py:115-138
    spec = helpers.small_layout()
    lay, olay, qt, kt, vt, _ = _case(spec)
    mask = torch.ones(4, lay.n_tiles, lay.n_tiles, dtype=torch.bool)
    out = kernels.block_sparse_attention(qt.cuda(), kt.cuda(), vt.cuda(), mask.cuda(), lay)
    ref = oa.block_sparse_attention(qt, kt, vt, mask, olay.valid_count)
    real = olay.slot_valid.bool()
    _close(out, ref, real)


def test_empty_query_tiles_give_zero_and_neg_inf_lse():
    lay, olay, qt, kt, vt, mask = _case(helpers.small_layout(), ratio=0.5)
    mask[1, 3] = False
    mask[0, :, :] = False
    out, lse = kernels.block_sparse_attention(qt.cuda(), kt.cuda(), vt.cuda(), mask.cuda(), lay,
                                              return_lse=True)
    out, lse = out.cpu(), lse.cpu()
    assert (out[:, 0] == 0).all() and torch.isinf(lse[0]).all() and (lse[0] < 0).all()
    assert (out[3 * 128:4 * 128, 1] == 0).all() and (lse[1, 3 * 128:4 * 128] == float('-inf')).all()
    ref, ref_lse = oa.block_sparse_attention(qt, kt, vt, mask, olay.valid_count, return_lse=True)
    real = olay.slot_valid.bool()
    _close(out, ref, real)
    _close(lse.T, ref_lse.T, real)


def test_all_zero_query_groups_match_the_oracle_on_every_row():
    """Query rows in 32-row groups that are all zero take the kernel's
    product-free step (padding rows of partial tiles, and here also a whole
    group of real rows zeroed): every row, padding included, against the
    oracle (the uniform average of the valid kept keys, LSE = log of their
    count), with an empty row and a tile whose groups are mixed."""
    lay, olay, qt, kt, vt, mask = _case(helpers.small_layout(), seed=7)
    assert olay.partial_tiles.numel() > 0
    qt = qt.clone()
    qt[2 * 128 + 32:2 * 128 + 64] = 0           # one whole group of real rows
    qt[3 * 128 + 40:3 * 128 + 64] = 0           # part of a group: stays on the full step
    mask[0, 5] = False                          # a query tile with no key at all
    out, lse = kernels.block_sparse_attention(qt.cuda(), kt.cuda(), vt.cuda(), mask.cuda(), lay,
                                              return_lse=True)
    ref, ref_lse = oa.block_sparse_attention(qt, kt, vt, mask, olay.valid_count, return_lse=True)
    _close(out, ref)
    _close(lse.T, ref_lse.T)


def test_narrow_walk_tiles_match_the_oracle_on_every_row():
    """Query tiles whose only non-zero rows are their first 32 take the
    narrow walk (one 32-key sub-block of every step per wave, the halves
    merged at the end). Made here by zeroing rows 32..127 of several tiles:
    one with all 32 first rows real, one with 24, one that keeps a single
    ragged key tile (its step's second sub-block has no valid key), one that
    keeps a single full key tile and one that keeps nothing. Every row
    (padding included) and the LSE against the oracle, in tile order and
    through the sequence-order entry with k and v in sequence order."""
    spec = helpers.small_layout(grid=(5, 12, 20), shape='2x8x8')
    lay, olay, qt, kt, vt, mask = _case(spec, heads=2, ratio=0.4, seed=11)
    vc = olay.valid_count
    ragged = int(torch.nonzero((vc > 0) & (vc <= 32)).flatten()[0])
    full = int(torch.nonzero(vc == 128).flatten()[0])
    tiles = [int(t) for t in torch.nonzero(vc == 128).flatten()[:5]]
    qt = qt.clone()
    for t in tiles:
        qt[t * 128 + 32:(t + 1) * 128] = 0
    qt[tiles[1] * 128 + 24:tiles[1] * 128 + 32] = 0
    mask[:, tiles[2]] = False
    mask[:, tiles[2], ragged] = True
    mask[:, tiles[3]] = False
    mask[:, tiles[3], full] = True
    mask[1, tiles[4]] = False
    out, lse = kernels.block_sparse_attention(qt.cuda(), kt.cuda(), vt.cuda(), mask.cuda(), lay,
                                              return_lse=True)
    ref, ref_lse = oa.block_sparse_attention(qt, kt, vt, mask, olay.valid_count, return_lse=True)
    _close(out, ref)
    _close(lse.T, ref_lse.T)
    rows = torch.cat([torch.arange(t * 128, (t + 1) * 128) for t in tiles])
    _close(out, ref, rows)
    # the sequence-order entry (q, k, v in sequence order, output scattered)
    perm = olay.perm
    ok = perm >= 0
    qs, ks, vs = (torch.zeros(lay.seq_len, 2, 128, dtype=torch.bfloat16) for _ in range(3))
    qs[perm[ok]], ks[perm[ok]], vs[perm[ok]] = qt[ok], kt[ok], vt[ok]
    lists = kernels.index_lists(mask.cuda(), lay)
    got = torch.zeros(lay.seq_len + 1, 2, 128, dtype=torch.bfloat16, device='cuda')
    kernels.block_sparse_attention_seq_kv_(got, qs.cuda(), ks.cuda(), vs.cuda(), lists, lay, None)
    want = torch.zeros(lay.seq_len, 2, 128, dtype=torch.bfloat16)
    want[perm[ok]] = out.cpu()[ok]
    assert torch.equal(got[:-1].cpu().view(torch.int16), want.view(torch.int16))


def test_query_tile_subset_rows():
    """q holds only some query tiles; mask rows follow q (fa4.py:308-313)."""
    lay, olay, qt, kt, vt, mask = _case(helpers.small_layout(), seed=3)
    rows = torch.tensor([1, 4, 5])
    qs = qt.view(-1, 128, 4, 128)[rows].reshape(-1, 4, 128)
    ms = mask[:, rows]
    out = kernels.block_sparse_attention(qs.cuda(), kt.cuda(), vt.cuda(), ms.cuda(), lay)
    ref = oa.block_sparse_attention(qs, kt, vt, ms, olay.valid_count)
    real = olay.slot_valid.view(-1, 128)[rows].reshape(-1).bool()
    _close(out, ref, real)


def test_config1_end_to_end_blocks_and_attention():
    """8 heads, grid 4x16x16 -> 8 tiles (2,8,8), uniform
    random tile scores, top 50% per query tile with the diagonal."""
    spec = helpers.CONFIGS['C1']
    lay = helpers.product_layout(*spec, device='cuda')
    olay = helpers.oracle_layout(*spec)
    q, k, v = helpers.qkv(1024, 8, 128, seed=0)
    scores = torch.rand(8, 8, 8, generator=torch.Generator().manual_seed(1))
    sel = pm.select_video_blocks(scores.cuda(), lay, pm.column_blocks(lay, pm.Budget(ratio=0.5)))
    idx, keep = om.select_video_blocks(scores, olay, om.column_blocks(olay, om.Budget(ratio=0.5)))
    assert torch.equal(sel.index.cpu(), idx) and torch.equal(sel.keep.cpu(), keep)
    mask = pm.dense_block_mask(sel, lay)
    assert (mask.sum(-1) == 4).all()
    qt, kt, vt = (kernels.gather_tiles(t.cuda(), lay, None) for t in (q, k, v))
    out, lse = kernels.block_sparse_attention(qt, kt, vt, mask, lay, return_lse=True)
    oq, ok, ov = (ot.gather_tiles(t, olay, None) for t in (q, k, v))
    ref, ref_lse = oa.block_sparse_attention(oq, ok, ov, mask.cpu(), olay.valid_count, return_lse=True)
    _close(out, ref)
    _close(lse, ref_lse)


@pytest.mark.parametrize('seq_len,used', [(2048, 2000), (1000, 1000), (64 * 21, 64 * 21 - 7)])
def test_dense_matches_oracle(seq_len, used):
    # reference tests/gpu/test_kernels_gpu.py:32-41
    q, k, v = helpers.qkv(seq_len, 4, 128)
    out, lse = kernels.dense_attention(q.cuda(), k.cuda(), v.cuda(), used, return_lse=True)
    ref, ref_lse = oa.dense_attention(q, k, v, used, return_lse=True)
    _close(out, ref)
    _close(lse, ref_lse)
    assert (out[used:] == 0).all() and (lse[used:] == 0).all()


def test_whole_heads_at_config2_size():
    """C2 geometry (592 tiles, 48 heads) at 90% sparsity: every query tile of
    two heads (the first and the last) of the full-size kernel call against
    the oracle. The step walk (full-list halves, split halves, ragged halves
    paired two to a step) differs from tile to tile, so whole heads cover
    every form it takes on this workload."""
    spec = helpers.CONFIGS['C2']
    lay = helpers.product_layout(*spec, device='cuda')
    olay = helpers.oracle_layout(*spec)
    H = 48
    g = torch.Generator(device='cuda').manual_seed(0)
    q, k, v = (torch.randn(lay.seq_len, H, 128, generator=g, device='cuda').to(torch.bfloat16)
               for _ in range(3))
    qt, kt, vt = (kernels.gather_tiles(t, lay, None) for t in (q, k, v))
    scores = torch.rand(H, lay.n_tiles, lay.n_tiles, generator=g, device='cuda')
    sel = pm.select_video_blocks(scores, lay, pm.column_blocks(lay, pm.Budget(ratio=0.1)))
    mask = pm.dense_block_mask(sel, lay)
    out, lse = kernels.block_sparse_attention(qt, kt, vt, mask, lay, return_lse=True)
    assert torch.isfinite(out.float()).all()
    heads = [0, 47]
    print(f'C2 whole heads {heads}: {lay.n_tiles} query tiles each against the oracle', flush=True)
    ref, ref_lse = oa.block_sparse_attention(qt[:, heads].cpu(), kt[:, heads].cpu(),
                                             vt[:, heads].cpu(), mask[heads].cpu(),
                                             olay.valid_count, return_lse=True)
    real = olay.slot_valid.bool()
    _close(out[:, heads], ref, real)
    _close(lse[heads].T, ref_lse.T, real)


def test_front_tiles_change_the_order_only():
    """Dispatching the global query tiles (dense rows, last in tile order)
    first gives the same bits as the plain order, forward and backward."""
    from miowtion_amd import ops
    lay, olay, qt, kt, vt, mask = _case(helpers.small_layout())
    front = lay.n_tiles - lay.n_video_tiles
    assert front > 0
    q, k, v, m = qt.cuda(), kt.cuda(), vt.cuda(), mask.cuda()
    lists = kernels.index_lists(m, lay)
    a = ops.block_sparse_fwd(q, k, v, *lists, lay.valid_count, True, 0)
    b = ops.block_sparse_fwd(q, k, v, *lists, lay.valid_count, True, front)
    assert all(torch.equal(x, y) for x, y in zip(a, b))
    lists_t = kernels.index_lists(m, lay, transpose=True)
    dout = torch.randn(q.shape, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16).cuda()
    ga = ops.block_sparse_bwd(q, k, v, a[0], dout, a[1], None, *lists, *lists_t, lay.valid_count, 0)
    gb = ops.block_sparse_bwd(q, k, v, a[0], dout, a[1], None, *lists, *lists_t, lay.valid_count,
                              front)
    assert all(torch.equal(x, y) for x, y in zip(ga, gb))


def test_irregular_lists_keep_list_order():
    """The walk visits a row's kept tiles in ascending key order from a
    rotation point. Lists that are not strictly ascending or hold an entry
    outside [0, n_k) keep list order (the full list, then the partial list)
    and give the oracle's result as well; an entry outside [0, n_k) is a void
    step and changes no bit of the list-order result."""
    from miowtion_amd import ops
    lay, olay, qt, kt, vt, mask = _case(helpers.small_layout())
    assert olay.partial_tiles.numel() > 0 and olay.partial_tiles.numel() < lay.n_tiles
    q, k, v, m = qt.cuda(), kt.cuda(), vt.cuda(), mask.cuda()
    pc, pi, fc, fi = kernels.index_lists(m, lay)

    def reversed_members(cnt, idx):
        t = torch.arange(idx.shape[-1], device=idx.device)
        c = cnt[..., None].long()
        return idx.gather(-1, torch.where(t < c, c - 1 - t, t)).contiguous()

    def with_bad_entry(cnt, idx):
        # one more entry, past n_k, at position cnt (a row's full list holds
        # at most the full tiles and its partial list the partial ones, so
        # every row has room when both kinds exist)
        assert (cnt < idx.shape[-1]).all()
        idx = idx.clone()
        idx.scatter_(-1, cnt.long()[..., None],
                     torch.full_like(idx[..., :1], lay.n_tiles + 7))
        return cnt + 1, idx

    pir, fir = reversed_members(pc, pi), reversed_members(fc, fi)
    assert not torch.equal(pir, pi) and not torch.equal(fir, fi)
    ref, ref_lse = oa.block_sparse_attention(qt, kt, vt, mask, olay.valid_count, return_lse=True)
    real = olay.slot_valid.bool()
    # every row in list order: members reversed, and a void full-list entry
    fc2, fi2 = with_bad_entry(fc, fir)
    a = ops.block_sparse_fwd(q, k, v, pc, pir, fc2, fi2, lay.valid_count, True, 0)
    _close(a[0], ref, real)
    _close(a[1].T, ref_lse.T, real)
    # a void partial-list entry too: the same bits
    pc2, pi2 = with_bad_entry(pc, pir)
    b = ops.block_sparse_fwd(q, k, v, pc2, pi2, fc2, fi2, lay.valid_count, True, 0)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    # ascending members with the void entries: list order with the same
    # members, so the oracle's result again
    c = ops.block_sparse_fwd(q, k, v, *with_bad_entry(pc, pi), *with_bad_entry(fc, fi),
                             lay.valid_count, True, 0)
    _close(c[0], ref, real)
    _close(c[1].T, ref_lse.T, real)


def test_largest_tile_count():
    """2048 tiles a side (FA4's cap on blocks per side, fa4_sm8x/block_sparsity.py:58-79;
    the kernels' list and step tables are sized to it), partial tiles
    included: sampled query tiles of the forward against the oracle; a
    2049th tile is refused."""
    spec = ([(0, (32, 62, 120))], 32 * 62 * 120, 32 * 62 * 120, '1x8x16')
    lay = helpers.product_layout(*spec, device='cuda')
    olay = helpers.oracle_layout(*spec)
    assert lay.n_tiles == 2048 and int((olay.valid_count < 128).sum()) > 0
    q, k, v = helpers.qkv(lay.seq_len, 1, 128, seed=3)
    qt, kt, vt = (ot.gather_tiles(t, olay, None) for t in (q, k, v))
    g = torch.Generator().manual_seed(4)
    mask = torch.rand(1, 2048, 2048, generator=g) < 0.05
    mask |= torch.eye(2048, dtype=torch.bool)[None]
    mask[0, 7] = olay.kv_ok          # one dense row: the longest list (2048 tiles)
    out, lse = kernels.block_sparse_attention(qt.cuda(), kt.cuda(), vt.cuda(), mask.cuda(), lay,
                                              return_lse=True)
    tiles = torch.tensor([0, 7, 1023, 2047])
    rows = (tiles[:, None] * 128 + torch.arange(128)[None, :]).reshape(-1)
    ref, ref_lse = oa.block_sparse_attention(qt[rows], kt, vt, mask[:, tiles], olay.valid_count,
                                             return_lse=True)
    real = olay.slot_valid.bool()[rows]
    _close(out.cpu()[rows], ref, real)
    _close(lse.cpu()[:, rows].T, ref_lse.T, real)
    # a 2049th key tile is refused before anything is launched
    from miowtion_amd import ops
    kv = torch.zeros(2049 * 128, 1, 128, dtype=torch.bfloat16, device='cuda')
    cnt = torch.zeros(1, 1, 1, dtype=torch.int32, device='cuda')
    idx = torch.zeros(1, 1, 1, 2049, dtype=torch.int32, device='cuda')
    with pytest.raises(ValueError, match='n_k_tiles'):
        ops.block_sparse_fwd(qt[:128].cuda(), kv, kv, cnt, idx, cnt, idx,
                             torch.full((2049,), 128, dtype=torch.int32, device='cuda'), False)


@pytest.mark.parametrize('name', ['small', 'C3b'])
def test_sequence_order_entry_equals_gather_attend_scatter(name):
    """veda_block_sparse_fwd_seq (q read through the gather index, rows
    written through the scatter index) against gather -> sparse forward ->
    scatter on the same inputs: bit-identical buffers, padding rows and the
    heads outside the subset untouched. The subset is heads 1 and 3 of 4."""
    spec = helpers.small_layout() if name == 'small' else helpers.CONFIGS[name]
    lay = helpers.product_layout(*spec, device='cuda')
    q, k, v = (t.cuda() for t in helpers.qkv(lay.seq_len, 4, 128, seed=5))
    heads = torch.tensor([1, 3], device='cuda')
    kt, vt = (kernels.gather_tiles(t, lay, heads) for t in (k, v))
    g = torch.Generator().manual_seed(6)
    mask = (torch.rand(2, lay.n_tiles, lay.n_tiles, generator=g) < 0.2) | torch.eye(
        lay.n_tiles, dtype=torch.bool)[None]
    lists = kernels.index_lists(mask.cuda(), lay)
    init = torch.randn(lay.seq_len + 1, 4, 128, generator=g).to(torch.bfloat16).cuda()
    want = init.clone()
    o_tiles = kernels.block_sparse_attention_lists(kernels.gather_tiles(q, lay, heads), kt, vt,
                                                   lists, lay)
    kernels.scatter_tiles_(want, o_tiles, lay, heads)
    got = init.clone()
    kernels.block_sparse_attention_seq_(got, q, kt, vt, lists, lay, heads)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want.cpu())
    assert torch.equal(got[:, [0, 2]].cpu(), init[:, [0, 2]].cpu())


@pytest.mark.parametrize('name', ['small', 'C3b', 'C2'])
def test_sequence_order_kv_entry_equals_gather_attend_scatter(name):
    """veda_block_sparse_fwd_seq_kv (q, k and v read through the gather
    index, rows written through the scatter index) against gather of q, k,
    v -> sparse forward -> scatter on the same inputs: bit-identical buffers
    (finite inputs), padding rows and the heads outside the subset untouched.
    The subset is heads 1 and 3 of 4; the masks keep 20 % of the blocks plus
    the diagonal, so steps pair ragged halves of partial key tiles."""
    spec = helpers.small_layout() if name == 'small' else helpers.CONFIGS[name]
    lay = helpers.product_layout(*spec, device='cuda')
    q, k, v = (t.cuda() for t in helpers.qkv(lay.seq_len, 4, 128, seed=7))
    heads = torch.tensor([1, 3], device='cuda')
    kt, vt = (kernels.gather_tiles(t, lay, heads) for t in (k, v))
    g = torch.Generator().manual_seed(8)
    mask = (torch.rand(2, lay.n_tiles, lay.n_tiles, generator=g) < 0.2) | torch.eye(
        lay.n_tiles, dtype=torch.bool)[None]
    lists = kernels.index_lists(mask.cuda(), lay)
    init = torch.randn(lay.seq_len + 1, 4, 128, generator=g).to(torch.bfloat16).cuda()
    want = init.clone()
    kernels.block_sparse_attention_seq_(want, q, kt, vt, lists, lay, heads)
    got = init.clone()
    kernels.block_sparse_attention_seq_kv_(got, q, k, v, lists, lay, heads)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16).cpu(), want.view(torch.int16).cpu())
    assert torch.equal(got[:, [0, 2]].cpu(), init[:, [0, 2]].cpu())
    # k and v must be laid out as q
    with pytest.raises(ValueError, match='laid out as q'):
        kernels.block_sparse_attention_seq_kv_(got, q, k[:-1], v, lists, lay, heads)


def test_sequence_order_kv_irregular_lists_keep_list_order():
    """Lists whose members are reversed and that hold a void full-list entry
    take list order in every form of the walk: the sequence-order entry
    equals the tiled one bit for bit on them, and both stay within the
    oracle's bar of the result on the regular lists."""
    spec = helpers.small_layout()
    lay = helpers.product_layout(*spec, device='cuda')
    q, k, v = (t.cuda() for t in helpers.qkv(lay.seq_len, 4, 128, seed=7))
    heads = torch.tensor([1, 3], device='cuda')
    kt, vt = (kernels.gather_tiles(t, lay, heads) for t in (k, v))
    g = torch.Generator().manual_seed(8)
    mask = (torch.rand(2, lay.n_tiles, lay.n_tiles, generator=g) < 0.2) | torch.eye(
        lay.n_tiles, dtype=torch.bool)[None]
    pc, pi, fc, fi = kernels.index_lists(mask.cuda(), lay)
    t = torch.arange(fi.shape[-1], device='cuda')
    rev = lambda c, idx: idx.gather(-1, torch.where(t < c[..., None].long(),
                                                    c[..., None].long() - 1 - t, t)).contiguous()
    fir = rev(fc, fi).clone()
    assert (fc < fir.shape[-1]).all()
    fir.scatter_(-1, fc.long()[..., None], torch.full_like(fir[..., :1], lay.n_tiles + 7))
    odd = (pc, rev(pc, pi), fc + 1, fir)
    init = torch.zeros(lay.seq_len + 1, 4, 128, dtype=torch.bfloat16, device='cuda')
    want, got, regular = init.clone(), init.clone(), init.clone()
    kernels.block_sparse_attention_seq_(want, q, kt, vt, odd, lay, heads)
    kernels.block_sparse_attention_seq_kv_(got, q, k, v, odd, lay, heads)
    kernels.block_sparse_attention_seq_kv_(regular, q, k, v, (pc, pi, fc, fi), lay, heads)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16).cpu(), want.view(torch.int16).cpu())
    d = (got.float() - regular.float())[:lay.used, [1, 3]]
    assert d.abs().max().item() <= MAX_ABS
    assert (d.norm() / regular.float()[:lay.used, [1, 3]].norm()).item() <= REL_L2


def test_sequence_order_kv_non_finite_rows_stay_in_their_blocks():
    """With k / v read in sequence order a key tile's padding rows come from
    its first real row, so an Inf in that row's v reaches exactly the query
    tiles that keep the block (as in the tiled form, where the real row
    itself carries it); every other row matches the tiled form bit for bit."""
    spec = helpers.small_layout()
    lay = helpers.product_layout(*spec, device='cuda')
    q, k, v = (t.cuda() for t in helpers.qkv(lay.seq_len, 2, 128, seed=9))
    heads = torch.tensor([0, 1], device='cuda')
    vc = lay.valid_count.cpu()
    j = int(torch.nonzero((vc > 0) & (vc < 128))[0])   # a partial key tile
    first = int(lay.gather_index[j * 128])             # its first real row
    v[first, :, 5] = float('inf')
    g = torch.Generator().manual_seed(10)
    mask = (torch.rand(2, lay.n_tiles, lay.n_tiles, generator=g) < 0.3) | torch.eye(
        lay.n_tiles, dtype=torch.bool)[None]
    lists = kernels.index_lists(mask.cuda(), lay)
    kt, vt = (kernels.gather_tiles(t, lay, heads) for t in (k, v))
    want = torch.zeros(lay.seq_len + 1, 2, 128, dtype=torch.bfloat16, device='cuda')
    kernels.block_sparse_attention_seq_(want, q, kt, vt, lists, lay, heads)
    got = torch.zeros_like(want)
    kernels.block_sparse_attention_seq_kv_(got, q, k, v, lists, lay, heads)
    torch.cuda.synchronize()
    keeps = (mask & lay.kv_ok.cpu()[None, None, :])[:, :, j]      # [heads, query tiles]
    rows_keep = torch.zeros(lay.seq_len + 1, 2, dtype=torch.bool)
    sc = lay.scatter_index.cpu().view(-1, 128)
    for h in range(2):
        for r in torch.nonzero(keeps[h]).flatten().tolist():
            rows_keep[sc[r], h] = True
    gotc, wantc = got.cpu(), want.cpu()
    bad = ~torch.isfinite(gotc.float()).all(-1)
    assert not (bad & ~rows_keep).any()          # nothing outside the keeping tiles
    same = ~rows_keep
    assert torch.equal(gotc.view(torch.int16)[same], wantc.view(torch.int16)[same])
