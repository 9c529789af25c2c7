"""GPU parity of the tile gather / pool / scatter kernels against the oracle
(bit-exact rows, max, min; mean and second moments to the reference's own
tolerance, tests/gpu/test_kernels_gpu.py:176-197)."""

import pytest
import torch

from miowtion_amd import kernels
from oracle import predictor as op
from oracle import tiling as ot
from tests import helpers

pytestmark = pytest.mark.gpu


def _pair(spec):
    return helpers.product_layout(*spec, device='cuda'), helpers.oracle_layout(*spec)


@pytest.mark.parametrize('heads', [None, [0, 2, 3], [3, 1]])
@pytest.mark.parametrize('dim', [128, 64])
def test_gather_pool_scatter_match_oracle(heads, dim):
    lay, olay = _pair(helpers.small_layout())
    assert olay.partial_tiles.numel() > 0
    x, = helpers.qkv(lay.seq_len, 4, dim, n=1)
    idx = None if heads is None else torch.tensor(heads)
    tiles, feats = kernels.gather_and_pool(x.cuda(), lay, None if idx is None else idx.cuda())
    ref_tiles = ot.gather_tiles(x, olay, idx)
    assert torch.equal(tiles.cpu(), ref_tiles)
    assert torch.equal(kernels.gather_tiles(x.cuda(), lay, None if idx is None else idx.cuda()).cpu(),
                       ref_tiles)
    ref_feats = op.pool_tiles(ref_tiles, olay)
    got = feats.cpu()
    assert torch.equal(got[..., dim:], ref_feats[..., dim:])  # max, min: exact
    torch.testing.assert_close(got[..., :dim], ref_feats[..., :dim], rtol=1e-5, atol=1e-6)
    out = torch.zeros(lay.seq_len + 1, *x.shape[1:], dtype=x.dtype, device='cuda')
    kernels.scatter_tiles_(out, tiles, lay, None if idx is None else idx.cuda())
    out_ref = torch.zeros(lay.seq_len + 1, *x.shape[1:], dtype=x.dtype)
    ot.scatter_tiles_(out_ref, ref_tiles, olay, idx)
    assert torch.equal(out[:lay.seq_len].cpu(), out_ref[:lay.seq_len])


def test_second_moments_match_oracle():
    lay, olay = _pair(helpers.small_layout(grid=(5, 12, 20), shape='2x8x8'))
    x, = helpers.qkv(lay.seq_len, 3, 128, seed=4, n=1)
    x = x + 3.0  # an offset makes the centred form matter (predictor.py:138-143)
    x = x.to(torch.bfloat16)
    tiles, feats, sq, var = kernels.gather_and_pool(x.cuda(), lay, None, second=True)
    ref_tiles = ot.gather_tiles(x, olay, None)
    torch.testing.assert_close(sq.cpu(), op.pool_tiles(ref_tiles, olay, 'raw'), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(var.cpu(), op.pool_tiles(ref_tiles, olay, 'central'), rtol=1e-4, atol=1e-5)
    # pool-only mode over tile-ordered rows gives the same statistics
    assert torch.equal(kernels.pool_tiles(tiles, lay), feats)
    assert torch.equal(kernels.pool_tiles(tiles, lay, 'raw'), sq)
    assert torch.equal(kernels.pool_tiles(tiles, lay, 'central'), var)


@pytest.mark.parametrize('second', [False, True])
def test_pooling_propagates_nan_like_torch(second):
    """torch's amax / amin return NaN when a reduced row holds NaN, of either
    sign (the reference pools with them, predictor.py:82-130). Both pooling
    forms (the packed int16 order keys of first-order pooling, and the
    4-wave form with second moments) must do the same: tiles with +NaN only,
    -NaN only, both, and +inf beside -inf (max / min stay finite-signed,
    the mean is NaN)."""
    lay, olay = _pair(helpers.small_layout())
    x, = helpers.qkv(lay.seq_len, 2, 128, seed=6, n=1)
    bits = x.view(torch.int16)     # bf16 +NaN 0x7fc0, -NaN 0xffc0 set as bits
    perm = olay.perm.view(olay.n_tiles, 128)
    rows = [perm[t, :olay.valid_count[t]] for t in range(4)]
    bits[rows[0][3], 0, 5] = 0x7fc0
    bits[rows[1][0], 1, 7] = -64
    bits[rows[2][1], 0, 9] = 0x7fc0
    bits[rows[2][2], 0, 9] = -64
    x[rows[3][4], 1, 11] = float('inf')
    x[rows[3][5], 1, 11] = float('-inf')
    assert torch.signbit(x[rows[1][0], 1, 7].float())
    res = kernels.gather_and_pool(x.cuda(), lay, None, second=second)
    tiles, feats = res[0], res[1]
    ref_tiles = ot.gather_tiles(x, olay, None)
    assert torch.equal(tiles.cpu().view(torch.int16), ref_tiles.view(torch.int16))
    want = op.pool_tiles(ref_tiles, olay)
    got = feats.cpu()
    assert torch.isnan(want[0, 0, [5, 128 + 5, 256 + 5]]).all()
    torch.testing.assert_close(got[..., 128:], want[..., 128:], rtol=0, atol=0, equal_nan=True)
    torch.testing.assert_close(got[..., :128], want[..., :128], rtol=1e-5, atol=1e-6, equal_nan=True)
    assert torch.equal(torch.isnan(got), torch.isnan(want))
    assert torch.equal(kernels.pool_tiles(tiles, lay).isnan(), got.isnan().cuda())


def test_empty_tile_pools_to_zero():
    lay, olay = _pair(helpers.small_layout())
    lay.valid_count[0] = 0
    lay.slot_valid[:128] = 0
    lay.kv_ok[0] = False
    olay.valid_count[0] = 0
    olay.kv_ok[0] = False
    x, = helpers.qkv(lay.seq_len, 2, 128, n=1)
    _, feats, sq, var = kernels.gather_and_pool(x.cuda(), lay, None, second=True)
    for t in (feats, sq, var):
        assert torch.isfinite(t).all() and (t[:, 0] == 0).all()


def test_gather_lse_matches_oracle():
    lay, olay = _pair(helpers.small_layout())
    lse = torch.randn(lay.seq_len, 4, generator=torch.Generator().manual_seed(1))
    heads = torch.tensor([2, 0])
    got = kernels.gather_lse(lse.cuda(), lay, heads.cuda()).cpu()
    assert torch.equal(got, ot.gather_lse(lse, olay, heads))


@pytest.mark.parametrize('name', ['C1', 'C3a', 'C3b', 'C5'])
def test_round_trip_bit_exact_at_full_size(name):
    """gather -> scatter is the identity on real rows (all heads), at the
    BASELINE geometry's full size; padding rows stay zero."""
    spans, used, seq_len, shape = helpers.CONFIGS[name]
    lay = helpers.product_layout(spans, used, seq_len, shape, device='cuda')
    heads = 8 if name == 'C1' else 48
    g = torch.Generator(device='cuda').manual_seed(7)
    x = torch.randn(seq_len, heads, 128, generator=g, device='cuda').to(torch.bfloat16)
    x[used:] = 0
    tiles = kernels.gather_tiles(x, lay, None)
    out = torch.zeros(seq_len + 1, heads, 128, dtype=torch.bfloat16, device='cuda')
    kernels.scatter_tiles_(out, tiles, lay, None)
    assert torch.equal(out[:seq_len], x)
    assert bool((tiles[lay.slot_valid == 0] == 0).all())
    # a permuted head subset round-trips into only those heads
    sub = torch.tensor([5, 1, 3], device='cuda')
    t2 = kernels.gather_tiles(x, lay, sub)
    out2 = torch.zeros_like(out)
    kernels.scatter_tiles_(out2, t2, lay, sub)
    assert torch.equal(out2[:seq_len, sub], x[:, sub])
    assert (out2[:seq_len, 0] == 0).all()


def test_supports_is_op_specific():
    """The routing predicate answers per kernel family: d64 only for the
    permutation kernels, d128 bf16 for all, on the gfx950 device."""
    from miowtion_amd import kernels
    assert kernels._device_arch(torch.device('cuda')) == 'gfx950'
    d128 = torch.zeros(256, 2, 128, dtype=torch.bfloat16, device='cuda')
    d64 = torch.zeros(256, 2, 64, dtype=torch.bfloat16, device='cuda')
    for op in ('gather', 'attention', 'heat'):
        assert kernels.supports(d128, op)
        assert not kernels.supports(d128.half(), op)
        assert not kernels.supports(d128.transpose(0, 2), op)
    assert kernels.supports(d64, 'gather')
    assert not kernels.supports(d64, 'attention') and not kernels.supports(d64, 'heat')
