"""The oracle's zero-order compensation (miowtion/veda/attention.py:591-689),
pinned by what the mathematics fixes rather than by retyping the formula:

  * exactness: when every real row of each dropped key tile carries the same
    key, the tile's centroid is that key, so the zero-order term is exact
    and compensated sparse attention equals dense attention over all keys;
  * identity: with nothing dropped the output is o_kept;
  * reference invariance: an independent float64 form that sums every kept
    key and every virtual key against an arbitrary reference L (the
    docstring's "the exponential reference cancels") gives the same output;
  * a row that kept nothing uses reference 0 and o_kept 0.
"""

import math

import torch

from oracle import attention as oa
from oracle import tiling as ot
from tests import helpers


def _case(seed=0, heads=2):
    spec = helpers.small_layout(grid=(4, 12, 12), shape='2x8x8', text=40, extra=16)
    lay = helpers.oracle_layout(*spec)
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(lay.seq_len, heads, 128, generator=g) for _ in range(3))
    hs = torch.arange(heads)
    qt, kt, vt = (ot.gather_tiles(t, lay, hs) for t in (q, k, v))
    n = lay.n_tiles
    mask = torch.rand(heads, n, n, generator=g) < 0.4
    mask |= torch.eye(n, dtype=torch.bool)[None]
    return lay, qt, kt, vt, mask


def test_exact_when_dropped_tiles_hold_one_key():
    lay, qt, kt, vt, mask = _case()
    n = lay.n_tiles
    # every real row of a tile gets the tile's first row's key
    k_same = kt.clone().view(n, 128, *kt.shape[1:])
    real = (torch.arange(128)[None, :] < lay.valid_count[:, None])
    k_same[:] = torch.where(real[:, :, None, None], k_same[:, :1], torch.zeros(()))
    k_same = k_same.view_as(kt)
    o, lse = oa.block_sparse_attention(qt, k_same, vt, mask, lay.valid_count, return_lse=True)
    comp = oa.zero_order_compensation(o, lse, qt, k_same, vt, mask, lay.valid_count)
    full = oa.block_sparse_attention(qt, k_same, vt, torch.ones_like(mask), lay.valid_count)
    torch.testing.assert_close(comp, full, rtol=2e-5, atol=2e-5)
    # and it is not the uncompensated output
    assert (comp - o).abs().max() > 1e-2


def test_nothing_dropped_is_identity():
    lay, qt, kt, vt, mask = _case(1)
    allm = torch.ones_like(mask)
    o, lse = oa.block_sparse_attention(qt, kt, vt, allm, lay.valid_count, return_lse=True)
    comp = oa.zero_order_compensation(o, lse, qt, kt, vt, allm, lay.valid_count)
    assert torch.equal(comp, o)


def test_matches_an_arbitrary_reference_float64_form():
    lay, qt, kt, vt, mask = _case(2)
    o, lse = oa.block_sparse_attention(qt, kt, vt, mask, lay.valid_count, return_lse=True)
    comp = oa.zero_order_compensation(o, lse, qt, kt, vt, mask, lay.valid_count)
    kc, vc = oa.tile_summaries(kt, vt, lay.valid_count, torch.float64)
    n, D = lay.n_tiles, 128
    real = (torch.arange(128)[None, :] < lay.valid_count[:, None]).reshape(-1)
    counts = lay.valid_count.double()
    for h in range(qt.shape[1]):
        for r in range(0, qt.shape[0], 37):
            qi = r // 128
            qv = qt[r, h].double()
            s = (kt[:, h].double() @ qv) / math.sqrt(D)
            kept_tok = mask[h, qi].repeat_interleave(128) & real
            sh = (kc[:, h] @ qv) / math.sqrt(D)
            drop = (~mask[h, qi]) & (lay.valid_count > 0)
            ref = 3.7  # any reference: it cancels
            num = (torch.exp(s[kept_tok] - ref)[:, None] * vt[kept_tok, h].double()).sum(0)
            den = torch.exp(s[kept_tok] - ref).sum()
            num = num + (torch.exp(sh[drop] - ref)[:, None] * vc[drop, h]).sum(0)
            den = den + (torch.exp(sh[drop] - ref) * counts[drop]).sum()
            torch.testing.assert_close(comp[r, h].double(), num / den, rtol=1e-5, atol=1e-5)


def test_row_that_kept_nothing_uses_reference_zero():
    lay, qt, kt, vt, mask = _case(3)
    m = mask.clone()
    m[0, 1] = False
    o, lse = oa.block_sparse_attention(qt, kt, vt, m, lay.valid_count, return_lse=True)
    assert torch.isinf(lse[0, 128:256]).all() and (o[128:256, 0] == 0).all()
    comp = oa.zero_order_compensation(o, lse, qt, kt, vt, m, lay.valid_count)
    kc, vc = oa.tile_summaries(kt, vt, lay.valid_count)
    p = torch.exp(qt[128:256, 0] @ kc[:, 0].T / math.sqrt(128)) * (lay.valid_count > 0)
    want = (p @ vc[:, 0]) / (1 + p @ lay.valid_count.float())[:, None]
    torch.testing.assert_close(comp[128:256, 0], want, rtol=1e-5, atol=1e-5)
