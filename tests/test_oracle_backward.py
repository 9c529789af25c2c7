"""The oracle's block-sparse attention gradients (autograd through the masked
softmax of miowtion/kernels/reference.py:23-56, the expected values of the
reference's tests/gpu/test_kernels_gpu.py:200-250), pinned by what does not
use autograd or restate the gradient formulas:

  * central finite differences of the float64 forward along random
    directions, for dq, dk, dv and for the LSE term (dlse);
  * with every tile kept and every key valid, torch's own
    scaled_dot_product_attention (another forward implementation) gives the
    same gradients;
  * block structure: a key tile no query tile keeps, padding keys and a
    query tile that keeps nothing get exactly zero gradient;
  * the transposed index lists (fa4.py:288-296) list, per key tile, exactly
    the query tiles that keep it;
  * the per-tile form (used at the BASELINE sizes) equals the masked-dense
    form.
"""

import torch

from oracle import attention as oa
from oracle import mask as om
from oracle import tiling as ot
from tests import helpers


def _case(seed=0, heads=2, density=0.4, grid=(2, 8, 12), shape='2x8x8', text=40):
    spec = helpers.small_layout(grid=grid, shape=shape, text=text, extra=16)
    lay = helpers.oracle_layout(*spec)
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(lay.seq_len, heads, 128, generator=g) for _ in range(3))
    hs = torch.arange(heads)
    qt, kt, vt = (ot.gather_tiles(t, lay, hs) for t in (q, k, v))
    n = lay.n_tiles
    mask = torch.rand(heads, n, n, generator=g) < density
    mask |= torch.eye(n, dtype=torch.bool)[None]
    return lay, qt.double(), kt.double(), vt.double(), mask, g


def _loss(q, k, v, mask, lay, dout, dlse):
    o, lse = oa.block_sparse_attention(q, k, v, mask, lay.valid_count, return_lse=True,
                                       compute_dtype=torch.float64)
    fin = torch.isfinite(lse)
    return (o * dout).sum() + (lse[fin] * dlse[fin]).sum()


def test_finite_differences_float64():
    lay, q, k, v, mask, g = _case()
    assert (lay.valid_count < 128).any() and (lay.valid_count == 128).any()
    dout = torch.randn(q.shape, generator=g, dtype=torch.float64)
    dlse = torch.randn(q.shape[1], q.shape[0], generator=g, dtype=torch.float64)
    grads = oa.block_sparse_attention_grads(q, k, v, mask, lay.valid_count, dout, dlse,
                                            dtype=torch.float64)
    eps = 1e-6
    for which, grad in enumerate(grads):
        for _ in range(2):
            d = torch.randn(grad.shape, generator=g, dtype=torch.float64)
            args = [q, k, v]
            plus, minus = list(args), list(args)
            plus[which] = args[which] + eps * d
            minus[which] = args[which] - eps * d
            fd = (_loss(*plus, mask, lay, dout, dlse) - _loss(*minus, mask, lay, dout, dlse)) / (2 * eps)
            an = (grad * d).sum()
            assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (which, fd.item(), an.item())


def test_dense_mask_matches_torch_sdpa():
    lay, q, k, v, mask, g = _case(1)
    n = lay.n_tiles
    N = k.shape[0]
    allm = torch.ones(q.shape[1], n, n, dtype=torch.bool)
    dout = torch.randn(q.shape, generator=g, dtype=torch.float64)
    got = oa.block_sparse_attention_grads(q, k, v, allm, lay.valid_count, dout,
                                          dtype=torch.float64)
    key_valid = (torch.arange(128)[None, :] < lay.valid_count[:, None]).reshape(-1)[:N]
    a, b, c = (t.clone().permute(1, 0, 2).requires_grad_(True) for t in (q, k, v))
    out = torch.nn.functional.scaled_dot_product_attention(a, b, c, attn_mask=key_valid[None, None, :])
    out.backward(dout.permute(1, 0, 2))
    for mine, ref in zip(got, (a.grad, b.grad, c.grad)):
        torch.testing.assert_close(mine, ref.permute(1, 0, 2), rtol=1e-9, atol=1e-9)


def test_structural_zeros():
    lay, q, k, v, mask, g = _case(2)
    m = mask.clone()
    m[:, :, 1] = False      # key tile 1: kept by no query tile
    m[0, 2, :] = False      # head 0, query tile 2 keeps nothing
    dout = torch.randn(q.shape, generator=g, dtype=torch.float64)
    dq, dk, dv = oa.block_sparse_attention_grads(q, k, v, m, lay.valid_count, dout,
                                                 dtype=torch.float64)
    assert (dk[128:256] == 0).all() and (dv[128:256] == 0).all()
    assert (dq[256:384, 0] == 0).all() and (dq[256:384, 1] != 0).any()
    pad = (torch.arange(128)[None, :] >= lay.valid_count[:, None]).reshape(-1)
    assert pad.any()
    assert (dk[pad] == 0).all() and (dv[pad] == 0).all()
    assert (dk[~pad] != 0).any()


def test_transposed_lists():
    lay, q, k, v, mask, g = _case(3)
    pc, pi, fc, fi = om.index_lists(mask, lay, transpose=True)
    H, n = mask.shape[0], lay.n_tiles
    assert tuple(fi.shape) == (1, H, n, n)
    want = (mask & lay.kv_ok).transpose(1, 2)
    for h in range(H):
        for j in range(n):
            full = bool(lay.full_tile[j])
            members = sorted(torch.nonzero(want[h, j]).flatten().tolist())
            cnt, idx = (fc, fi) if full else (pc, pi)
            other_cnt = (pc if full else fc)[0, h, j]
            assert other_cnt == 0
            assert idx[0, h, j, :cnt[0, h, j]].tolist() == members
            rest = idx[0, h, j, cnt[0, h, j]:].tolist()
            assert rest == sorted(set(range(n)) - set(members))
    # and the scale convention of the gradients: doubling dout doubles them
    dout = torch.randn(q.shape, generator=g, dtype=torch.float64)
    a = oa.block_sparse_attention_grads(q, k, v, mask, lay.valid_count, dout, dtype=torch.float64)
    b = oa.block_sparse_attention_grads(q, k, v, mask, lay.valid_count, 2 * dout,
                                        dtype=torch.float64)
    for x, y in zip(a, b):
        torch.testing.assert_close(2 * x, y, rtol=1e-12, atol=1e-12)


def test_by_tile_form_equals_masked_dense_form():
    lay, q, k, v, mask, g = _case(4, heads=3)
    m = mask.clone()
    m[1, 0, :] = False  # a query tile with no key
    dout = torch.randn(q.shape, generator=g, dtype=torch.float64)
    dlse = torch.randn(q.shape[1], q.shape[0], generator=g, dtype=torch.float64)
    a = oa.block_sparse_attention_grads(q, k, v, m & lay.kv_ok, lay.valid_count, dout, dlse,
                                        dtype=torch.float64)
    b = oa.block_sparse_attention_grads_by_tile(q, k, v, m, lay.valid_count, dout, dlse,
                                                dtype=torch.float64)
    for x, y in zip(a, b):
        torch.testing.assert_close(x, y, rtol=1e-10, atol=1e-10)
