"""veda_block_sparse_bwd_noalloc (the backward whose per-row statistics live
in the library's own device array, for callers that cannot allocate) against
veda_block_sparse_bwd with a caller workspace, both through the C ABI:
bit-identical gradients on two calls in a row, the first at BASELINE C2
geometry with all 48 heads (28,416 (head, query tile) pairs, near the
array's 32,768), the second on a smaller layout (the array keeps the first
call's contents, which must not leak into the second). A call beyond the
array is refused on the host."""

import math

import pytest
import torch

from miowtion_amd import _native
from miowtion_amd import kernels
from miowtion_amd import mask as pm
from miowtion_amd import ops
from tests import helpers

SCRATCH_BYTES = 64 << 20


def _case(spec, heads, ratio, seed):
    lay = helpers.product_layout(*spec, device='cuda')
    g = torch.Generator(device='cuda').manual_seed(seed)
    q, k, v = (kernels.gather_tiles(
        torch.randn(lay.seq_len, heads, 128, generator=g, device='cuda').to(torch.bfloat16), lay,
        None) for _ in range(3))
    scores = torch.rand(heads, lay.n_tiles, lay.n_tiles, generator=g, device='cuda')
    sel = pm.select_video_blocks(scores[:, :lay.n_video_tiles], lay,
                                 pm.column_blocks(lay, pm.Budget(ratio=ratio)))
    mask = pm.dense_block_mask(sel, lay)
    lists = kernels.index_lists(mask, lay)
    lists_t = kernels.index_lists(mask, lay, transpose=True)
    out, lse = ops.block_sparse_fwd(q, k, v, *lists, lay.valid_count, True, 0)
    dout = torch.randn(q.shape, generator=g, device='cuda').to(torch.bfloat16)
    dlse = torch.randn(lse.shape, generator=g, device='cuda')
    return dict(lay=lay, q=q, k=k, v=v, out=out, lse=lse, dout=dout, dlse=dlse, lists=lists,
                lists_t=lists_t)


def _grads(c, workspace):
    """Calls the backward entry point through the C ABI; workspace None: the
    no-allocation one."""
    q, k, v, out, dout, lse, dlse = (c[n] for n in ('q', 'k', 'v', 'out', 'dout', 'lse', 'dlse'))
    part_cnt, part_idx, full_cnt, full_idx = c['lists']
    part_cnt_t, part_idx_t, full_cnt_t, full_idx_t = c['lists_t']
    heads = q.shape[1]
    r_tiles, n_k = q.shape[0] // 128, k.shape[0] // 128
    dq, dk, dv = (torch.full_like(t, float('nan')) for t in (q, k, v))
    args = [q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
            v.data_ptr(), v.stride(0), v.stride(1), out.data_ptr(), out.stride(0), out.stride(1),
            dout.data_ptr(), dout.stride(0), dout.stride(1), lse.data_ptr(), lse.stride(0),
            lse.stride(1), dlse.data_ptr(), dlse.stride(0), dlse.stride(1), heads, 128, r_tiles,
            n_k, full_cnt.data_ptr(), full_idx.data_ptr(), part_cnt.data_ptr(),
            part_idx.data_ptr(), part_idx.shape[3], full_cnt_t.data_ptr(), full_idx_t.data_ptr(),
            part_cnt_t.data_ptr(), part_idx_t.data_ptr(), part_idx_t.shape[3],
            c['lay'].valid_count.data_ptr(), 1.0 / math.sqrt(128), dq.data_ptr(), dq.stride(0),
            dq.stride(1), dk.data_ptr(), dk.stride(0), dk.stride(1), dv.data_ptr(), dv.stride(0),
            dv.stride(1)]
    stream = torch.cuda.current_stream().cuda_stream
    if workspace is None:
        _native.call('veda_block_sparse_bwd_noalloc', *args, 0, stream)
    else:
        _native.call('veda_block_sparse_bwd', *args, workspace.data_ptr(), workspace.numel(), 0,
                     stream)
    torch.cuda.synchronize()
    return dq, dk, dv


@pytest.mark.gpu
def test_no_alloc_backward_matches_the_workspace_backward():
    cases = [('C2', helpers.CONFIGS['C2'], 48, 0.1), ('small', helpers.small_layout(), 3, 0.3)]
    for name, spec, heads, ratio in cases:
        print(f'no-alloc backward: {name}, {heads} heads', flush=True)
        c = _case(spec, heads, ratio, seed=len(name))
        pairs = heads * (c['q'].shape[0] // 128)
        assert pairs * 2048 <= SCRATCH_BYTES
        work = torch.empty(pairs * 2048, dtype=torch.uint8, device='cuda')
        want = _grads(c, work)
        got = _grads(c, None)
        for a, b in zip(got, want):
            assert not torch.isnan(a.float()).any()
            assert torch.equal(a, b)
        assert any(t.float().abs().max() > 0 for t in got)


def test_no_alloc_backward_refuses_more_than_its_scratch():
    # 48 heads x 700 query tiles need 68.8 MB of statistics: refused on the
    # host, before any launch (every pointer may stay NULL)
    args = [None, 0, 0] * 5 + [None, 0, 0, None, 0, 0] + [48, 128, 700, 700] + \
        [None, None, None, None, 700, None, None, None, None, 700, None, 1.0] + [None, 0, 0] * 3
    with pytest.raises(ValueError, match='scratch'):
        _native.call('veda_block_sparse_bwd_noalloc', *args, 0, None)
