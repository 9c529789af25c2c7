"""The kernels' store paths for rows that are not 16-byte aligned.

The sparse forward stages its output rows in LDS and stores them 16 bytes
per lane when every row start is 16-byte aligned; rows whose strides are
multiples of 4 elements (but not 8) take 8-byte stores. The backward's dQ
epilogue and the dK / dV stores have the same split (dq / dk / dv need only
8-byte alignment), and the compensation of a given output reads o_kept rows
through LDS only when they are 16-byte aligned. Each fallback is driven
here through the C ABI with row views into [rows, H, 132] buffers (strides
that are multiples of 4, not 8) and 8-byte base offsets, and must give
bit-identical results to the aligned form.
"""

import math

import pytest
import torch

from miowtion_amd import _native
from miowtion_amd import kernels
from miowtion_amd import mask as pm
from miowtion_amd import ops
from tests import helpers

pytestmark = pytest.mark.gpu


def _rows_view(rows, heads, offset_elems=0, pad=4):
    """[rows, heads, 128] bf16 view into a [rows, heads, 128 + pad] buffer,
    its first element `offset_elems` past a 16-byte-aligned allocation."""
    flat = torch.full((rows * heads * (128 + pad) + offset_elems,), float('nan'),
                      dtype=torch.bfloat16, device='cuda')
    v = flat[offset_elems:].view(rows, heads, 128 + pad)[..., :128]
    assert v.data_ptr() % 16 == 2 * offset_elems % 16
    return v


def _case(seed=0, heads=4):
    spec = helpers.small_layout()
    lay = helpers.product_layout(*spec, device='cuda')
    q, k, v = helpers.qkv(lay.seq_len, heads, 128, seed=seed)
    hs = torch.arange(heads, device='cuda')
    qt, kt, vt = (kernels.gather_tiles(t.cuda(), lay, hs) for t in (q, k, v))
    scores = torch.rand(heads, lay.n_video_tiles, lay.n_video_tiles,
                        generator=torch.Generator().manual_seed(seed)).cuda()
    sel = pm.select_video_blocks(scores, lay, pm.column_blocks(lay, pm.Budget(ratio=0.3)))
    mask = pm.dense_block_mask(sel, lay)
    return lay, q.cuda(), qt, kt, vt, mask


def test_forward_output_rows_8_byte_aligned():
    lay, q, qt, kt, vt, mask = _case()
    lists = kernels.index_lists(mask, lay)
    want, want_lse = kernels.block_sparse_attention_lists(qt, kt, vt, lists, lay, return_lse=True)
    part_cnt, part_idx, full_cnt, full_idx = lists
    heads, r = qt.shape[1], qt.shape[0] // 128
    out = _rows_view(qt.shape[0], heads)
    assert (out.stride(0) | out.stride(1)) % 8 == 4   # rows 8-byte aligned only
    lse = torch.empty(heads, qt.shape[0], dtype=torch.float32, device='cuda')
    _native.call('veda_block_sparse_fwd', qt.data_ptr(), qt.stride(0), qt.stride(1),
                 kt.data_ptr(), kt.stride(0), kt.stride(1), vt.data_ptr(), vt.stride(0),
                 vt.stride(1), heads, 128, r, kt.shape[0] // 128, full_cnt.data_ptr(),
                 full_idx.data_ptr(), part_cnt.data_ptr(), part_idx.data_ptr(),
                 part_idx.shape[3], lay.valid_count.data_ptr(), 1.0 / math.sqrt(128),
                 out.data_ptr(), out.stride(0), out.stride(1), lse.data_ptr(), lse.stride(0),
                 lse.stride(1), 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    assert torch.equal(lse, want_lse)
    # the sequence-order entry (gather of q and scatter of out fused in)
    seq = torch.zeros(lay.seq_len + 1, heads, 128, dtype=torch.bfloat16, device='cuda')
    kernels.block_sparse_attention_seq_(seq, q, kt, vt, lists, lay, None)
    strided = _rows_view(lay.seq_len + 1, heads)
    strided.zero_()
    kernels.block_sparse_attention_seq_(strided, q, kt, vt, lists, lay, None)
    assert torch.equal(strided.view(torch.int16), seq.view(torch.int16))


def test_backward_gradients_into_8_byte_aligned_rows():
    lay, _, qt, kt, vt, mask = _case(seed=1)
    g = torch.Generator(device='cuda').manual_seed(2)
    dout = torch.randn(qt.shape, generator=g, device='cuda').to(torch.bfloat16)
    lists = kernels.index_lists(mask, lay)
    lists_t = kernels.index_lists(mask, lay, transpose=True)
    out, lse = ops.block_sparse_fwd(qt, kt, vt, *lists, lay.valid_count, True, 0)
    want = ops.block_sparse_bwd(qt, kt, vt, out, dout, lse, None, *lists, *lists_t,
                                lay.valid_count, 0)
    heads, r, n_k = qt.shape[1], qt.shape[0] // 128, kt.shape[0] // 128
    dq, dk, dv = (_rows_view(t.shape[0], heads, offset_elems=4) for t in (qt, kt, vt))
    for t in (dq, dk, dv):
        assert t.data_ptr() % 16 == 8 and (t.stride(0) | t.stride(1)) % 8 == 4
    work = torch.empty(heads * r * 512, dtype=torch.float32, device='cuda')
    pc, pi, fc, fi = lists
    pct, pit, fct, fit = lists_t
    _native.call('veda_block_sparse_bwd', qt.data_ptr(), qt.stride(0), qt.stride(1),
                 kt.data_ptr(), kt.stride(0), kt.stride(1), vt.data_ptr(), vt.stride(0),
                 vt.stride(1), out.data_ptr(), out.stride(0), out.stride(1), dout.data_ptr(),
                 dout.stride(0), dout.stride(1), lse.data_ptr(), lse.stride(0), lse.stride(1),
                 None, 0, 0, heads, 128, r, n_k, fc.data_ptr(), fi.data_ptr(), pc.data_ptr(),
                 pi.data_ptr(), pi.shape[3], fct.data_ptr(), fit.data_ptr(), pct.data_ptr(),
                 pit.data_ptr(), pit.shape[3], lay.valid_count.data_ptr(), 1.0 / math.sqrt(128),
                 dq.data_ptr(), dq.stride(0), dq.stride(1), dk.data_ptr(), dk.stride(0),
                 dk.stride(1), dv.data_ptr(), dv.stride(0), dv.stride(1), work.data_ptr(),
                 work.numel() * 4, 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for name, got, w in zip(('dq', 'dk', 'dv'), (dq, dk, dv), want):
        assert torch.equal(got.view(torch.int16), w.view(torch.int16)), name


def test_compensation_reads_o_kept_rows_8_byte_aligned():
    lay, _, qt, kt, vt, mask = _case(seed=3)
    o, lse = kernels.block_sparse_attention(qt, kt, vt, mask, lay, return_lse=True)
    want = kernels.zero_order_compensation(o, lse, qt, kt, vt, mask, lay)
    heads = qt.shape[1]
    for offset in (4, 0):   # 8-byte base, then 16-byte base with 8-byte row strides
        o_kept = _rows_view(o.shape[0], heads, offset_elems=offset)
        o_kept.copy_(o)
        got = kernels.zero_order_compensation(o_kept, lse, qt, kt, vt, mask, lay)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), offset
