"""Layout-level entry points of the HIP kernels, with the reference's
signatures:

  gather_tiles / gather_and_pool / scatter_tiles_
      miowtion/kernels/tile_gather_triton.py:156-224
  pool_tiles                      miowtion/veda/predictor.py:82-130
  gather_lse                      miowtion/veda/attention.py:299-305
  index_lists                     miowtion/kernels/fa4.py:275-296
  block_sparse_attention          miowtion/kernels/fa4.py:299-377 (and its
                                  backward, fa4_sm8x/interface.py:2099)
  dense_attention                 miowtion/h3/attention.py:28-102
  teacher_heat                    miowtion/kernels/block_heat_triton.py:141-173

All run on the GPU through `miowtion_amd.ops`; CPU tensors raise
NotImplementedError (no fallback, never a silent dense path).
"""

from __future__ import annotations

import torch

from miowtion_amd import ops
from miowtion_amd import tiling

SECOND_RAW = 'raw'
SECOND_CENTRAL = 'central'


SUPPORTED_ARCH = 'gfx950'
# head_dim each family of kernels takes: the permutation and pooling kernels
# are written for 64 and 128 (tile_gather_triton.py:55-66), the attention,
# heat and compensation kernels for 128 only.
_HEAD_DIMS = {'gather': (64, 128), 'attention': (128,), 'heat': (128,)}


def _device_arch(device: torch.device) -> str:
    return torch.cuda.get_device_properties(device).gcnArchName.split(':')[0]


def supports(x: torch.Tensor, op: str = 'gather') -> bool:
    """Whether the kernels of `op` ('gather' for gather / pool / scatter,
    'attention' for the sparse and dense forwards, their backward and the
    compensation, 'heat' for the block heat) can take this tensor: the
    library loads, x is a bf16 tensor with a unit last stride and a head_dim
    that family implements, on a gfx950 device. The routing predicate of
    tile_gather_triton.py:55-66: a caller with another path falls through to
    it when this answers False, instead of reaching a kernel that raises.

    Raises:
        ValueError: If op is not one of the families above.
    """
    if op not in _HEAD_DIMS:
        raise ValueError(f'op must be one of {sorted(_HEAD_DIMS)}: {op!r}')
    if not (x.is_cuda and x.dtype == torch.bfloat16 and x.dim() >= 1
            and x.shape[-1] in _HEAD_DIMS[op] and x.stride(-1) == 1):
        return False
    if _device_arch(x.device) != SUPPORTED_ARCH:
        return False
    from miowtion_amd import _native
    try:
        _native.load()
    except ImportError:
        return False
    return True


def _heads(x: torch.Tensor, heads: torch.Tensor | None) -> torch.Tensor:
    if heads is None:
        return torch.arange(x.shape[1], device=x.device)
    return heads


def gather_tiles(x: torch.Tensor, layout: tiling.TileLayout,
                 heads: torch.Tensor | None) -> torch.Tensor:
    """[S, H, D] -> [N, H', D] tile order, padding slots zero."""
    return ops.gather(x, layout.gather_index, layout.slot_valid, layout.valid_count,
                      _heads(x, heads), True, False, False)[0]


def gather_and_pool(x: torch.Tensor, layout: tiling.TileLayout,
                    heads: torch.Tensor | None, second: bool = False) -> tuple:
    """gather_tiles and the predictor pooling in one pass over x.

    Returns (rows [N, H', D], feats [H', n, 3D] fp32) plus
    (E[x^2], Var(x)) [H', n, D] fp32 when `second`.
    """
    res = ops.gather(x, layout.gather_index, layout.slot_valid, layout.valid_count,
                     _heads(x, heads), True, True, second)
    return tuple(res)


def pool_seq(x: torch.Tensor, layout: tiling.TileLayout, heads: torch.Tensor | None,
             second: bool = False) -> tuple:
    """The pooling of gather_and_pool without writing the tile-ordered rows
    (one read of x): (feats,) or (feats, E[x^2], Var(x))."""
    res = ops.gather(x, layout.gather_index, layout.slot_valid, layout.valid_count,
                     _heads(x, heads), False, True, second)
    return tuple(res[1:])


def pool_tiles(x: torch.Tensor, layout: tiling.TileLayout, second: str | None = None) -> torch.Tensor:
    """Pooling of already tile-ordered rows [N, H', D] (predictor.py:82-130):
    [H', n, 3D] fp32 [mean | max | min], or [H', n, D] E[x^2] ('raw') /
    centred Var(x) ('central')."""
    if second not in (None, SECOND_RAW, SECOND_CENTRAL):
        raise ValueError(f'unknown second moment {second!r}')
    ident = _identity(layout)
    res = ops.gather(x, ident, layout.slot_valid, layout.valid_count,
                     torch.arange(x.shape[1], device=x.device), False, True, second is not None)
    if second is None:
        return res[1]
    return res[2] if second == SECOND_RAW else res[3]


def _identity(layout: tiling.TileLayout) -> torch.Tensor:
    """arange(num_slots) on the layout's device, cached for the layout."""
    return tiling.layout_cached(
        layout, 'identity',
        lambda: torch.arange(layout.n_tiles * tiling.TILE_SIZE, device=layout.valid_count.device))


def scatter_tiles_(out: torch.Tensor, tiled: torch.Tensor, layout: tiling.TileLayout,
                   heads: torch.Tensor | None) -> None:
    """Writes tile-ordered rows into out[S + 1, H, D] (padding slots dropped)."""
    if out.shape[0] != layout.seq_len + 1:
        raise ValueError(f'scatter buffer needs {layout.seq_len + 1} rows')
    ops.scatter_(out, tiled, layout.scatter_index, layout.slot_valid, _heads(out, heads))


def gather_lse(lse: torch.Tensor, layout: tiling.TileLayout, heads: torch.Tensor) -> torch.Tensor:
    """[S, H] LSE -> [N, H'] tile order, 0 on padding slots."""
    return ops.gather_lse(lse, layout.gather_index, layout.slot_valid, heads)


def index_lists(block_mask: torch.Tensor, layout: tiling.TileLayout,
                transpose: bool = False) -> tuple[torch.Tensor, ...]:
    """(partial_cnt, partial_idx, full_cnt, full_idx) (fa4.py:275-296): cnt
    [1, H', rows] and idx [1, H', rows, cols] int32, members ascending then
    non-members ascending.

    transpose: the Q-direction lists of the backward (per key tile, its query
    tiles; a key tile's members are all full or all partial, by its own
    fullness). Needs the mask of all n_tiles query tiles.
    """
    if not transpose:
        return tuple(ops.index_lists(block_mask, layout.kv_ok, layout.full_tile))
    if block_mask.shape[1] != layout.n_tiles:
        raise ValueError('transposed lists need the block mask of all query tiles')
    mt = (block_mask & layout.kv_ok[None, None, :]).transpose(1, 2).contiguous()
    ones = torch.ones(mt.shape[2], dtype=torch.bool, device=mt.device)
    # with every column "full", each row's members land in the full list
    empty_cnt, empty_idx, cnt, idx = ops.index_lists(mt, ones, ones)
    full_row = layout.full_tile.to(mt.device)[None, None, :]
    return (torch.where(full_row, empty_cnt, cnt),
            torch.where(full_row[..., None], empty_idx, idx).contiguous(),
            torch.where(full_row, cnt, empty_cnt),
            torch.where(full_row[..., None], idx, empty_idx).contiguous())


def _front_tiles(layout: tiling.TileLayout, rows: int) -> int:
    """Tiles dispatched first: the ones a Veda mask makes dense (the global
    rows keep every key tile and every row keeps the global columns,
    mask.py:288-317; they come after the video tiles in tile order), when
    all `rows` query tiles are present. Order only, no value changes."""
    return layout.n_tiles - layout.n_video_tiles if rows == layout.n_tiles else 0


class _BlockSparseAttention(torch.autograd.Function):
    """Block-sparse attention with gradients: the forward kernel, then the
    backward kernels on the forward and the transposed block lists
    (FlashAttnFunc, fa4_sm8x/interface.py:3641-3790, given
    block_sparse_tensors_bwd as fa4.py:352-360 builds them). The LSE output
    is differentiable too (its gradient enters through D)."""

    @staticmethod
    def forward(ctx, q, k, v, block_mask, layout):
        lists = index_lists(block_mask, layout)
        lists_t = index_lists(block_mask, layout, transpose=True)
        ctx.front = _front_tiles(layout, q.shape[0] // 128)
        out, lse = ops.block_sparse_fwd(q, k, v, *lists, layout.valid_count, True, ctx.front)
        ctx.save_for_backward(q, k, v, out, lse, *lists, *lists_t, layout.valid_count)
        ctx.set_materialize_grads(False)
        return out, lse

    @staticmethod
    def backward(ctx, dout, dlse):
        q, k, v, out, lse, *rest = ctx.saved_tensors
        lists, lists_t, valid_count = rest[:4], rest[4:8], rest[8]
        if dout is None:
            dout = torch.zeros_like(out)
        dq, dk, dv = ops.block_sparse_bwd(
            q, k, v, out, dout.contiguous(), lse, None if dlse is None else dlse.contiguous(),
            *lists, *lists_t, valid_count, ctx.front)
        return dq, dk, dv, None, None


def block_sparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           block_mask: torch.Tensor, layout: tiling.TileLayout,
                           return_lse: bool = False):
    """Block-sparse attention on tile-ordered tensors (fa4.py:299-377).

    Args:
        q: [R * 128, H', D] bf16 query tiles (rows of `block_mask`).
        k, v: [N, H', D] bf16, all key tiles.
        block_mask: [H', R, n_tiles] bool.
        layout: Tile layout (valid key prefix of every key tile).
        return_lse: Also return the [H', R * 128] fp32 natural-log LSE.

    Returns:
        [R * 128, H', D] bf16, or (out, lse). Differentiable in q, k, v
        (and through the LSE) when they require grad.

    Raises:
        ValueError: If gradients are required for a subset of query tiles.
    """
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        if block_mask.shape[1] != layout.n_tiles:
            raise ValueError('backward needs the block mask of all query tiles')
        out, lse = _BlockSparseAttention.apply(q, k, v, block_mask, layout)
        return (out, lse) if return_lse else out
    lists = index_lists(block_mask, layout)
    return block_sparse_attention_lists(q, k, v, lists, layout, return_lse)


def block_sparse_attention_lists(q, k, v, lists, layout: tiling.TileLayout,
                                 return_lse: bool = False):
    """Same as block_sparse_attention with prebuilt (part_cnt, part_idx,
    full_cnt, full_idx) lists (the BlockSparseTensorsTorch path of fa4.py)."""
    part_cnt, part_idx, full_cnt, full_idx = lists
    res = ops.block_sparse_fwd(q, k, v, part_cnt, part_idx, full_cnt, full_idx,
                               layout.valid_count, return_lse,
                               _front_tiles(layout, q.shape[0] // 128))
    return (res[0], res[1]) if return_lse else res[0]


def block_sparse_attention_seq_(out: torch.Tensor, q: torch.Tensor, k: torch.Tensor,
                                v: torch.Tensor, lists, layout: tiling.TileLayout,
                                heads: torch.Tensor | None) -> None:
    """scatter_tiles_(out, block_sparse_attention_lists(gather_tiles(q), k, v,
    lists), layout, heads) in one kernel: q [S, H, D] in sequence order,
    out the [S + 1, H, D] scatter buffer, k / v tile-ordered [N, H', D]
    (the sequence of miowtion/veda/attention.py:760-788)."""
    part_cnt, part_idx, full_cnt, full_idx = lists
    ops.block_sparse_fwd_seq_(out, q, k, v, layout.gather_index, layout.scatter_index,
                              layout.slot_valid, _heads(q, heads), part_cnt, part_idx, full_cnt,
                              full_idx, layout.valid_count,
                              _front_tiles(layout, layout.gather_index.numel() // 128))


def block_sparse_attention_seq_kv_(out: torch.Tensor, q: torch.Tensor, k: torch.Tensor,
                                   v: torch.Tensor, lists, layout: tiling.TileLayout,
                                   heads: torch.Tensor | None) -> None:
    """block_sparse_attention_seq_ with the gather of k and v fused in too:
    q, k, v [S, H, D] in sequence order (the sequence gather_tiles of q, k,
    v, fa4.block_sparse_attention, scatter_tiles_ of
    miowtion/veda/attention.py:760-788, in one kernel)."""
    part_cnt, part_idx, full_cnt, full_idx = lists
    ops.block_sparse_fwd_seq_kv_(out, q, k, v, layout.gather_index, layout.scatter_index,
                                 layout.slot_valid, _heads(q, heads), part_cnt, part_idx,
                                 full_cnt, full_idx, layout.valid_count,
                                 _front_tiles(layout, layout.gather_index.numel() // 128))


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, used: int,
                    return_lse: bool = False):
    """Dense attention of rows [0, used) among themselves (h3/attention.py:28-102):
    out [S, H, D] zero on padding rows, lse [S, H] fp32 (0 on padding) or None."""
    res = ops.dense_fwd(q, k, v, used, return_lse)
    return (res[0], res[1]) if return_lse else (res[0], None)


def teacher_heat(q: torch.Tensor, k: torch.Tensor, lse: torch.Tensor,
                 layout: tiling.TileLayout, q_tiles: torch.Tensor,
                 reduce: str = 'max') -> torch.Tensor:
    """[H', R, n_tiles] fp32 block heat ('max' peak / 'sum' mass) of query
    tiles `q_tiles` (heatmap.py:36-110)."""
    return ops.block_heat(q, k, lse, layout.valid_count, q_tiles, reduce)


def dense_heat(q: torch.Tensor, k: torch.Tensor, layout: tiling.TileLayout,
               q_tiles: torch.Tensor, reduce: str = 'max', v: torch.Tensor | None = None):
    """The teacher's dense pass in tile order, fused with the block heat.

    One pass over every valid key of the layout gives, for the query tiles
    `q_tiles`, the row LSE and a per-(key tile, row) log2 statistic; a second,
    HBM-bound kernel turns those into the heat of heatmap.py:36-110 (the
    same values as teacher_heat with the dense LSE). With `v` the pass also
    returns the dense output in tile order (the form
    docs/features/veda_kernel.md:285-289 plans for the teacher).

    Returns:
        (heat [H', R, n] fp32, lse [H', R * 128] fp32, out [R * 128, H', D]
        bf16 or None).
    """
    res = ops.dense_heat(q, k, v, layout.valid_count, q_tiles, reduce)
    return res[0], res[1], (res[2] if v is not None else None)


def tile_summaries(k: torch.Tensor, v: torch.Tensor, layout: tiling.TileLayout):
    """(kc, vc) [n, H', D] bf16: per key tile the mean of K and the sum of V
    over its real rows (compensation_triton.py:150-170)."""
    kc, vc = ops.tile_summaries(k, v, layout.valid_count)
    return kc, vc


def zero_order_compensation(o_kept: torch.Tensor, lse_kept: torch.Tensor, q: torch.Tensor,
                            k: torch.Tensor, v: torch.Tensor, block_mask: torch.Tensor,
                            layout: tiling.TileLayout) -> torch.Tensor:
    """Adds the zero-order term of every dropped key tile to a block-sparse
    output (miowtion/veda/attention.py:591-689; the arithmetic of
    compensation_triton.compensate, :173-225): a dropped tile is one virtual
    key at its centroid carrying the sum of its values, weighted by its real
    row count.

    Args:
        o_kept: [R * 128, H', D] bf16 block-sparse output over the kept blocks.
        lse_kept: [H', R * 128] fp32 natural-log LSE over the kept blocks.
        q: [R * 128, H', D] bf16 query tiles; k, v: [N, H', D] bf16 key tiles.
        block_mask: [H', R, n] bool, True where the block was kept.
        layout: Tile layout (real rows of every key tile).

    Returns:
        [R * 128, H', D] bf16.
    """
    kc, vc = tile_summaries(k, v, layout)
    return ops.zero_order_compensation(o_kept, lse_kept, q, kc, vc, block_mask,
                                       layout.valid_count)


def compensated_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          block_mask: torch.Tensor, layout: tiling.TileLayout,
                          lists: tuple[torch.Tensor, ...] | None = None) -> torch.Tensor:
    """Block-sparse attention over the kept blocks plus the zero-order term
    of the dropped ones (compensation_triton.attention, :228-258), in one
    pass: the kept blocks and then every dropped tile's virtual key go
    through the same online softmax, so o_kept and its LSE never leave the
    kernel. Same result as zero_order_compensation after
    block_sparse_attention, without the bf16 rounding of o_kept between
    them.

    Args:
        q: [R * 128, H', D] bf16 query tiles; k, v: [N, H', D] bf16 key tiles.
        block_mask: [H', R, n] bool, True where the block is kept exactly.
        layout: Tile layout.
        lists: index_lists of block_mask & kv_ok, if already built.

    Returns:
        [R * 128, H', D] bf16.
    """
    kept = block_mask & layout.kv_ok[None, None, :]
    if lists is None:
        lists = index_lists(kept, layout)
    kc, vc = tile_summaries(k, v, layout)
    return ops.compensated_attention(q, k, v, *lists, kc, vc, kept, layout.valid_count,
                                     _front_tiles(layout, q.shape[0] // 128))
