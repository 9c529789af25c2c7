"""PyTorch-ROCm custom ops (`torch.ops.veda.*`) over the C ABI of
libveda_hip.so.

Each op validates shapes and devices on the host, allocates its outputs with
torch (device memory and the current stream are all torch provides here), and
launches the HIP kernels through `_native.call` on the current stream. The
ops take plain tensors; `miowtion_amd.kernels` wraps them in the reference's
layout-level signatures.

Every op refuses CPU tensors with NotImplementedError: there is no CPU path.
"""

from __future__ import annotations

import math

import torch

from miowtion_amd import _native

TILE = 128


def _require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise NotImplementedError(
                'miowtion_amd kernels run on the GPU only (got a tensor on '
                f'{t.device}); there is no CPU fallback')


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _p(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def _check_rows(name: str, t: torch.Tensor) -> None:
    if t.dim() != 3 or t.stride(-1) != 1:
        raise ValueError(f'{name} must be [rows, heads, head_dim] with a contiguous last dim')
    if t.dtype != torch.bfloat16:
        raise ValueError(f'{name} must be bfloat16, got {t.dtype}')


# --------------------------------------------------------------------------
# gather / pool / scatter (miowtion/kernels/tile_gather_triton.py:156-224)


@torch.library.custom_op('veda::gather', mutates_args=())
def gather(x: torch.Tensor, gather_index: torch.Tensor, slot_valid: torch.Tensor,
           valid_count: torch.Tensor, heads: torch.Tensor, write_rows: bool, pool: bool,
           second: bool) -> list[torch.Tensor]:
    """Returns [tiles] or [tiles, feats] or [tiles, feats, sq, var]; `tiles`
    is an empty tensor when write_rows is False (pool-only)."""
    _require_gpu(x, gather_index, slot_valid, valid_count, heads)
    _check_rows('x', x)
    n_slots = gather_index.numel()
    if n_slots % TILE:
        raise ValueError('gather_index must hold n_tiles * 128 slots')
    n_tiles = n_slots // TILE
    d = x.shape[-1]
    if d not in (64, 128):
        raise ValueError('tile kernels need contiguous head_dim 64 or 128')
    hp = heads.numel()
    dev = x.device
    out = (torch.empty(n_slots, hp, d, dtype=x.dtype, device=dev) if write_rows
           else torch.empty(0, dtype=x.dtype, device=dev))
    feats = sq = var = None
    if pool:
        feats = torch.empty(hp, n_tiles, 3 * d, dtype=torch.float32, device=dev)
        if second:
            sq = torch.empty(hp, n_tiles, d, dtype=torch.float32, device=dev)
            var = torch.empty(hp, n_tiles, d, dtype=torch.float32, device=dev)
    _native.call('veda_gather_tiles', x.data_ptr(), x.shape[0], x.shape[1], x.stride(0),
                 x.stride(1), gather_index.data_ptr(), slot_valid.data_ptr(),
                 valid_count.data_ptr(), n_tiles, heads.data_ptr(), hp, d,
                 out.data_ptr() if write_rows else None,
                 out.stride(0) if write_rows else 0, out.stride(1) if write_rows else 0,
                 _p(feats), _p(sq), _p(var), _stream(x))
    res = [out]
    if pool:
        res.append(feats)
        if second:
            res += [sq, var]
    return res


@gather.register_fake
def _(x, gather_index, slot_valid, valid_count, heads, write_rows, pool, second):
    n_slots, hp, d = gather_index.numel(), heads.numel(), x.shape[-1]
    n_tiles = n_slots // TILE
    res = [x.new_empty(n_slots, hp, d) if write_rows else x.new_empty(0)]
    if pool:
        res.append(x.new_empty(hp, n_tiles, 3 * d, dtype=torch.float32))
        if second:
            res += [x.new_empty(hp, n_tiles, d, dtype=torch.float32) for _ in range(2)]
    return res


@torch.library.custom_op('veda::scatter_', mutates_args=('out',))
def scatter_(out: torch.Tensor, tiled: torch.Tensor, scatter_index: torch.Tensor,
             slot_valid: torch.Tensor, heads: torch.Tensor) -> None:
    _require_gpu(out, tiled, scatter_index, slot_valid, heads)
    _check_rows('out', out)
    _check_rows('tiled', tiled)
    n_slots = scatter_index.numel()
    if tiled.shape[0] != n_slots or tiled.shape[1] != heads.numel():
        raise ValueError(f'tiled {tuple(tiled.shape)} does not match {n_slots} slots x '
                         f'{heads.numel()} heads')
    if tiled.dtype != out.dtype or tiled.shape[-1] != out.shape[-1]:
        raise ValueError('tiled and out differ in dtype or head_dim')
    _native.call('veda_scatter_tiles', tiled.data_ptr(), tiled.stride(0), tiled.stride(1),
                 scatter_index.data_ptr(), slot_valid.data_ptr(), n_slots // TILE,
                 heads.data_ptr(), heads.numel(), out.shape[-1], out.data_ptr(),
                 out.shape[0], out.shape[1], out.stride(0), out.stride(1), _stream(out))


@torch.library.custom_op('veda::gather_lse', mutates_args=())
def gather_lse(lse: torch.Tensor, gather_index: torch.Tensor, slot_valid: torch.Tensor,
               heads: torch.Tensor) -> torch.Tensor:
    _require_gpu(lse, gather_index, slot_valid, heads)
    if lse.dtype != torch.float32 or lse.dim() != 2:
        raise ValueError('lse must be fp32 [S, H]')
    out = torch.empty(gather_index.numel(), heads.numel(), dtype=torch.float32,
                      device=lse.device)
    _native.call('veda_gather_lse', lse.data_ptr(), lse.shape[0], lse.shape[1], lse.stride(0),
                 lse.stride(1), gather_index.data_ptr(), slot_valid.data_ptr(),
                 gather_index.numel(), heads.data_ptr(), heads.numel(), out.data_ptr(),
                 _stream(lse))
    return out


@gather_lse.register_fake
def _(lse, gather_index, slot_valid, heads):
    return lse.new_empty(gather_index.numel(), heads.numel())


# --------------------------------------------------------------------------
# selection, block mask, lists (miowtion/veda/mask.py, miowtion/kernels/fa4.py)


@torch.library.custom_op('veda::select_topk', mutates_args=('index', 'keep'))
def select_topk(scores: torch.Tensor, block_start: int, n_cols: int, kv_ok: torch.Tensor,
                rows: torch.Tensor, k_lo: int, k_hi: int, extra: torch.Tensor,
                index: torch.Tensor, keep: torch.Tensor, col0: int) -> None:
    """One column block of the top-k; writes index/keep[:, :, col0:col0+k_hi]."""
    _require_gpu(scores, kv_ok, rows, extra, index, keep)
    if scores.dtype != torch.float32 or scores.stride(-1) != 1:
        raise ValueError('scores must be fp32 with contiguous columns')
    if index.stride() != keep.stride() or index.stride(-1) != 1:
        raise ValueError('index and keep must share contiguous strides')
    if scores.shape[2] < block_start + n_cols:
        raise ValueError('scores has fewer columns than the block needs')
    _native.call('veda_select_topk', scores.data_ptr(), scores.shape[0], scores.shape[1],
                 scores.stride(0), scores.stride(1), block_start, n_cols, kv_ok.data_ptr(),
                 rows.data_ptr(), k_lo, k_hi, extra.data_ptr(), extra.numel(), index.data_ptr(),
                 keep.data_ptr(), index.stride(0), index.stride(1), col0, _stream(scores))


@torch.library.custom_op('veda::dense_block_mask', mutates_args=())
def dense_block_mask(index: torch.Tensor, keep: torch.Tensor, kv_ok: torch.Tensor,
                     n_video: int, global_rows: bool) -> torch.Tensor:
    _require_gpu(index, keep, kv_ok)
    heads, n_sel, k_total = index.shape
    n = kv_ok.numel()
    if global_rows and n_sel != n_video:
        raise ValueError('global_rows needs a selection of all video rows')
    mask = torch.empty(heads, n if global_rows else n_sel, n, dtype=torch.bool,
                       device=index.device)
    idx_c, keep_c = index.contiguous(), keep.contiguous()  # held until the launch
    _native.call('veda_dense_block_mask', idx_c.data_ptr(), keep_c.data_ptr(), heads, n_sel,
                 k_total, kv_ok.data_ptr(), n, n_video, int(global_rows), mask.data_ptr(),
                 _stream(index))
    return mask


@dense_block_mask.register_fake
def _(index, keep, kv_ok, n_video, global_rows):
    heads, n_sel, _ = index.shape
    n = kv_ok.numel()
    return index.new_empty(heads, n if global_rows else n_sel, n, dtype=torch.bool)


@torch.library.custom_op('veda::index_lists', mutates_args=())
def index_lists(block_mask: torch.Tensor, kv_ok: torch.Tensor,
                full_tile: torch.Tensor) -> list[torch.Tensor]:
    """-> [part_cnt, part_idx, full_cnt, full_idx], cnt [1, H', R] and idx
    [1, H', R, n] int32 (miowtion/kernels/fa4.py:275-296)."""
    _require_gpu(block_mask, kv_ok, full_tile)
    if block_mask.dtype != torch.bool or block_mask.dim() != 3:
        raise ValueError('block_mask must be bool [H\', R, n_tiles]')
    heads, rows, n = block_mask.shape
    if kv_ok.numel() != n or full_tile.numel() != n:
        raise ValueError('kv_ok / full_tile do not match the mask columns')
    bm = block_mask.contiguous()
    dev = block_mask.device
    pc = torch.empty(1, heads, rows, dtype=torch.int32, device=dev)
    fc = torch.empty(1, heads, rows, dtype=torch.int32, device=dev)
    pi = torch.empty(1, heads, rows, n, dtype=torch.int32, device=dev)
    fi = torch.empty(1, heads, rows, n, dtype=torch.int32, device=dev)
    _native.call('veda_index_lists', bm.data_ptr(), heads, rows, n, kv_ok.data_ptr(),
                 full_tile.data_ptr(), pc.data_ptr(), pi.data_ptr(), fc.data_ptr(),
                 fi.data_ptr(), _stream(block_mask))
    return [pc, pi, fc, fi]


@index_lists.register_fake
def _(block_mask, kv_ok, full_tile):
    h, r, n = block_mask.shape
    c = block_mask.new_empty(1, h, r, dtype=torch.int32)
    i = block_mask.new_empty(1, h, r, n, dtype=torch.int32)
    return [c, i, c.clone(), i.clone()]


# --------------------------------------------------------------------------
# attention (miowtion/kernels/fa4.py:299-377, miowtion/h3/attention.py:28-102)


@torch.library.custom_op('veda::block_sparse_fwd', mutates_args=())
def block_sparse_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     part_cnt: torch.Tensor, part_idx: torch.Tensor, full_cnt: torch.Tensor,
                     full_idx: torch.Tensor, valid_count: torch.Tensor,
                     return_lse: bool, front_tiles: int = 0) -> list[torch.Tensor]:
    """-> [out] or [out, lse [H', R*128]]; lists as returned by index_lists.
    front_tiles: the last query tiles of every head to dispatch first (the
    rows the mask makes dense); it changes the order only."""
    _require_gpu(q, k, v, part_cnt, part_idx, full_cnt, full_idx, valid_count)
    for name, t in (('q', q), ('k', k), ('v', v)):
        _check_rows(name, t)
    if q.shape[-1] != 128:
        raise ValueError('block_sparse_fwd supports head_dim 128')
    rq, heads, d = q.shape
    if rq % TILE or k.shape[0] % TILE or k.shape != v.shape or k.shape[1:] != q.shape[1:]:
        raise ValueError(f'bad shapes q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}')
    r_tiles, n_k = rq // TILE, k.shape[0] // TILE
    for name, t in (('part_idx', part_idx), ('full_idx', full_idx)):
        if t.dtype != torch.int32 or tuple(t.shape[:3]) != (1, heads, r_tiles) or not t.is_contiguous():
            raise ValueError(f'{name} must be contiguous int32 [1, {heads}, {r_tiles}, n]')
    for name, t in (('part_cnt', part_cnt), ('full_cnt', full_cnt)):
        if t.dtype != torch.int32 or t.numel() != heads * r_tiles or not t.is_contiguous():
            raise ValueError(f'{name} must be contiguous int32 [1, {heads}, {r_tiles}]')
    if part_idx.shape[3] != full_idx.shape[3] or part_idx.shape[3] < n_k:
        raise ValueError('list rows must hold at least n_k_tiles entries')
    if valid_count.numel() < n_k or valid_count.dtype != torch.int32:
        raise ValueError('valid_count must be int32 [n_k_tiles]')
    out = torch.empty_like(q, memory_format=torch.contiguous_format)
    lse = torch.empty(heads, rq, dtype=torch.float32, device=q.device) if return_lse else None
    _native.call('veda_block_sparse_fwd', q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
                 k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), heads, d,
                 r_tiles, n_k, full_cnt.data_ptr(), full_idx.data_ptr(), part_cnt.data_ptr(),
                 part_idx.data_ptr(), part_idx.shape[3], valid_count.data_ptr(),
                 1.0 / math.sqrt(d), out.data_ptr(), out.stride(0), out.stride(1), _p(lse),
                 rq, 1, front_tiles, _stream(q))
    return [out, lse] if return_lse else [out]


@block_sparse_fwd.register_fake
def _(q, k, v, part_cnt, part_idx, full_cnt, full_idx, valid_count, return_lse, front_tiles=0):
    out = torch.empty_like(q)
    if return_lse:
        return [out, q.new_empty(q.shape[1], q.shape[0], dtype=torch.float32)]
    return [out]


@torch.library.custom_op('veda::block_sparse_fwd_seq_', mutates_args=('out',))
def block_sparse_fwd_seq_(out: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          gather_index: torch.Tensor, scatter_index: torch.Tensor,
                          slot_valid: torch.Tensor, heads: torch.Tensor, part_cnt: torch.Tensor,
                          part_idx: torch.Tensor, full_cnt: torch.Tensor, full_idx: torch.Tensor,
                          valid_count: torch.Tensor, front_tiles: int = 0) -> None:
    """block_sparse_fwd with the permutation of q and out fused in: q [S, H,
    D] in sequence order is read through gather_index, and out [S + 1, H, D]
    receives the rows through scatter_index (what gather, block_sparse_fwd
    and scatter_ do in sequence). heads maps the H' heads of k / v / lists
    to heads of q and out."""
    _require_gpu(out, q, k, v, gather_index, scatter_index, slot_valid, heads, part_cnt,
                 part_idx, full_cnt, full_idx, valid_count)
    for name, t in (('out', out), ('q', q), ('k', k), ('v', v)):
        _check_rows(name, t)
    if q.shape[-1] != 128 or out.shape[1:] != q.shape[1:] or out.dtype != q.dtype:
        raise ValueError(f'q {tuple(q.shape)} and out {tuple(out.shape)} must be [*, H, 128] alike')
    n_slots = gather_index.numel()
    hp = heads.numel()
    if (n_slots % TILE or scatter_index.numel() != n_slots or slot_valid.numel() != n_slots
            or gather_index.dtype != torch.int64 or scatter_index.dtype != torch.int64
            or slot_valid.dtype != torch.int32 or heads.dtype != torch.int64):
        raise ValueError('gather_index / scatter_index int64 and slot_valid int32 of n_tiles * 128 '
                         'slots, heads int64')
    if k.shape != v.shape or k.shape[0] % TILE or k.shape[1] != hp or k.shape[2] != q.shape[2]:
        raise ValueError(f'k {tuple(k.shape)} / v {tuple(v.shape)} must be [n_k * 128, {hp}, 128]')
    r_tiles, n_k = n_slots // TILE, k.shape[0] // TILE
    _check_lists('part', part_cnt, part_idx, hp, r_tiles, n_k)
    _check_lists('full', full_cnt, full_idx, hp, r_tiles, n_k)
    if part_idx.shape[3] != full_idx.shape[3]:
        raise ValueError('part and full lists must have the same row length')
    if valid_count.numel() < n_k or valid_count.dtype != torch.int32:
        raise ValueError('valid_count must be int32 [n_k_tiles]')
    _native.call('veda_block_sparse_fwd_seq', q.data_ptr(), q.shape[0], q.shape[1], q.stride(0),
                 q.stride(1), gather_index.data_ptr(), scatter_index.data_ptr(),
                 slot_valid.data_ptr(), heads.data_ptr(), hp, k.data_ptr(), k.stride(0),
                 k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), q.shape[2], r_tiles, n_k,
                 full_cnt.data_ptr(), full_idx.data_ptr(), part_cnt.data_ptr(),
                 part_idx.data_ptr(), part_idx.shape[3], valid_count.data_ptr(),
                 1.0 / math.sqrt(q.shape[2]), out.data_ptr(), out.shape[0], out.stride(0),
                 out.stride(1), front_tiles, _stream(q))


@torch.library.custom_op('veda::block_sparse_fwd_seq_kv_', mutates_args=('out',))
def block_sparse_fwd_seq_kv_(out: torch.Tensor, q: torch.Tensor, k: torch.Tensor,
                             v: torch.Tensor, gather_index: torch.Tensor,
                             scatter_index: torch.Tensor, slot_valid: torch.Tensor,
                             heads: torch.Tensor, part_cnt: torch.Tensor, part_idx: torch.Tensor,
                             full_cnt: torch.Tensor, full_idx: torch.Tensor,
                             valid_count: torch.Tensor, front_tiles: int = 0) -> None:
    """block_sparse_fwd_seq_ with k and v in sequence order too: q, k, v
    [S, H, D] alike are read through gather_index (key tile row t is row
    gather_index[t]), out [S + 1, H, D] receives the rows through
    scatter_index. heads maps the H' heads of the lists to heads of q, k, v
    and out."""
    _require_gpu(out, q, k, v, gather_index, scatter_index, slot_valid, heads, part_cnt,
                 part_idx, full_cnt, full_idx, valid_count)
    for name, t in (('out', out), ('q', q), ('k', k), ('v', v)):
        _check_rows(name, t)
    if q.shape[-1] != 128 or out.shape[1:] != q.shape[1:] or out.dtype != q.dtype:
        raise ValueError(f'q {tuple(q.shape)} and out {tuple(out.shape)} must be [*, H, 128] alike')
    if k.shape != q.shape or v.shape != q.shape or k.stride() != q.stride() or v.stride() != q.stride():
        raise ValueError(f'k {tuple(k.shape)} / v {tuple(v.shape)} must be laid out as q '
                         f'{tuple(q.shape)}')
    n_slots = gather_index.numel()
    hp = heads.numel()
    if (n_slots % TILE or scatter_index.numel() != n_slots or slot_valid.numel() != n_slots
            or gather_index.dtype != torch.int64 or scatter_index.dtype != torch.int64
            or slot_valid.dtype != torch.int32 or heads.dtype != torch.int64):
        raise ValueError('gather_index / scatter_index int64 and slot_valid int32 of n_tiles * 128 '
                         'slots, heads int64')
    r_tiles = n_slots // TILE
    n_k = r_tiles
    _check_lists('part', part_cnt, part_idx, hp, r_tiles, n_k)
    _check_lists('full', full_cnt, full_idx, hp, r_tiles, n_k)
    if part_idx.shape[3] != full_idx.shape[3]:
        raise ValueError('part and full lists must have the same row length')
    if valid_count.numel() < n_k or valid_count.dtype != torch.int32:
        raise ValueError('valid_count must be int32 [n_k_tiles]')
    _native.call('veda_block_sparse_fwd_seq_kv', q.data_ptr(), k.data_ptr(), v.data_ptr(),
                 q.shape[0], q.shape[1], q.stride(0), q.stride(1), gather_index.data_ptr(),
                 scatter_index.data_ptr(), slot_valid.data_ptr(), heads.data_ptr(), hp,
                 q.shape[2], r_tiles, n_k, full_cnt.data_ptr(), full_idx.data_ptr(),
                 part_cnt.data_ptr(), part_idx.data_ptr(), part_idx.shape[3],
                 valid_count.data_ptr(), 1.0 / math.sqrt(q.shape[2]), out.data_ptr(),
                 out.shape[0], out.stride(0), out.stride(1), front_tiles, _stream(q))


def _check_lists(name: str, cnt: torch.Tensor, idx: torch.Tensor, heads: int, rows: int,
                 cols: int) -> None:
    if (idx.dtype != torch.int32 or idx.dim() != 4 or tuple(idx.shape[:3]) != (1, heads, rows)
            or idx.shape[3] < cols or not idx.is_contiguous()):
        raise ValueError(f'{name} index must be contiguous int32 [1, {heads}, {rows}, >= {cols}]')
    if cnt.dtype != torch.int32 or cnt.numel() != heads * rows or not cnt.is_contiguous():
        raise ValueError(f'{name} count must be contiguous int32 [1, {heads}, {rows}]')


@torch.library.custom_op('veda::block_sparse_bwd', mutates_args=())
def block_sparse_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
                     dout: torch.Tensor, lse: torch.Tensor, dlse: torch.Tensor | None,
                     part_cnt: torch.Tensor, part_idx: torch.Tensor, full_cnt: torch.Tensor,
                     full_idx: torch.Tensor, part_cnt_t: torch.Tensor, part_idx_t: torch.Tensor,
                     full_cnt_t: torch.Tensor, full_idx_t: torch.Tensor,
                     valid_count: torch.Tensor, front_tiles: int = 0) -> list[torch.Tensor]:
    """-> [dq, dk, dv] of block_sparse_fwd (fa4_sm8x/interface.py:2099
    _flash_attn_bwd with the Q-direction lists). lse: the forward's [H', R*128]
    fp32 LSE; dlse: its gradient or None; *_t: index_lists(transpose=True)."""
    _require_gpu(q, k, v, out, dout, lse, dlse, part_cnt, part_idx, full_cnt, full_idx,
                 part_cnt_t, part_idx_t, full_cnt_t, full_idx_t, valid_count)
    for name, t in (('q', q), ('k', k), ('v', v), ('out', out), ('dout', dout)):
        _check_rows(name, t)
    if q.shape[-1] != 128:
        raise ValueError('block_sparse_bwd supports head_dim 128')
    rq, heads, d = q.shape
    if (rq % TILE or k.shape[0] % TILE or k.shape != v.shape or k.shape[1:] != q.shape[1:]
            or out.shape != q.shape or dout.shape != q.shape):
        raise ValueError(f'bad shapes q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)} '
                         f'out {tuple(out.shape)} dout {tuple(dout.shape)}')
    r_tiles, n_k = rq // TILE, k.shape[0] // TILE
    for name, t in (('lse', lse), ('dlse', dlse)):
        if t is not None and (t.dtype != torch.float32 or tuple(t.shape) != (heads, rq)):
            raise ValueError(f'{name} must be fp32 [{heads}, {rq}]')
    _check_lists('part', part_cnt, part_idx, heads, r_tiles, n_k)
    _check_lists('full', full_cnt, full_idx, heads, r_tiles, n_k)
    _check_lists('transposed part', part_cnt_t, part_idx_t, heads, n_k, r_tiles)
    _check_lists('transposed full', full_cnt_t, full_idx_t, heads, n_k, r_tiles)
    if part_idx.shape[3] != full_idx.shape[3] or part_idx_t.shape[3] != full_idx_t.shape[3]:
        raise ValueError('the part and full lists of one direction must have equal rows')
    if valid_count.numel() < n_k or valid_count.dtype != torch.int32:
        raise ValueError('valid_count must be int32 [n_k_tiles]')
    dq = torch.empty_like(q, memory_format=torch.contiguous_format)
    dk = torch.empty_like(k, memory_format=torch.contiguous_format)
    dv = torch.empty_like(v, memory_format=torch.contiguous_format)
    work = torch.empty(max(heads * r_tiles * 512, 4), dtype=torch.float32, device=q.device)
    _native.call('veda_block_sparse_bwd', q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
                 k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1),
                 out.data_ptr(), out.stride(0), out.stride(1), dout.data_ptr(), dout.stride(0),
                 dout.stride(1), lse.data_ptr(), lse.stride(0), lse.stride(1), _p(dlse),
                 0 if dlse is None else dlse.stride(0), 0 if dlse is None else dlse.stride(1),
                 heads, d, r_tiles, n_k, full_cnt.data_ptr(), full_idx.data_ptr(),
                 part_cnt.data_ptr(), part_idx.data_ptr(), part_idx.shape[3],
                 full_cnt_t.data_ptr(), full_idx_t.data_ptr(), part_cnt_t.data_ptr(),
                 part_idx_t.data_ptr(), part_idx_t.shape[3], valid_count.data_ptr(),
                 1.0 / math.sqrt(d), dq.data_ptr(), dq.stride(0), dq.stride(1), dk.data_ptr(),
                 dk.stride(0), dk.stride(1), dv.data_ptr(), dv.stride(0), dv.stride(1),
                 work.data_ptr(), work.numel() * 4, front_tiles, _stream(q))
    return [dq, dk, dv]


@block_sparse_bwd.register_fake
def _(q, k, v, out, dout, lse, dlse, part_cnt, part_idx, full_cnt, full_idx, part_cnt_t,
      part_idx_t, full_cnt_t, full_idx_t, valid_count, front_tiles=0):
    return [torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)]


@torch.library.custom_op('veda::dense_fwd', mutates_args=())
def dense_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, used: int,
              return_lse: bool) -> list[torch.Tensor]:
    """Dense attention of rows [0, used) of packed [S, H, D]; -> [out] or
    [out, lse [S, H]] with 0 on rows [used, S)."""
    _require_gpu(q, k, v)
    for name, t in (('q', q), ('k', k), ('v', v)):
        _check_rows(name, t)
    if q.shape != k.shape or q.shape != v.shape or q.shape[-1] != 128:
        raise ValueError('dense_fwd needs equal [S, H, 128] q, k, v')
    s, heads, d = q.shape
    if not 0 <= used <= s:
        raise ValueError(f'used={used} outside [0, {s}]')
    out = torch.empty_like(q, memory_format=torch.contiguous_format)
    lse = torch.empty(s, heads, dtype=torch.float32, device=q.device) if return_lse else None
    _native.call('veda_dense_fwd', q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
                 k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1), s, used,
                 heads, d, 1.0 / math.sqrt(d), out.data_ptr(), out.stride(0), out.stride(1),
                 _p(lse), heads, 1, _stream(q))
    return [out, lse] if return_lse else [out]


@dense_fwd.register_fake
def _(q, k, v, used, return_lse):
    out = torch.empty_like(q)
    if return_lse:
        return [out, q.new_empty(q.shape[0], q.shape[1], dtype=torch.float32)]
    return [out]


# --------------------------------------------------------------------------
# teacher heat (miowtion/kernels/block_heat_triton.py:141-173)


@torch.library.custom_op('veda::block_heat', mutates_args=())
def block_heat(q: torch.Tensor, k: torch.Tensor, lse: torch.Tensor, valid_count: torch.Tensor,
               q_tiles: torch.Tensor, reduce: str) -> torch.Tensor:
    """[H', R, n_tiles] fp32 block heat; the real rows of tile t are its first
    valid_count[t] slots (the tile layout's prefix rule)."""
    _require_gpu(q, k, lse, valid_count, q_tiles)
    if reduce not in ('max', 'sum'):
        raise ValueError(f"reduce must be 'max' or 'sum': {reduce!r}")
    _check_rows('q', q)
    _check_rows('k', k)
    if q.shape[-1] != 128 or k.shape != q.shape:
        raise ValueError('heat kernel needs equal [N, H\', 128] q and k')
    if lse.dtype != torch.float32 or tuple(lse.shape) != tuple(q.shape[:2]):
        raise ValueError('lse must be fp32 [N, H\']')
    n_slots, heads, d = q.shape
    n_tiles = n_slots // TILE
    if valid_count.numel() != n_tiles or valid_count.dtype != torch.int32:
        raise ValueError(f'valid_count must be int32 [{n_tiles}]')
    qt = q_tiles.to(torch.int64).contiguous()
    heat = torch.empty(heads, qt.numel(), n_tiles, dtype=torch.float32, device=q.device)
    _native.call('veda_block_heat', q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
                 k.stride(0), k.stride(1), lse.data_ptr(), lse.stride(0), lse.stride(1),
                 valid_count.contiguous().data_ptr(), qt.data_ptr(), qt.numel(), n_tiles, heads, d,
                 1 if reduce == 'max' else 0, 1.0 / math.sqrt(d), heat.data_ptr(), _stream(q))
    return heat


@block_heat.register_fake
def _(q, k, lse, slot_valid, q_tiles, reduce):
    return q.new_empty(q.shape[1], q_tiles.numel(), q.shape[0] // TILE, dtype=torch.float32)


# Teacher dense pass in tile order with the heat statistics
# (miowtion/veda/attention.py:549-588, the fused form of
# docs/features/veda_kernel.md:285-289).

# Workspace bound of the per-(key tile, query row) statistics: heads are
# processed in chunks whose workspace stays below this.
HEAT_WORKSPACE_BYTES = 4 * 2 ** 30


@torch.library.custom_op('veda::dense_heat', mutates_args=())
def dense_heat(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor | None,
               valid_count: torch.Tensor, q_tiles: torch.Tensor, reduce: str,
               workspace_bytes: int = HEAT_WORKSPACE_BYTES) -> list[torch.Tensor]:
    """Dense attention of the query tiles `q_tiles` over every valid key of a
    tile layout, in one pass that also yields the block heat.

    q, k (and v): tile-ordered [N, H', 128] bf16; q_tiles: [R] tile ids.
    Returns [heat [H', R, n] fp32, lse [H', R*128] fp32 (natural log)] and,
    when v is given, out [R*128, H', 128] bf16 as a third entry.
    """
    _require_gpu(q, k, v, valid_count, q_tiles)
    if reduce not in ('max', 'sum'):
        raise ValueError(f"reduce must be 'max' or 'sum': {reduce!r}")
    _check_rows('q', q)
    _check_rows('k', k)
    if v is not None:
        _check_rows('v', v)
        if v.shape != k.shape:
            raise ValueError('v must match k')
    if q.shape[-1] != 128 or k.shape != q.shape:
        raise ValueError("dense_heat needs equal [N, H', 128] q and k")
    n_slots, heads, d = q.shape
    if n_slots % TILE:
        raise ValueError(f'{n_slots} rows is not a whole number of {TILE}-row tiles')
    n_tiles = n_slots // TILE
    if valid_count.numel() != n_tiles or valid_count.dtype != torch.int32:
        raise ValueError(f'valid_count must be int32 [{n_tiles}]')
    qt = q_tiles.to(torch.int64).contiguous()
    n_items = qt.numel()
    if n_items and (int(qt.min()) < 0 or int(qt.max()) >= n_tiles):
        raise ValueError(f'q_tiles outside [0, {n_tiles})')
    heat = torch.empty(heads, n_items, n_tiles, dtype=torch.float32, device=q.device)
    lse = torch.empty(heads, n_items * TILE, dtype=torch.float32, device=q.device)
    out = None if v is None else q.new_empty(n_items * TILE, heads, d)
    per_head = n_tiles * n_items * TILE * 4
    chunk = max(1, min(heads, workspace_bytes // max(per_head, 1)))
    part = torch.empty(chunk * per_head // 4, dtype=torch.float32, device=q.device)
    vc = valid_count.contiguous()
    for h0 in range(0, heads, chunk):
        h1 = min(heads, h0 + chunk)
        qh, kh = q[:, h0:h1], k[:, h0:h1]
        vh = None if v is None else v[:, h0:h1]
        oh = None if out is None else out[:, h0:h1]
        _native.call('veda_dense_heat_fwd', qh.data_ptr(), qh.stride(0), qh.stride(1), n_tiles,
                     kh.data_ptr(), kh.stride(0), kh.stride(1), _p(vh),
                     0 if vh is None else vh.stride(0), 0 if vh is None else vh.stride(1),
                     h1 - h0, d, qt.data_ptr(), n_items, n_tiles, vc.data_ptr(),
                     1.0 / math.sqrt(d), 1 if reduce == 'max' else 0, _p(oh),
                     0 if oh is None else oh.stride(0), 0 if oh is None else oh.stride(1),
                     lse[h0:h1].data_ptr(), lse.stride(0), lse.stride(1), part.data_ptr(),
                     _stream(q))
        _native.call('veda_heat_combine', part.data_ptr(), lse[h0:h1].data_ptr(), lse.stride(0),
                     lse.stride(1), vc.data_ptr(), qt.data_ptr(), n_items, n_tiles, h1 - h0,
                     1 if reduce == 'max' else 0, heat[h0:h1].data_ptr(), _stream(q))
    return [heat, lse] if out is None else [heat, lse, out]


@dense_heat.register_fake
def _(q, k, v, valid_count, q_tiles, reduce, workspace_bytes=HEAT_WORKSPACE_BYTES):
    n = q.shape[0] // TILE
    res = [q.new_empty(q.shape[1], q_tiles.numel(), n, dtype=torch.float32),
           q.new_empty(q.shape[1], q_tiles.numel() * TILE, dtype=torch.float32)]
    if v is not None:
        res.append(q.new_empty(q_tiles.numel() * TILE, q.shape[1], q.shape[2]))
    return res


# Zero-order compensation (miowtion/veda/attention.py:591-689,
# miowtion/kernels/compensation_triton.py:80-258)


@torch.library.custom_op('veda::tile_summaries', mutates_args=())
def tile_summaries(k: torch.Tensor, v: torch.Tensor, valid_count: torch.Tensor) -> list[torch.Tensor]:
    """[kc, vc], both [n, H', D] bf16: mean of K and sum of V over each key
    tile's real rows (compensation_triton.py:80-99)."""
    _require_gpu(k, v, valid_count)
    _check_rows('k', k)
    _check_rows('v', v)
    if k.shape != v.shape or k.shape[-1] != 128 or k.shape[0] % TILE:
        raise ValueError("tile_summaries needs equal [n * 128, H', 128] k and v")
    n = k.shape[0] // TILE
    if valid_count.numel() != n or valid_count.dtype != torch.int32:
        raise ValueError(f'valid_count must be int32 [{n}]')
    kc = k.new_empty(n, k.shape[1], k.shape[2])
    vc = torch.empty_like(kc)
    _native.call('veda_tile_summaries', k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(),
                 v.stride(0), v.stride(1), valid_count.contiguous().data_ptr(), n, k.shape[1],
                 k.shape[2], kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
                 _stream(k))
    return [kc, vc]


@tile_summaries.register_fake
def _(k, v, valid_count):
    kc = k.new_empty(k.shape[0] // TILE, k.shape[1], k.shape[2])
    return [kc, torch.empty_like(kc)]


@torch.library.custom_op('veda::zero_order_compensation', mutates_args=())
def zero_order_compensation(o_kept: torch.Tensor, lse_kept: torch.Tensor, q: torch.Tensor,
                            kc: torch.Tensor, vc: torch.Tensor, block_mask: torch.Tensor,
                            valid_count: torch.Tensor) -> torch.Tensor:
    """(o_kept + sum over dropped tiles of p vc) / (1 + sum of p B), p =
    exp(q . kc / sqrt(D) - lse_kept); shapes as the reference's compensate()."""
    _require_gpu(o_kept, lse_kept, q, kc, vc, block_mask, valid_count)
    for name, t in (('o_kept', o_kept), ('q', q), ('kc', kc), ('vc', vc)):
        _check_rows(name, t)
    rows, heads, d = o_kept.shape
    if q.shape != o_kept.shape or d != 128 or rows % TILE:
        raise ValueError(f'q is {tuple(q.shape)}, o_kept {tuple(o_kept.shape)}; need equal '
                         "[R * 128, H', 128]")
    n = kc.shape[0]
    if vc.shape != kc.shape or kc.shape[1:] != (heads, d):
        raise ValueError(f"kc / vc must be [n, {heads}, {d}]")
    if lse_kept.dtype != torch.float32 or tuple(lse_kept.shape) != (heads, rows):
        raise ValueError(f'lse_kept must be fp32 [{heads}, {rows}]')
    if block_mask.dtype != torch.bool or tuple(block_mask.shape) != (heads, rows // TILE, n):
        raise ValueError(f'block_mask must be bool [{heads}, {rows // TILE}, {n}]')
    if valid_count.numel() != n or valid_count.dtype != torch.int32:
        raise ValueError(f'valid_count must be int32 [{n}]')
    out = torch.empty_like(o_kept, memory_format=torch.contiguous_format)
    keep = block_mask.contiguous()
    _native.call('veda_zero_order_compensation', o_kept.data_ptr(), o_kept.stride(0),
                 o_kept.stride(1), lse_kept.data_ptr(), lse_kept.stride(0), lse_kept.stride(1),
                 q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(),
                 kc.stride(0), kc.stride(1), keep.data_ptr(), valid_count.contiguous().data_ptr(),
                 heads, d, rows // TILE, n, 1.0 / math.sqrt(d), out.data_ptr(), out.stride(0),
                 out.stride(1), _stream(q))
    return out


@zero_order_compensation.register_fake
def _(o_kept, lse_kept, q, kc, vc, block_mask, valid_count):
    return torch.empty_like(o_kept)


@torch.library.custom_op('veda::compensated_attention', mutates_args=())
def compensated_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          part_cnt: torch.Tensor, part_idx: torch.Tensor, full_cnt: torch.Tensor,
                          full_idx: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor,
                          block_mask: torch.Tensor, valid_count: torch.Tensor,
                          front_tiles: int = 0) -> torch.Tensor:
    """Block-sparse attention over the listed (kept) blocks plus the
    zero-order term of every other non-empty key tile, in one pass
    (compensation_triton.attention, :228-258). Lists as index_lists returns
    them for block_mask (the kept blocks, kv_ok applied); kc / vc the tile
    summaries."""
    _require_gpu(q, k, v, part_cnt, part_idx, full_cnt, full_idx, kc, vc, block_mask,
                 valid_count)
    for name, t in (('q', q), ('k', k), ('v', v), ('kc', kc), ('vc', vc)):
        _check_rows(name, t)
    rq, heads, d = q.shape
    if (d != 128 or rq % TILE or k.shape[0] % TILE or k.shape != v.shape
            or k.shape[1:] != q.shape[1:]):
        raise ValueError(f'bad shapes q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}')
    r_tiles, n = rq // TILE, k.shape[0] // TILE
    _check_lists('part', part_cnt, part_idx, heads, r_tiles, n)
    _check_lists('full', full_cnt, full_idx, heads, r_tiles, n)
    if part_idx.shape[3] != full_idx.shape[3]:
        raise ValueError('the part and full lists must have equal rows')
    if vc.shape != kc.shape or tuple(kc.shape) != (n, heads, d):
        raise ValueError(f"kc / vc must be [{n}, {heads}, {d}]")
    if block_mask.dtype != torch.bool or tuple(block_mask.shape) != (heads, r_tiles, n):
        raise ValueError(f'block_mask must be bool [{heads}, {r_tiles}, {n}]')
    if valid_count.numel() != n or valid_count.dtype != torch.int32:
        raise ValueError(f'valid_count must be int32 [{n}]')
    out = torch.empty_like(q, memory_format=torch.contiguous_format)
    keep = block_mask.contiguous()
    _native.call('veda_compensated_attention', q.data_ptr(), q.stride(0), q.stride(1),
                 k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1),
                 heads, d, r_tiles, n, full_cnt.data_ptr(), full_idx.data_ptr(),
                 part_cnt.data_ptr(), part_idx.data_ptr(), part_idx.shape[3], kc.data_ptr(),
                 vc.data_ptr(), kc.stride(0), kc.stride(1), keep.data_ptr(),
                 valid_count.contiguous().data_ptr(), 1.0 / math.sqrt(d), out.data_ptr(),
                 out.stride(0), out.stride(1), front_tiles, _stream(q))
    return out


@compensated_attention.register_fake
def _(q, k, v, part_cnt, part_idx, full_cnt, full_idx, kc, vc, block_mask, valid_count,
      front_tiles=0):
    return torch.empty_like(q)


# --------------------------------------------------------------------------
# predictor (miowtion/veda/predictor.py:251-338)

W_BF16, W_FP32, W_E4M3 = 0, 1, 2


@torch.library.custom_op('veda::predictor_embed', mutates_args=())
def predictor_embed(feats: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor | None,
                    heads: torch.Tensor, residual: bool) -> torch.Tensor:
    _require_gpu(feats, weight, weight_scale, heads)
    if feats.dtype != torch.float32 or feats.dim() != 3:
        raise ValueError('feats must be fp32 [H\', n, K]')
    hp, n, kd = feats.shape
    if weight.dim() != 3 or weight.shape[1] != kd:
        raise ValueError(f'weight {tuple(weight.shape)} does not take {kd} features')
    n_out = weight.shape[2]
    if residual and kd < n_out:
        raise ValueError('residual needs at least n_out features')
    if weight.dtype == torch.bfloat16:
        wd = W_BF16
    elif weight.dtype == torch.float32:
        wd = W_FP32
    elif weight.dtype == torch.float8_e4m3fn:
        wd = W_E4M3
        if weight_scale is None or weight_scale.numel() != weight.shape[0]:
            raise ValueError('e4m3 weights need a per-head fp32 scale')
    else:
        raise ValueError(f'unsupported weight dtype {weight.dtype}')
    f = feats.contiguous()
    w = weight.contiguous()
    out = torch.empty(hp, n, n_out, dtype=torch.float32, device=feats.device)
    _native.call('veda_predictor_embed', f.data_ptr(), hp, n, kd, w.data_ptr(), wd,
                 _p(weight_scale), weight.shape[0], heads.data_ptr(), n_out, int(residual),
                 out.data_ptr(), _stream(feats))
    return out


@predictor_embed.register_fake
def _(feats, weight, weight_scale, heads, residual):
    return feats.new_empty(feats.shape[0], feats.shape[1], weight.shape[2])


@torch.library.custom_op('veda::predictor_logits', mutates_args=())
def predictor_logits(a: torch.Tensor, b: torch.Tensor, scale: float, gain: torch.Tensor | None,
                     heads: torch.Tensor | None, log_count: torch.Tensor | None,
                     base: torch.Tensor | None) -> torch.Tensor:
    """scale * a b^T (+ gain[heads] log_count) (+ base), fp32 [H', n_q, n_k]."""
    _require_gpu(a, b, gain, heads, log_count, base)
    if a.dtype != torch.float32 or b.dtype != torch.float32 or a.dim() != 3 or b.dim() != 3:
        raise ValueError('a and b must be fp32 [H\', n, dim]')
    hp, nq, dim = a.shape
    nk = b.shape[1]
    if b.shape[0] != hp or b.shape[2] != dim:
        raise ValueError('a and b disagree in heads or dim')
    if base is not None:
        out = base.contiguous().clone()
    else:
        out = torch.empty(hp, nq, nk, dtype=torch.float32, device=a.device)
    a_c, b_c = a.contiguous(), b.contiguous()  # held until the launch
    _native.call('veda_predictor_logits', a_c.data_ptr(), b_c.data_ptr(), hp, nq, nk, dim,
                 scale, _p(gain), _p(heads), _p(log_count), int(base is not None),
                 out.data_ptr(), _stream(a))
    return out


@predictor_logits.register_fake
def _(a, b, scale, gain, heads, log_count, base):
    return a.new_empty(a.shape[0], a.shape[1], b.shape[1])
