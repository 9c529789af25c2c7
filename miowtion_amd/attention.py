"""Veda attention plug-ins with the reference's `AttentionFn` signature
`(q, k, v, layer_index) -> out` (`miowtion/h3/model.py:40-45`): q, k, v are
[S, H, D] bf16 (post norm / RoPE), rows [used, S) padding; out is [S, H, D]
bf16 with padding rows zero.

  SparseStudent  (miowtion/veda/attention.py:692-794): gather + pool q/k,
                 gather v, predictor logits, top-k, block mask, block-sparse
                 attention, scatter -- all HIP kernels.
  OracleStudent  (miowtion/veda/attention.py:478-588): the teacher's LSE and
                 block heat (one fused QK pass in tile order by default;
                 dense attention + heat kernel with fused=False), top-k on
                 heat, block-sparse attention.
  DenseAttention (miowtion/h3/model.py:48-58): the dense kernel.

Heads are processed per plan head group (<= 2 shapes per layer) and in
chunks bounded by `collect_bytes` (attention.py:204-206); heads are
independent, so chunking never changes a value.
"""

from __future__ import annotations

import dataclasses

import torch

from miowtion_amd import kernels
from miowtion_amd import mask as veda_mask
from miowtion_amd import plan as veda_plan
from miowtion_amd import predictor as veda_predictor
from miowtion_amd import tiling

# One tile-ordered bf16 copy of a head group is bounded by this (the
# reference's 256 MiB default targets 24 GB cards; 288 GB of HBM holds a whole
# 48-head group at C2 -- 931 MB -- comfortably, so the default runs every
# group in one launch).
DEFAULT_COLLECT_BYTES = 8 * 2 ** 30

ORACLE_TARGETS = ('mass', 'max', 'mean')


@dataclasses.dataclass(frozen=True)
class VedaConfig:
    """Sparsity settings (the hot-path subset of attention.py:37-135)."""

    target_budget: veda_mask.Budget = veda_mask.Budget(ratio=0.1)
    ref_budget: veda_mask.Budget | None = None
    tile_conditions: bool = False
    contiguous_tiles: bool = False
    dense_layers: frozenset = frozenset()
    collect_bytes: int = DEFAULT_COLLECT_BYTES
    # Zero-order compensation of the dropped tiles (attention.py:70-93).
    # zero_order_compensation (torch form) and triton_compensation (the
    # kernel form with bf16 tile summaries) are the same arithmetic and both
    # run the `veda::zero_order_compensation` HIP kernel here;
    # fused_compensation is the Sol INT8 kernel, which this build does not
    # have (refused, not replaced).
    zero_order_compensation: bool = False
    triton_compensation: bool = False
    fused_compensation: bool = False

    def __post_init__(self):
        chosen = [n for n in ('zero_order_compensation', 'fused_compensation',
                              'triton_compensation') if getattr(self, n)]
        if len(chosen) > 1:
            raise ValueError(f'at most one compensation arm may be set, got {chosen}')
        if self.fused_compensation:
            raise NotImplementedError('fused_compensation (the Sol INT8 kernel) is not part of '
                                      'this build; zero_order_compensation computes the same '
                                      'term around the block-sparse kernel')


@dataclasses.dataclass(frozen=True)
class VideoSpan:
    start: int
    grid: tuple[int, int, int]


@dataclasses.dataclass(frozen=True)
class PackedLayout:
    """What the attention path reads of `miowtion/h3/layout.py:PackedLayout`:
    the video spans in packed order (target last), real rows and length."""

    spans: tuple[VideoSpan, ...]
    used: int
    seq_len: int

    @property
    def target(self) -> VideoSpan:
        return self.spans[-1]


class ClipTiling:
    """Tile layouts of one clip, one per target shape (attention.py:138-197)."""

    def __init__(self, layout: PackedLayout, config: VedaConfig, device,
                 condition_spans: tuple[tiling.TiledSpan, ...] = ()):
        self.layout = layout
        self.config = config
        self.device = torch.device(device)
        spans = list(condition_spans)
        if config.tile_conditions:
            spans += [tiling.TiledSpan(s.start, s.grid, tiling.least_padding_shape(s.grid))
                      for s in layout.spans[:-1]]
        self._condition_spans = sorted(spans, key=lambda s: s.start)
        self._cache: dict = {}

    def get(self, shape: tiling.TileShape) -> tiling.TileLayout:
        if shape not in self._cache:
            target = self.layout.target
            spans = self._condition_spans + [tiling.TiledSpan(target.start, target.grid, shape)]
            tiler = tiling.contiguous_span_tiles if self.config.contiguous_tiles else tiling.span_tiles
            self._cache[shape] = tiling.build_tile_layout(
                spans, self.layout.used, self.layout.seq_len, self.device, tiler=tiler)
        return self._cache[shape]

    def blocks(self, tile_layout: tiling.TileLayout) -> list[veda_mask.ColumnBlock]:
        return veda_mask.column_blocks(tile_layout, self.config.target_budget,
                                       self.config.ref_budget)


_HEAD_DIM_BYTES = 128 * 2


def _seq_kv_ok(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    """Whether the attention kernel can read k and v in sequence order: laid
    out as q, and every row within a 32-bit load offset of its head's first
    row."""
    return (k.shape == q.shape and v.shape == q.shape and k.stride() == q.stride()
            and v.stride() == q.stride() and k.dtype == q.dtype and v.dtype == q.dtype
            and (q.shape[0] - 1) * q.stride(0) * 2 + 2 * q.shape[2] < 1 << 32)


def _chunk_heads(tile_layout: tiling.TileLayout, collect_bytes: int) -> int:
    """Heads per chunk so one tile-ordered copy stays under collect_bytes."""
    return max(1, collect_bytes // (tile_layout.num_slots * _HEAD_DIM_BYTES))


def _require_kernels(device: torch.device, who: str) -> None:
    if device.type != 'cuda':
        raise RuntimeError(f'{who} needs the HIP block-sparse kernels on a GPU, not {device}; '
                           'refusing to fall back silently')
    from miowtion_amd import _native
    _native.load()


class DenseAttention:
    """Dense attention over the real rows (h3/model.py:48-58)."""

    def __init__(self, used: int):
        self.used = used

    def __call__(self, q, k, v, layer_index: int) -> torch.Tensor:
        return kernels.dense_attention(q, k, v, self.used)[0]


class SparseStudent:
    """Predictor-masked block sparsity (attention.py:692-794)."""

    def __init__(self, clip: ClipTiling, plan: veda_plan.TilePlan,
                 predictor: veda_predictor.TileScorePredictor):
        _require_kernels(clip.device, 'SparseStudent')
        self.clip = clip
        self.plan = plan
        self.predictor = predictor
        self.calls = {'sparse': 0, 'dense': 0}
        # Per-call diagnostics of the last layer (selection and lists), kept
        # on the device for the parity tests and the bench.
        self.last: dict = {}

    def __call__(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                 layer_index: int) -> torch.Tensor:
        used = self.clip.layout.used
        if layer_index in self.clip.config.dense_layers:
            self.calls['dense'] += 1
            return kernels.dense_attention(q, k, v, used)[0]
        self.calls['sparse'] += 1
        seq_len = q.shape[0]
        groups = self.plan.head_groups(layer_index, self.clip.device)
        # The reference zero-fills the [S + 1, H, D] buffer (attention.py:732).
        # When the plan's groups hold every head, every (real row, head) is
        # written below (each real row is one valid slot of every layout), so
        # only rows [used, S] need the zeros; the result is the same.
        out = self._output_buffer(q, seq_len + 1)
        if sum(g.heads.numel() for g in groups) == q.shape[1]:
            out[used:].zero_()
        else:
            out.zero_()
        self.last = {}
        for group in groups:
            tile_layout = self.clip.get(group.shape)
            for heads in group.heads.split(_chunk_heads(tile_layout, self.clip.config.collect_bytes)):
                self._attend(q, k, v, layer_index, tile_layout, heads, out)
        out = out[:seq_len]
        if used < seq_len:
            out[used:] = 0
        return out

    def _output_buffer(self, q: torch.Tensor, rows: int) -> torch.Tensor:
        """The [rows, H, D] scatter buffer, uninitialised (every row the
        layer does not write is zeroed by the caller)."""
        return q.new_empty(rows, *q.shape[1:])

    def _attend(self, q, k, v, layer_index: int, tile_layout: tiling.TileLayout,
                heads: torch.Tensor, out: torch.Tensor) -> None:
        pred = self.predictor
        want = pred.second_order_rank
        cfg = self.clip.config
        compensated = cfg.zero_order_compensation or cfg.triton_compensation
        # Without compensation the attention kernel reads q in sequence order
        # and scatters its rows itself, so q is only pooled, not permuted;
        # when k and v are laid out as q it gathers their key tiles itself
        # too, so they are only pooled (k) or not touched (v) here.
        q_tiles = None
        if compensated:
            q_res = kernels.gather_and_pool(q, tile_layout, heads, second=bool(want))
            q_tiles, q_res = q_res[0], q_res[1:]
        else:
            q_res = kernels.pool_seq(q, tile_layout, heads, second=bool(want))
        kv_seq = not compensated and _seq_kv_ok(q, k, v)
        k_tiles = v_tiles = None
        if want:
            feats_q, sq_q, _ = q_res
            if kv_seq:
                feats_k, _, var_k = kernels.pool_seq(k, tile_layout, heads, second=True)
            else:
                k_tiles, feats_k, _, var_k = kernels.gather_and_pool(k, tile_layout, heads,
                                                                     second=True)
        else:
            (feats_q,) = q_res
            if kv_seq:
                (feats_k,) = kernels.pool_seq(k, tile_layout, heads)
            else:
                k_tiles, feats_k = kernels.gather_and_pool(k, tile_layout, heads)
            sq_q = var_k = None
        if not kv_seq:
            v_tiles = kernels.gather_tiles(v, tile_layout, heads)
        with torch.no_grad():
            extra = {}
            if pred.count_term:
                extra['log_count'] = veda_predictor.log_count(tile_layout)
            if want:
                extra['sq_q'], extra['var_k'] = sq_q, var_k
            logits = pred.layers[layer_index](feats_q, feats_k, heads, **extra)
            selection = veda_mask.select_video_blocks(
                logits[:, :tile_layout.n_video_tiles], tile_layout, self.clip.blocks(tile_layout))
            block_mask = veda_mask.dense_block_mask(selection, tile_layout)
            lists = kernels.index_lists(block_mask, tile_layout)
            if compensated:
                # the lists already hold only kv_ok tiles (index_lists applies it)
                o_tiles = kernels.compensated_attention(q_tiles, k_tiles, v_tiles, block_mask,
                                                        tile_layout, lists)
                kernels.scatter_tiles_(out, o_tiles, tile_layout, heads)
            elif kv_seq:
                kernels.block_sparse_attention_seq_kv_(out, q, k, v, lists, tile_layout, heads)
            else:
                kernels.block_sparse_attention_seq_(out, q, k_tiles, v_tiles, lists, tile_layout,
                                                    heads)
        self.last.setdefault('parts', []).append(
            dict(shape=tile_layout, heads=heads, selection=selection, lists=lists,
                 logits=logits))


class OracleStudent:
    """Block sparsity masked by the true block statistic (attention.py:478-588).

    The reference runs dense attention for its LSE only (its output is
    discarded, attention.py:549-553) and then recomputes QK^T for the heat.
    With `fused` (the default) one pass over the tile-ordered q / k gives
    both: the LSE and a per-(key tile, row) statistic that an HBM-bound
    kernel turns into the heat (the fusion docs/features/veda_kernel.md:
    285-289 plans). `fused=False` keeps the reference's two passes.
    """

    def __init__(self, clip: ClipTiling, plan: veda_plan.TilePlan, target: str = 'mass',
                 fused: bool = True):
        if target not in ORACLE_TARGETS:
            raise ValueError(f'target must be one of {ORACLE_TARGETS}: {target!r}')
        _require_kernels(clip.device, 'OracleStudent')
        self.clip = clip
        self.plan = plan
        self.target = target
        self.fused = fused
        self.calls = {'sparse': 0, 'dense': 0}
        self.last: dict = {}

    def __call__(self, q, k, v, layer_index: int) -> torch.Tensor:
        used = self.clip.layout.used
        if layer_index in self.clip.config.dense_layers:
            self.calls['dense'] += 1
            return kernels.dense_attention(q, k, v, used)[0]
        self.calls['sparse'] += 1
        lse = None
        if not self.fused:
            with torch.no_grad():
                _, lse = kernels.dense_attention(q, k, v, used, return_lse=True)
        seq_len = q.shape[0]
        out = q.new_zeros(seq_len + 1, *q.shape[1:])
        self.last = {'lse': lse}
        for group in self.plan.head_groups(layer_index, self.clip.device):
            tile_layout = self.clip.get(group.shape)
            for heads in group.heads.split(_chunk_heads(tile_layout, self.clip.config.collect_bytes)):
                self._attend(q, k, v, lse, tile_layout, heads, out)
        out = out[:seq_len]
        if used < seq_len:
            out[used:] = 0
        return out

    def _attend(self, q, k, v, lse, tile_layout: tiling.TileLayout, heads, out) -> None:
        q_tiles = kernels.gather_tiles(q, tile_layout, heads)
        k_tiles = kernels.gather_tiles(k, tile_layout, heads)
        v_tiles = kernels.gather_tiles(v, tile_layout, heads)
        rows = torch.arange(tile_layout.n_video_tiles, device=q.device)
        with torch.no_grad():
            reduce = 'max' if self.target == 'max' else 'sum'
            lse_tiles = None
            if self.fused:
                heat, lse_tiles, _ = kernels.dense_heat(q_tiles, k_tiles, tile_layout, rows, reduce)
            else:
                heat = kernels.teacher_heat(q_tiles, k_tiles,
                                            kernels.gather_lse(lse, tile_layout, heads),
                                            tile_layout, rows, reduce)
            if self.target == 'mean':
                counts = tile_layout.valid_count.clamp(min=1).to(heat.dtype)
                heat = heat / counts[None, None, :]
            selection = veda_mask.select_video_blocks(
                heat[:, :, :tile_layout.n_video_tiles], tile_layout, self.clip.blocks(tile_layout),
                rows)
            block_mask = veda_mask.dense_block_mask(selection, tile_layout)
            o_tiles = kernels.block_sparse_attention(q_tiles, k_tiles, v_tiles, block_mask,
                                                     tile_layout)
        kernels.scatter_tiles_(out, o_tiles, tile_layout, heads)
        self.last.setdefault('parts', []).append(
            dict(shape=tile_layout, heads=heads, heat=heat, selection=selection,
                 lse_tiles=lse_tiles))
