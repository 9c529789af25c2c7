"""Tile-score predictor on the GPU: pooled [mean | max | min] features ->
per-head residual projection -> fp32 block logits.

Host mirror of `miowtion/veda/predictor.py` (LayerPredictor :197-338,
TileScorePredictor :341-410). Pooling is the fused gather kernel
(`kernels.gather_and_pool` / `kernels.pool_tiles`); the projection and the
(q-tile, k-tile) scores are the `veda::predictor_embed` and
`veda::predictor_logits` HIP kernels. Weights may be held as bf16 / fp32, or
as fp8 e4m3 with a per-head fp32 scale (the bundle format of
`miowtion/veda/bundle.py:71-93`), decoded inside the kernel to the same bf16
value the reference keeps resident.
"""

from __future__ import annotations

import math

import torch

from miowtion_amd import kernels
from miowtion_amd import ops
from miowtion_amd import tiling

INIT_STD = 1e-4
SECOND_RAW = kernels.SECOND_RAW
SECOND_CENTRAL = kernels.SECOND_CENTRAL
E4M3_MAX = 448.0


def pool_tiles(x: torch.Tensor, layout: tiling.TileLayout, second: str | None = None) -> torch.Tensor:
    """Masked mean / max / min of every tile of tile-ordered rows
    (predictor.py:82-130); the fused HIP pooling."""
    return kernels.pool_tiles(x, layout, second)


class ProjWeight:
    """One [H, K, N] projection: plain tensor, or e4m3 values + per-head scale."""

    def __init__(self, values: torch.Tensor, scale: torch.Tensor | None = None):
        if values.dtype == torch.float8_e4m3fn and scale is None:
            raise ValueError('e4m3 weights need their per-head scale')
        self.values = values.contiguous()
        self.scale = None if scale is None else scale.float().contiguous()

    @classmethod
    def quantize_fp8(cls, weight: torch.Tensor) -> 'ProjWeight':
        """Per-head amax onto 448 (bundle.py:71-86); done once at load."""
        dims = tuple(range(1, weight.dim()))
        amax = weight.float().abs().amax(dim=dims)
        scale = (amax / E4M3_MAX).clamp(min=torch.finfo(torch.float32).tiny)
        vals = weight.float() / scale.view(-1, *([1] * len(dims)))
        return cls(vals.to(torch.float8_e4m3fn), scale)

    def to(self, device) -> 'ProjWeight':
        return ProjWeight(self.values.to(device),
                          None if self.scale is None else self.scale.to(device))

    @property
    def shape(self):
        return self.values.shape


class LayerPredictor:
    """Projections of one layer: proj_q, proj_k [num_heads, 3D, D]; with
    second_order_rank > 0 also so_q, so_k [num_heads, D, rank]; with
    count_term a gain [num_heads] on log B_j (predictor.py:197-229)."""

    def __init__(self, proj_q: ProjWeight, proj_k: ProjWeight, so_q: ProjWeight | None = None,
                 so_k: ProjWeight | None = None, count_gain: torch.Tensor | None = None):
        self.proj_q, self.proj_k = proj_q, proj_k
        self.so_q, self.so_k = so_q, so_k
        self.count_gain = None if count_gain is None else count_gain.float().contiguous()
        self.head_dim = proj_q.shape[-1]
        self.second_order_rank = 0 if so_q is None else so_q.shape[-1]

    @classmethod
    def random(cls, num_heads: int, head_dim: int, std: float = INIT_STD,
               generator: torch.Generator | None = None, device='cpu',
               second_order_rank: int = 0, count_term: bool = False,
               fp8: bool = False) -> 'LayerPredictor':
        def w(*shape):
            t = torch.randn(*shape, generator=generator) * std
            return (ProjWeight.quantize_fp8(t) if fp8 else ProjWeight(t.to(torch.bfloat16))).to(device)
        pq, pk = w(num_heads, 3 * head_dim, head_dim), w(num_heads, 3 * head_dim, head_dim)
        so_q = so_k = None
        if second_order_rank:
            so_q, so_k = w(num_heads, head_dim, second_order_rank), w(num_heads, head_dim, second_order_rank)
        gain = torch.ones(num_heads, device=device) if count_term else None
        return cls(pq, pk, so_q, so_k, gain)

    def embed(self, feats: torch.Tensor, heads: torch.Tensor, proj: ProjWeight) -> torch.Tensor:
        """[H', n, 3D] fp32 features -> [H', n, D] tile embeddings."""
        return ops.predictor_embed(feats, proj.values, proj.scale, heads, True)

    def __call__(self, feats_q, feats_k, heads, sq_q=None, var_k=None, log_count=None):
        return self.forward(feats_q, feats_k, heads, sq_q, var_k, log_count)

    def forward(self, feats_q: torch.Tensor, feats_k: torch.Tensor, heads: torch.Tensor,
                sq_q: torch.Tensor | None = None, var_k: torch.Tensor | None = None,
                log_count: torch.Tensor | None = None) -> torch.Tensor:
        """Block logits [H', n_q, n_k] fp32 (predictor.py:299-338).

        Raises:
            ValueError: If a feature is missing, or given when its term is off.
        """
        if (self.count_gain is not None) != (log_count is not None):
            raise ValueError('log_count and count_term must be set together')
        if bool(self.second_order_rank) != (sq_q is not None and var_k is not None):
            raise ValueError('second-order features and second_order_rank must be set together')
        q_hat = self.embed(feats_q, heads, self.proj_q)
        k_hat = self.embed(feats_k, heads, self.proj_k)
        logits = ops.predictor_logits(q_hat, k_hat, 1.0 / math.sqrt(self.head_dim),
                                      self.count_gain, heads if log_count is not None else None,
                                      log_count, None)
        if not self.second_order_rank:
            return logits
        u = ops.predictor_embed(sq_q, self.so_q.values, self.so_q.scale, heads, False)
        w = ops.predictor_embed(var_k, self.so_k.values, self.so_k.scale, heads, False)
        return ops.predictor_logits(u, w, 1.0, None, None, None, logits)


class TileScorePredictor:
    """All layers of the predictor (predictor.py:341-410)."""

    def __init__(self, layers: list[LayerPredictor]):
        self.layers = layers
        first = layers[0]
        self.second_order_rank = first.second_order_rank
        self.count_term = first.count_gain is not None

    @classmethod
    def random(cls, num_layers: int, num_heads: int, head_dim: int, **kw) -> 'TileScorePredictor':
        return cls([LayerPredictor.random(num_heads, head_dim, **kw) for _ in range(num_layers)])

    def scores(self, layer: int, q_tiles: torch.Tensor, k_tiles: torch.Tensor,
               layout: tiling.TileLayout, heads: torch.Tensor) -> torch.Tensor:
        feats_q = pool_tiles(q_tiles, layout)
        feats_k = pool_tiles(k_tiles, layout)
        extra = {}
        if self.count_term:
            extra['log_count'] = log_count(layout)
        if self.second_order_rank:
            extra['sq_q'] = pool_tiles(q_tiles, layout, SECOND_RAW)
            extra['var_k'] = pool_tiles(k_tiles, layout, SECOND_CENTRAL)
        return self.layers[layer](feats_q, feats_k, heads, **extra)


def log_count(layout: tiling.TileLayout) -> torch.Tensor:
    """log(max(valid_count, 1)) per key tile, cached for the layout (so it
    lives exactly as long as the layout does)."""
    return tiling.layout_cached(
        layout, 'log_count',
        lambda: torch.log(layout.valid_count.clamp(min=1).to(torch.float32)))
