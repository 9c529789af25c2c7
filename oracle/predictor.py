"""Oracle: tile pooling, predictor logits and the fp8 predictor weights
(CPU torch, test-only).

Restates:
  * pool_tiles / _second_moment   -> `miowtion/veda/predictor.py:82-168`
  * LayerPredictor.embed          -> `miowtion/veda/predictor.py:251-255`
  * LayerPredictor.forward        -> `miowtion/veda/predictor.py:299-338`
  * _quantize_fp8 / _dequantize   -> `miowtion/veda/bundle.py:71-93`,
    bf16 resident copy as loaded at `miowtion/veda/bundle.py:280-297`
"""

from __future__ import annotations

import math

import torch

from oracle.tiling import TILE, Layout

E4M3_MAX = 448.0


def pool_tiles(x: torch.Tensor, lay: Layout, second: str | None = None) -> torch.Tensor:
    """[N, H', D] bf16 tile rows (padding zero) -> [H', n, 3D] fp32
    [mean | max | min], or [H', n, D] E[x^2] ('raw') / Var(x) ('central')."""
    n = lay.n_tiles
    t = x.view(n, TILE, *x.shape[1:]).float()
    cnt = lay.valid_count.clamp(min=1).float()
    valid = (torch.arange(TILE)[None, :] < lay.valid_count[:, None])[:, :, None, None]
    mean = t.sum(1) / cnt[:, None, None]
    if second == 'raw':
        feats = (t * t).sum(1) / cnt[:, None, None]
    elif second == 'central':
        c = torch.where(valid, t - mean[:, None], 0.0)
        feats = (c * c).sum(1) / cnt[:, None, None]
    elif second is None:
        tmax = t.masked_fill(~valid, float('-inf')).amax(1)
        tmin = t.masked_fill(~valid, float('inf')).amin(1)
        feats = torch.cat([mean, tmax, tmin], -1)
    else:
        raise ValueError(f'unknown second moment {second!r}')
    # predictor.py:128-129: `where`, not a product, so empty tiles give 0.
    feats = torch.where(lay.kv_ok[:, None, None], feats, 0.0)
    return feats.permute(1, 0, 2).contiguous()


def embed(feats: torch.Tensor, proj: torch.Tensor, heads: torch.Tensor) -> torch.Tensor:
    """predictor.py:251-255: feats @ P[h] + mean, fp32."""
    d = proj.shape[-1]
    return torch.bmm(feats, proj.index_select(0, heads).float()) + feats[..., :d]


def logits(feats_q, feats_k, proj_q, proj_k, heads, *, gain=None, log_count=None,
           sq_q=None, var_k=None, so_q=None, so_k=None) -> torch.Tensor:
    """predictor.py:299-338 -> [H', n_q, n_k] fp32."""
    d = proj_q.shape[-1]
    qh = embed(feats_q, proj_q, heads)
    kh = embed(feats_k, proj_k, heads)
    out = torch.bmm(qh, kh.transpose(1, 2)) / math.sqrt(d)
    if log_count is not None:
        out = out + gain.index_select(0, heads).float()[:, None, None] * log_count[None, None, :]
    if so_q is not None:
        u = torch.bmm(sq_q, so_q.index_select(0, heads).float())
        w = torch.bmm(var_k, so_k.index_select(0, heads).float())
        out = out + torch.bmm(u, w.transpose(1, 2))
    return out


def quantize_fp8(weight: torch.Tensor):
    """bundle.py:71-86: per-head amax onto 448 -> (e4m3 values, fp32 scale)."""
    dims = tuple(range(1, weight.dim()))
    amax = weight.float().abs().amax(dim=dims)
    scale = (amax / E4M3_MAX).clamp(min=torch.finfo(torch.float32).tiny)
    vals = weight.float() / scale.view(-1, *([1] * len(dims)))
    return vals.to(torch.float8_e4m3fn).contiguous(), scale.contiguous()


def dequantize_fp8(values: torch.Tensor, scale: torch.Tensor, dtype=torch.bfloat16):
    """bundle.py:89-93 (loaded as bf16 at bundle.py:280-297)."""
    return (values.float() * scale.view(-1, *([1] * (values.dim() - 1)))).to(dtype)
