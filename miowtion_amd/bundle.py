"""Predictor bundles: the live predictor weights and the tile plans in one
safetensors file (host mirror of `miowtion/veda/bundle.py:48-359`, format
'miowtion-veda-predictor-v1', unchanged on disk).

The file holds the predictor's tensors under their state-dict names
(`layers.<l>.proj_q`, `proj_k`, and `so_q`, `so_k`, `count_gain` when the
predictor has those terms), stored as fp32, bf16 or e4m3. An e4m3 tensor
carries a per-head fp32 scale (amax / 448) under '<name>.__scale'. All
settings are strings in the safetensors `__metadata__`: format, shape
(num_layers, num_heads, head_dim, second_order_rank, count_term), storage
dtype, budgets ('<target|ref>_budget_kind' in {ratio, tiles} and
'_budget_value'), tile_conditions, provenance (source, source_weights,
step) and every plan of the plan table as one JSON blob under 'plans'.

Resident form. The reference loads an e4m3 bundle back as bf16 parameters
(`values.float() * scale -> bf16`, bundle.py:86-93, 296-312). Here the
projections of an e4m3 bundle stay resident as e4m3 + scale by default (half
the memory of the bf16 copy): the predictor kernel decodes every element to
that same bf16 value (`veda::predictor_embed`), so the logits are the same
bits; `keep_fp8=False` materialises the bf16 copy instead.

Only safetensors and JSON are read: nothing in a bundle is executed.
"""

from __future__ import annotations

import dataclasses
import json
from collections.abc import Sequence

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from miowtion_amd import geometry as veda_geometry
from miowtion_amd import mask as veda_mask
from miowtion_amd import plan as veda_plan
from miowtion_amd import predictor as veda_predictor
from miowtion_amd import tiling

FORMAT = 'miowtion-veda-predictor-v1'
PREFIX = 'predictor.'
DTYPES = {'float32': torch.float32, 'bfloat16': torch.bfloat16,
          'float8_e4m3fn': torch.float8_e4m3fn}
E4M3_MAX = 448.0
SCALE_SUFFIX = '.__scale'
LEGACY_DTYPE = 'float32'  # bundles written before the dtype was recorded


def quantize_fp8(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """[H, ...] -> (e4m3 values, [H] fp32 scale) with the head's amax mapped
    onto 448; an all-zero head keeps the smallest normal scale
    (bundle.py:71-86). A 1-D tensor (count_gain) gets one scale for all its
    entries: amax over an empty dim tuple reduces every dim, as in the
    reference."""
    dims = tuple(range(1, weight.dim()))
    amax = weight.float().abs().amax(dim=dims)
    scale = (amax / E4M3_MAX).clamp(min=torch.finfo(torch.float32).tiny)
    values = weight.float() / scale.view(-1, *([1] * len(dims)))
    return values.to(torch.float8_e4m3fn).contiguous(), scale.contiguous()


def dequantize_fp8(values: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """values * scale in fp32, then rounded to `dtype` (bundle.py:89-93)."""
    return (values.float() * scale.view(-1, *([1] * (values.dim() - 1)))).to(dtype)


@dataclasses.dataclass
class Bundle:
    """A loaded bundle (bundle.py:96-117)."""

    predictor: veda_predictor.TileScorePredictor
    plans: veda_plan.PlanTable
    target_budget: veda_mask.Budget
    ref_budget: veda_mask.Budget | None
    tile_conditions: bool
    keep_ratio: float | None
    metadata: dict[str, str]


def _budget_metadata(prefix: str, ratio: float | None, tiles: float | None) -> dict[str, str]:
    if (ratio is None) == (tiles is None):
        raise ValueError(f'set exactly one of {prefix}_ratio / {prefix}_tiles')
    if tiles is not None:
        veda_mask.Budget(tiles=tiles)
        return {f'{prefix}_budget_kind': 'tiles', f'{prefix}_budget_value': repr(float(tiles))}
    veda_mask.Budget(ratio=ratio)
    return {f'{prefix}_budget_kind': 'ratio', f'{prefix}_budget_value': repr(float(ratio))}


def _read_budget(metadata: dict[str, str], prefix: str,
                 legacy_ratio: str | None = None) -> veda_mask.Budget | None:
    kind = metadata.get(f'{prefix}_budget_kind')
    value = metadata.get(f'{prefix}_budget_value')
    if kind is None:
        if legacy_ratio and legacy_ratio in metadata:
            return veda_mask.Budget(ratio=float(metadata[legacy_ratio]))
        return None
    if kind not in ('ratio', 'tiles') or value is None:
        raise ValueError(f'invalid {prefix} budget metadata: kind={kind!r}, value={value!r}')
    return veda_mask.Budget(**{kind: float(value)})


def state_dict(predictor: veda_predictor.TileScorePredictor) -> dict[str, torch.Tensor]:
    """The predictor's weights under the reference's state-dict names, in the
    resident value (an e4m3 projection decoded to its bf16 value)."""
    out = {}
    for i, layer in enumerate(predictor.layers):
        for name in ('proj_q', 'proj_k', 'so_q', 'so_k'):
            w = getattr(layer, name)
            if w is None:
                continue
            if w.scale is not None:
                out[f'layers.{i}.{name}'] = dequantize_fp8(w.values, w.scale, torch.bfloat16)
            else:
                out[f'layers.{i}.{name}'] = w.values
        if layer.count_gain is not None:
            out[f'layers.{i}.count_gain'] = layer.count_gain
    return out


def save(path: str, weights: dict[str, torch.Tensor], plans: veda_plan.PlanTable, *,
         num_layers: int, num_heads: int, head_dim: int, keep_ratio: float | None = None,
         keep_tiles: float | None = None, ref_keep_ratio: float | None = None,
         ref_keep_tiles: float | None = None, tile_conditions: bool = False, source: str,
         source_weights: str, step: int, dtype: torch.dtype = torch.bfloat16,
         second_order_rank: int = 0, count_term: bool = False) -> None:
    """Writes a bundle (bundle.py:147-235).

    Raises:
        ValueError: On empty weights, prefixed and bare keys mixed, an
            unsupported dtype, missing plans, or inconsistent budgets.
    """
    if not weights:
        raise ValueError('no predictor weights to save')
    target_metadata = _budget_metadata('target', keep_ratio, keep_tiles)
    if ref_keep_ratio is not None or ref_keep_tiles is not None:
        if not tile_conditions:
            raise ValueError('a reference budget requires tile_conditions')
        ref_metadata = _budget_metadata('ref', ref_keep_ratio, ref_keep_tiles)
    else:
        if tile_conditions:
            raise ValueError('tile_conditions requires a reference budget')
        ref_metadata = {}
    names = {v: k for k, v in DTYPES.items()}
    if dtype not in names:
        raise ValueError(f'unsupported storage dtype {dtype}; expected one of {sorted(DTYPES)}')
    prefixed = [k for k in weights if k.startswith(PREFIX)]
    if prefixed and len(prefixed) != len(weights):
        raise ValueError('weights mix prefixed and bare keys')
    bare = {k[len(PREFIX):] if prefixed else k: v.detach().cpu() for k, v in weights.items()}
    if dtype is torch.float8_e4m3fn:
        tensors = {}
        for key, value in bare.items():
            tensors[key], tensors[key + SCALE_SUFFIX] = quantize_fp8(value)
    else:
        tensors = {k: v.to(dtype).contiguous() for k, v in bare.items()}
    if not plans.plans:
        raise ValueError("bundle without plans; pass the run's plan table")
    metadata = {
        'format': FORMAT,
        'num_layers': str(num_layers),
        'num_heads': str(num_heads),
        'head_dim': str(head_dim),
        'dtype': names[dtype],
        'tile_conditions': str(bool(tile_conditions)).lower(),
        'source': source,
        'source_weights': source_weights,
        'step': str(step),
        'second_order_rank': str(second_order_rank),
        'count_term': '1' if count_term else '0',
        'plans': json.dumps({name: p.to_json() for name, p in sorted(plans.plans.items())}),
    }
    metadata.update(target_metadata)
    metadata.update(ref_metadata)
    if keep_ratio is not None:  # readers of ratio-only bundles use this key
        metadata['keep_ratio'] = repr(float(keep_ratio))
    save_file(tensors, path, metadata=metadata)


def read_metadata(path: str) -> dict[str, str]:
    """The string metadata, without reading a tensor.

    Raises:
        ValueError: If the file is not a bundle of this format.
    """
    with safe_open(path, framework='pt', device='cpu') as f:
        metadata = dict(f.metadata() or {})
    if metadata.get('format') != FORMAT:
        raise ValueError(f'{path}: not a {FORMAT} bundle (format {metadata.get("format")!r})')
    return metadata


def _expected_shapes(num_layers: int, num_heads: int, head_dim: int, rank: int,
                     count_term: bool) -> dict[str, tuple[int, ...]]:
    shapes = {}
    for i in range(num_layers):
        shapes[f'layers.{i}.proj_q'] = (num_heads, 3 * head_dim, head_dim)
        shapes[f'layers.{i}.proj_k'] = (num_heads, 3 * head_dim, head_dim)
        if rank:
            shapes[f'layers.{i}.so_q'] = (num_heads, head_dim, rank)
            shapes[f'layers.{i}.so_k'] = (num_heads, head_dim, rank)
        if count_term:
            shapes[f'layers.{i}.count_gain'] = (num_heads,)
    return shapes


def load(path: str, device: torch.device | str = 'cpu', keep_fp8: bool = True) -> Bundle:
    """Loads a bundle strictly: every stored tensor must be a weight the
    metadata's predictor has, with its shape, and none may be missing
    (bundle.py:254-335).

    Raises:
        ValueError: If the file is not a bundle of this format, has an
            unknown dtype, fp8 tensors without scales, or weights that do not
            match the declared predictor.
    """
    metadata = read_metadata(path)
    with safe_open(path, framework='pt', device='cpu') as f:
        tensors = {k: f.get_tensor(k) for k in f.keys()}
    stored = metadata.get('dtype', LEGACY_DTYPE)
    if stored not in DTYPES:
        raise ValueError(f'{path}: unknown storage dtype {stored!r}')
    num_layers, num_heads = int(metadata['num_layers']), int(metadata['num_heads'])
    head_dim = int(metadata['head_dim'])
    rank = int(metadata.get('second_order_rank', 0))
    count_term = metadata.get('count_term', '0') == '1'
    scales = {}
    if stored == 'float8_e4m3fn':
        scales = {k[:-len(SCALE_SUFFIX)]: v for k, v in tensors.items()
                  if k.endswith(SCALE_SUFFIX)}
        tensors = {k: v for k, v in tensors.items() if not k.endswith(SCALE_SUFFIX)}
        missing = sorted(set(tensors) - set(scales))
        if missing:
            raise ValueError(f'{path}: fp8 tensors without a {SCALE_SUFFIX} scale: {missing}')
    shape = f'{num_layers} layers x {num_heads} heads x {head_dim}'
    want = _expected_shapes(num_layers, num_heads, head_dim, rank, count_term)
    if set(tensors) != set(want):
        raise ValueError(f'{path}: predictor weights do not match the {shape} the metadata '
                         f'declares: missing {sorted(set(want) - set(tensors))}, unexpected '
                         f'{sorted(set(tensors) - set(want))}')
    for k, v in tensors.items():
        if tuple(v.shape) != want[k]:
            raise ValueError(f'{path}: {k} has shape {tuple(v.shape)}, the {shape} predictor '
                             f'needs {want[k]}')
    # The reference holds an e4m3 bundle as bf16 parameters; fp32 and bf16
    # bundles stay in their stored dtype.
    resident = torch.bfloat16 if stored == 'float8_e4m3fn' else DTYPES[stored]

    def proj(key: str) -> veda_predictor.ProjWeight:
        v = tensors[key]
        if key in scales and keep_fp8:
            return veda_predictor.ProjWeight(v, scales[key]).to(device)
        if key in scales:
            v = dequantize_fp8(v, scales[key], resident)
        return veda_predictor.ProjWeight(v.to(resident)).to(device)

    def gain(key: str) -> torch.Tensor:
        v = tensors[key]
        if key in scales:
            v = dequantize_fp8(v, scales[key], resident)
        return v.to(resident).float().to(device)

    layers = []
    for i in range(num_layers):
        pre = f'layers.{i}.'
        layers.append(veda_predictor.LayerPredictor(
            proj(pre + 'proj_q'), proj(pre + 'proj_k'),
            proj(pre + 'so_q') if rank else None, proj(pre + 'so_k') if rank else None,
            gain(pre + 'count_gain') if count_term else None))
    plans = veda_plan.PlanTable([veda_plan.TilePlan.from_json(p)
                                 for p in json.loads(metadata['plans']).values()])
    target_budget = _read_budget(metadata, 'target', legacy_ratio='keep_ratio')
    if target_budget is None:
        raise ValueError(f'{path}: bundle has no target budget')
    ref_budget = _read_budget(metadata, 'ref')
    tile_conditions = metadata.get('tile_conditions', 'false') == 'true'
    if tile_conditions and ref_budget is None:
        raise ValueError(f'{path}: tiled references need a ref budget')
    return Bundle(predictor=veda_predictor.TileScorePredictor(layers), plans=plans,
                  target_budget=target_budget, ref_budget=ref_budget,
                  tile_conditions=tile_conditions, keep_ratio=target_budget.ratio,
                  metadata=metadata)


def random_bundle(num_layers: int, num_heads: int, head_dim: int,
                  geometries: Sequence[veda_geometry.Geometry], keep_ratio: float, seed: int = 0,
                  device: torch.device | str = 'cpu') -> Bundle:
    """A randomly initialised predictor with a uniform least-padding plan per
    geometry, for benchmarks (bundle.py:338-359): the cost of a Veda step is
    fixed by the budget, the shapes and the predictor's size, not by the
    scores."""
    gen = torch.Generator().manual_seed(seed)
    predictor = veda_predictor.TileScorePredictor.random(num_layers, num_heads, head_dim,
                                                         generator=gen, device=device)
    plans = veda_plan.PlanTable([
        veda_plan.TilePlan.uniform(g, tiling.least_padding_shape(g.video_grid), num_layers,
                                   num_heads) for g in geometries])
    return Bundle(predictor=predictor, plans=plans,
                  target_budget=veda_mask.Budget(ratio=keep_ratio), ref_budget=None,
                  tile_conditions=False, keep_ratio=keep_ratio,
                  metadata={'source': 'random', 'seed': str(seed)})
