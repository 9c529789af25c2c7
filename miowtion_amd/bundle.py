"""Predictor bundles: the live predictor weights and the tile plans in one
safetensors file, format 'miowtion-veda-predictor-v1' (the reference's
`miowtion/veda/bundle.py:48-359`; files load in both directions).

On disk:
  tensors   the predictor's state-dict names, `layers.<l>.proj_q`,
            `proj_k`, and `so_q`, `so_k`, `count_gain` when the predictor has
            those terms, stored as float32, bfloat16 or float8_e4m3fn; an
            e4m3 tensor has a per-head fp32 scale (its amax / 448; one
            scale for a 1-D tensor) under '<name>.__scale';
  metadata  strings: format; num_layers, num_heads, head_dim,
            second_order_rank, count_term ('1' / '0'); dtype;
            tile_conditions ('true' / 'false'); source, source_weights,
            step; the target budget as target_budget_kind ('ratio' /
            'tiles') and target_budget_value (repr of a float), likewise
            ref_* when references are tiled, plus keep_ratio for a ratio
            target (the key older readers use); plans, every plan of the
            table as one JSON object keyed by geometry name.

Here the file is handled by three small pieces: `Header` (the metadata as
typed fields, `to_metadata` / `from_metadata`), `weight_schema` (the tensor
names and shapes a header implies) and the e4m3 codec.

Resident form. The reference loads an e4m3 bundle back as bf16 parameters
(`values.float() * scale -> bf16`). Here the projections of an e4m3 bundle
stay e4m3 + scale by default (half the memory of the bf16 copy); the
predictor kernel decodes every element to that same bf16 value
(`veda::predictor_embed`), so the logits are the same bits.
`keep_fp8=False` materialises the bf16 copy instead.

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
CHECKPOINT_PREFIX = 'predictor.'
SCALE_SUFFIX = '.__scale'
E4M3_MAX = 448.0
DTYPES = {'float32': torch.float32, 'bfloat16': torch.bfloat16,
          'float8_e4m3fn': torch.float8_e4m3fn}
_DTYPE_NAMES = {dtype: name for name, dtype in DTYPES.items()}
# the dtype of bundles written before the dtype was recorded
_UNRECORDED_DTYPE = 'float32'


# ---------------------------------------------------------------------------
# e4m3 with a per-head scale

def quantize_fp8(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """[H, ...] -> (e4m3 values, fp32 scale [H]): each head divided by its
    absolute maximum / 448 (never below the smallest normal fp32), then
    rounded to e4m3 by torch's conversion. A 1-D tensor is one head."""
    w = weight.float()
    per_head = w.abs().reshape(w.shape[0], -1).amax(dim=1) if w.dim() > 1 else w.abs().amax()
    scale = torch.clamp(per_head / E4M3_MAX, min=torch.finfo(torch.float32).tiny)
    values = w / scale.reshape(scale.shape + (1,) * (w.dim() - scale.dim()))
    return values.to(torch.float8_e4m3fn).contiguous(), scale.contiguous()


def dequantize_fp8(values: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """values * scale in fp32, then rounded to `dtype`."""
    s = scale.float()
    return (values.float() * s.reshape(s.shape + (1,) * (values.dim() - s.dim()))).to(dtype)


# ---------------------------------------------------------------------------
# metadata

def _budget_from(prefix: str, ratio: float | None, tiles: float | None) -> veda_mask.Budget:
    if (ratio is None) == (tiles is None):
        raise ValueError(f'a {prefix} budget takes exactly one of a ratio or a tile count')
    return veda_mask.Budget(ratio=ratio) if tiles is None else veda_mask.Budget(tiles=tiles)


@dataclasses.dataclass
class Header:
    """The bundle's metadata as typed fields."""

    num_layers: int
    num_heads: int
    head_dim: int
    dtype: str
    target: veda_mask.Budget
    ref: veda_mask.Budget | None
    tile_conditions: bool
    source: str
    source_weights: str
    step: int
    second_order_rank: int
    count_term: bool
    plans: dict  # geometry name -> plan JSON

    @staticmethod
    def _budget_strings(prefix: str, budget: veda_mask.Budget) -> dict[str, str]:
        kind, value = ('ratio', budget.ratio) if budget.ratio is not None else ('tiles',
                                                                             budget.tiles)
        return {prefix + '_budget_kind': kind, prefix + '_budget_value': repr(float(value))}

    def to_metadata(self) -> dict[str, str]:
        meta = {'format': FORMAT, 'num_layers': str(self.num_layers),
                'num_heads': str(self.num_heads), 'head_dim': str(self.head_dim),
                'dtype': self.dtype, 'tile_conditions': 'true' if self.tile_conditions else 'false',
                'source': self.source, 'source_weights': self.source_weights,
                'step': str(self.step), 'second_order_rank': str(self.second_order_rank),
                'count_term': '1' if self.count_term else '0',
                'plans': json.dumps({k: self.plans[k] for k in sorted(self.plans)})}
        meta.update(self._budget_strings('target', self.target))
        if self.ref is not None:
            meta.update(self._budget_strings('ref', self.ref))
        if self.target.ratio is not None:
            meta['keep_ratio'] = repr(float(self.target.ratio))
        return meta

    @staticmethod
    def _budget(meta: dict[str, str], prefix: str) -> veda_mask.Budget | None:
        kind = meta.get(prefix + '_budget_kind')
        if kind is None:
            return None
        value = meta.get(prefix + '_budget_value')
        if kind not in ('ratio', 'tiles') or value is None:
            raise ValueError(f'bad {prefix} budget in the metadata: kind {kind!r}, '
                             f'value {value!r}')
        return veda_mask.Budget(**{kind: float(value)})

    @classmethod
    def from_metadata(cls, meta: dict[str, str], where: str) -> 'Header':
        target = cls._budget(meta, 'target')
        if target is None and 'keep_ratio' in meta:     # bundles older than the budget keys
            target = veda_mask.Budget(ratio=float(meta['keep_ratio']))
        if target is None:
            raise ValueError(f'{where}: the bundle records no target budget')
        header = cls(num_layers=int(meta['num_layers']), num_heads=int(meta['num_heads']),
                     head_dim=int(meta['head_dim']), dtype=meta.get('dtype', _UNRECORDED_DTYPE),
                     target=target, ref=cls._budget(meta, 'ref'),
                     tile_conditions=meta.get('tile_conditions', 'false') == 'true',
                     source=meta.get('source', ''), source_weights=meta.get('source_weights', ''),
                     step=int(meta.get('step', 0)),
                     second_order_rank=int(meta.get('second_order_rank', 0)),
                     count_term=meta.get('count_term', '0') == '1',
                     plans=json.loads(meta['plans']))
        if header.dtype not in DTYPES:
            raise ValueError(f'{where}: storage dtype {header.dtype!r} is not one of '
                             f'{sorted(DTYPES)}')
        if header.tile_conditions and header.ref is None:
            raise ValueError(f'{where}: tiled references without a ref budget')
        return header


def weight_schema(h: Header) -> dict[str, tuple[int, ...]]:
    """Tensor name -> shape of the predictor a header declares."""
    d = h.head_dim
    per_layer = {'proj_q': (h.num_heads, 3 * d, d), 'proj_k': (h.num_heads, 3 * d, d)}
    if h.second_order_rank:
        per_layer.update(so_q=(h.num_heads, d, h.second_order_rank),
                         so_k=(h.num_heads, d, h.second_order_rank))
    if h.count_term:
        per_layer['count_gain'] = (h.num_heads,)
    return {f'layers.{i}.{name}': shape for i in range(h.num_layers)
            for name, shape in per_layer.items()}


# ---------------------------------------------------------------------------
# files

@dataclasses.dataclass
class Bundle:
    """A loaded bundle: the predictor on its device, the plan table, the
    budgets it was trained with, and the raw metadata (provenance)."""

    predictor: veda_predictor.TileScorePredictor
    plans: veda_plan.PlanTable
    target_budget: veda_mask.Budget
    ref_budget: veda_mask.Budget | None
    tile_conditions: bool
    keep_ratio: float | None
    metadata: dict[str, str]


def state_dict(predictor: veda_predictor.TileScorePredictor) -> dict[str, torch.Tensor]:
    """The predictor's weights under their bundle names, in their resident
    value (an e4m3 projection as its bf16 decoding)."""
    out = {}
    for i, layer in enumerate(predictor.layers):
        for name in ('proj_q', 'proj_k', 'so_q', 'so_k'):
            w = getattr(layer, name)
            if w is not None:
                out[f'layers.{i}.{name}'] = (w.values if w.scale is None else
                                             dequantize_fp8(w.values, w.scale, torch.bfloat16))
        if layer.count_gain is not None:
            out[f'layers.{i}.count_gain'] = layer.count_gain
    return out


def _strip_prefix(weights: dict[str, torch.Tensor]) -> dict[str, torch.Tensor]:
    """Bare names from either bare or checkpoint ('predictor.'-prefixed) keys."""
    tagged = sum(k.startswith(CHECKPOINT_PREFIX) for k in weights)
    if tagged not in (0, len(weights)):
        raise ValueError("the weights mix prefixed ('predictor.') and bare keys")
    cut = len(CHECKPOINT_PREFIX) if tagged else 0
    return {k[cut:]: v.detach().cpu() for k, v in weights.items()}


def save(path: str, weights: dict[str, torch.Tensor], plans: veda_plan.PlanTable, *,
         num_layers: int, num_heads: int, head_dim: int, keep_ratio: float | None = None,
         keep_tiles: float | None = None, ref_keep_ratio: float | None = None,
         ref_keep_tiles: float | None = None, tile_conditions: bool = False, source: str,
         source_weights: str, step: int, dtype: torch.dtype = torch.bfloat16,
         second_order_rank: int = 0, count_term: bool = False) -> None:
    """Writes a bundle (the arguments of `miowtion/veda/bundle.py:147`).

    Raises:
        ValueError: On no weights, keys that mix the checkpoint prefix with
            bare names, a storage dtype outside DTYPES, an empty plan table,
            a budget given both or neither way, a reference budget without
            tile_conditions, or tile_conditions without one.
    """
    if dtype not in _DTYPE_NAMES:
        raise ValueError(f'storage dtype {dtype} is not one of {sorted(DTYPES)}')
    if not weights:
        raise ValueError('there are no predictor weights to save')
    bare = _strip_prefix(weights)
    if not plans.plans:
        raise ValueError('a bundle carries its plans: the plan table is empty')
    has_ref = ref_keep_ratio is not None or ref_keep_tiles is not None
    if has_ref != bool(tile_conditions):
        raise ValueError('a reference budget requires tile_conditions' if has_ref else
                         'tile_conditions requires a reference budget')
    header = Header(num_layers=num_layers, num_heads=num_heads, head_dim=head_dim,
                    dtype=_DTYPE_NAMES[dtype], target=_budget_from('target', keep_ratio,
                                                                   keep_tiles),
                    ref=_budget_from('ref', ref_keep_ratio, ref_keep_tiles) if has_ref else None,
                    tile_conditions=bool(tile_conditions), source=source,
                    source_weights=source_weights, step=step,
                    second_order_rank=second_order_rank, count_term=count_term,
                    plans={name: p.to_json() for name, p in plans.plans.items()})
    tensors = {}
    for name, value in bare.items():
        if dtype is torch.float8_e4m3fn:
            tensors[name], tensors[name + SCALE_SUFFIX] = quantize_fp8(value)
        else:
            tensors[name] = value.to(dtype).contiguous()
    save_file(tensors, path, metadata=header.to_metadata())


def read_metadata(path: str) -> dict[str, str]:
    """The string metadata, without reading a tensor.

    Raises:
        ValueError: If the file is not a bundle of this format.
    """
    with safe_open(path, framework='pt', device='cpu') as f:
        meta = dict(f.metadata() or {})
    if meta.get('format') != FORMAT:
        raise ValueError(f'{path} is not a {FORMAT} bundle (its format is '
                         f'{meta.get("format")!r})')
    return meta


def load(path: str, device: torch.device | str = 'cpu', keep_fp8: bool = True) -> Bundle:
    """Loads a bundle strictly: exactly the tensors of the predictor its
    metadata declares, with their shapes.

    Raises:
        ValueError: If the file is not a bundle of this format, records an
            unknown dtype or no target budget, has an e4m3 tensor without its
            scale, or tensors that do not match the declared predictor.
    """
    meta = read_metadata(path)
    header = Header.from_metadata(meta, path)
    with safe_open(path, framework='pt', device='cpu') as f:
        stored = {k: f.get_tensor(k) for k in f.keys()}
    fp8 = header.dtype == 'float8_e4m3fn'
    scales = {k[:-len(SCALE_SUFFIX)]: stored.pop(k) for k in list(stored)
              if fp8 and k.endswith(SCALE_SUFFIX)}
    if fp8 and set(stored) - set(scales):
        raise ValueError(f'{path}: e4m3 tensors without a {SCALE_SUFFIX} scale: '
                         f'{sorted(set(stored) - set(scales))}')
    schema = weight_schema(header)
    wrong = sorted(k for k in stored if k in schema and tuple(stored[k].shape) != schema[k])
    if set(stored) != set(schema) or wrong:
        raise ValueError(
            f'{path}: the weights do not match the {header.num_layers}-layer, '
            f'{header.num_heads}-head, d{header.head_dim} predictor its metadata declares '
            f'(missing {sorted(set(schema) - set(stored))}, extra '
            f'{sorted(set(stored) - set(schema))}, wrong shape {wrong})')
    # the reference's resident dtype: bf16 for an e4m3 file, else as stored
    resident = torch.bfloat16 if fp8 else DTYPES[header.dtype]

    def decoded(name: str) -> torch.Tensor:
        if name in scales:
            return dequantize_fp8(stored[name], scales[name], resident)
        return stored[name].to(resident)

    def projection(name: str) -> veda_predictor.ProjWeight:
        if name in scales and keep_fp8:
            return veda_predictor.ProjWeight(stored[name], scales[name]).to(device)
        return veda_predictor.ProjWeight(decoded(name)).to(device)

    layers = []
    for i in range(header.num_layers):
        so = header.second_order_rank > 0
        layers.append(veda_predictor.LayerPredictor(
            projection(f'layers.{i}.proj_q'), projection(f'layers.{i}.proj_k'),
            projection(f'layers.{i}.so_q') if so else None,
            projection(f'layers.{i}.so_k') if so else None,
            decoded(f'layers.{i}.count_gain').float().to(device) if header.count_term else None))
    table = veda_plan.PlanTable([veda_plan.TilePlan.from_json(p) for p in header.plans.values()])
    return Bundle(predictor=veda_predictor.TileScorePredictor(layers), plans=table,
                  target_budget=header.target, ref_budget=header.ref,
                  tile_conditions=header.tile_conditions, keep_ratio=header.target.ratio,
                  metadata=meta)


def random_bundle(num_layers: int, num_heads: int, head_dim: int,
                  geometries: Sequence[veda_geometry.Geometry], keep_ratio: float, seed: int = 0,
                  device: torch.device | str = 'cpu') -> Bundle:
    """A random predictor with, per geometry, a plan that gives every head
    the least-padding shape of its grid: what a Veda step costs depends on
    the budget, the shapes and the predictor's size, not on the weights, so
    this serves benchmarks (the reference's `random_bundle`)."""
    predictor = veda_predictor.TileScorePredictor.random(
        num_layers, num_heads, head_dim, generator=torch.Generator().manual_seed(seed),
        device=device)
    table = veda_plan.PlanTable([
        veda_plan.TilePlan.uniform(g, tiling.least_padding_shape(g.video_grid), num_layers,
                                   num_heads) for g in geometries])
    return Bundle(predictor=predictor, plans=table,
                  target_budget=veda_mask.Budget(ratio=keep_ratio), ref_budget=None,
                  tile_conditions=False, keep_ratio=keep_ratio,
                  metadata={'source': 'random', 'seed': str(seed)})
