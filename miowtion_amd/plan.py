"""Per-(layer, head) tile-shape plans and the plan table (host mirror of
miowtion/veda/plan.py:36-188): at most two shapes per layer, heads grouped
by shape, JSON files saved atomically, and the table's rule for picking the
plan of a geometry. The released plan files (`plans/released/*.json`) load
unchanged."""

from __future__ import annotations

import dataclasses
import glob
import json
import os
from collections.abc import Sequence

import torch

from miowtion_amd import geometry as veda_geometry
from miowtion_amd import tiling


@dataclasses.dataclass
class HeadGroup:
    """Heads of one layer that share a tile shape."""

    shape: tiling.TileShape
    heads: torch.Tensor  # [H'] int64


@dataclasses.dataclass
class TilePlan:
    geometry: str
    grid: tuple[int, int, int]
    shapes: list[tiling.TileShape]
    head_shape: list[list[int]]
    provenance: dict = dataclasses.field(default_factory=dict)

    def __post_init__(self):
        for layer, row in enumerate(self.head_shape):
            if len(set(row)) > 2:
                raise ValueError(f'layer {layer} uses {len(set(row))} shapes; '
                                 'at most 2 per layer are allowed')
        self._groups: dict = {}

    @property
    def num_layers(self) -> int:
        return len(self.head_shape)

    def layer_shapes(self, layer: int) -> list[tiling.TileShape]:
        return [self.shapes[i] for i in sorted(set(self.head_shape[layer]))]

    def head_groups(self, layer: int, device: torch.device | str) -> list[HeadGroup]:
        """Groups of heads sharing a shape, in shape-index order (cached)."""
        key = (layer, str(device))
        if key not in self._groups:
            row = self.head_shape[layer]
            self._groups[key] = [
                HeadGroup(self.shapes[i],
                          torch.tensor([h for h, s in enumerate(row) if s == i],
                                       dtype=torch.int64).to(device))
                for i in sorted(set(row))]
        return self._groups[key]

    def to_json(self) -> dict:
        return {'geometry': self.geometry, 'grid': list(self.grid),
                'shapes': [str(s) for s in self.shapes], 'head_shape': self.head_shape,
                'provenance': self.provenance}

    @classmethod
    def from_json(cls, data: dict) -> 'TilePlan':
        return cls(geometry=data['geometry'], grid=tuple(data['grid']),
                   shapes=[tiling.TileShape.parse(s) for s in data['shapes']],
                   head_shape=[list(r) for r in data['head_shape']],
                   provenance=data.get('provenance', {}))

    def save(self, path: str) -> None:
        tmp = path + '.tmp'
        with open(tmp, 'w') as f:
            json.dump(self.to_json(), f, indent=1)
        os.replace(tmp, path)

    @classmethod
    def load(cls, path: str) -> 'TilePlan':
        with open(path) as f:
            return cls.from_json(json.load(f))

    @classmethod
    def uniform(cls, geometry, *args) -> 'TilePlan':
        """Every head uses one shape (plan.py:113-119).

        uniform(geometry: Geometry, shape, num_layers, num_heads), the
        reference's form, or uniform(name: str, grid, shape, num_layers,
        num_heads) for a grid without a resolved geometry.
        """
        if isinstance(geometry, veda_geometry.Geometry):
            name, grid = geometry.name, geometry.video_grid
            shape, num_layers, num_heads = args
        else:
            name = geometry
            grid, shape, num_layers, num_heads = args
        return cls(name, tuple(grid), [shape], [[0] * num_heads for _ in range(num_layers)],
                   {'source': 'uniform'})

    def mirrored(self) -> 'TilePlan':
        """The plan of the H<->W mirrored geometry, e.g. 9x16_t37 from
        16x9_t37 (plan.py:121-142): shapes and grid transposed, the mirrored
        geometry's name.

        Raises:
            ValueError: If that geometry's grid is not the transposed grid
                (the canvas rounding differs between the two aspects).
        """
        aspect, latent_t = self.geometry.split('_t')
        w, h = aspect.split('x')
        mirror = veda_geometry.geometry_from_latent_t(f'{h}:{w}', int(latent_t))
        t, grid_h, grid_w = self.grid
        if tuple(mirror.video_grid) != (t, grid_w, grid_h):
            raise ValueError(f'{mirror.name} grid {mirror.video_grid} is not the transpose of '
                             f'{self.geometry} {self.grid}')
        return TilePlan(mirror.name, (t, grid_w, grid_h), [s.transposed() for s in self.shapes],
                        [list(r) for r in self.head_shape],
                        {**self.provenance, 'mirrored_from': self.geometry})

    def transposed(self) -> 'TilePlan':
        """H<->W transposed plan under the name '<geometry>_T' (the table's
        fallback only, plan.py:144-150)."""
        t, h, w = self.grid
        return TilePlan(self.geometry + '_T', (t, w, h), [s.transposed() for s in self.shapes],
                        [list(r) for r in self.head_shape],
                        {**self.provenance, 'transposed_from': self.geometry})


class PlanTable:
    """Every searched plan, by geometry name (plan.py:153-188)."""

    def __init__(self, plans: Sequence[TilePlan]):
        self.plans = {p.geometry: p for p in plans}

    @classmethod
    def load_dir(cls, directory: str) -> 'PlanTable':
        paths = sorted(glob.glob(os.path.join(directory, '*.json')))
        if not paths:
            raise FileNotFoundError(f'no plans in {directory}')
        return cls([TilePlan.load(p) for p in paths])

    def select(self, geometry: veda_geometry.Geometry) -> TilePlan:
        """The plan for `geometry`: the exact geometry if present; else the
        same aspect ratio with the nearest latent_t (ties to the shorter
        clip); else, when no plan of this aspect exists, the mirrored
        aspect's nearest plan, as is or transposed, whichever pads the
        target grid least.

        Raises:
            KeyError: If no plan of this or the mirrored aspect exists.
        """
        if geometry.name in self.plans:
            return self.plans[geometry.name]
        aspect_key = geometry.aspect.replace(':', 'x')
        same = [p for p in self.plans.values() if p.geometry.split('_t')[0] == aspect_key]
        if same:
            return min(same, key=lambda p: (abs(p.grid[0] - geometry.latent_t), p.grid[0]))
        w, h = geometry.aspect.split(':')
        mirrored = [p for p in self.plans.values() if p.geometry.split('_t')[0] == f'{h}x{w}']
        if not mirrored:
            raise KeyError(f'no plan for {geometry.name}')
        nearest = min(mirrored, key=lambda p: abs(p.grid[0] - geometry.latent_t))
        grid = geometry.video_grid
        return min((nearest, nearest.transposed()),
                   key=lambda plan: sum(s.num_tiles(grid) for s in plan.shapes))
