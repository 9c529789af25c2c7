"""Tile plans: the tile shape of every (layer, head) for one geometry, and
the table that picks a geometry's plan.

The JSON form is the reference's plan-file format (`plans/*.json`, written
by `miowtion/veda/plan.py:81-101`): {'geometry', 'grid', 'shapes' (shape
strings), 'head_shape' ([layer][head] index into shapes), 'provenance'}; the
released plan files load unchanged. A layer uses at most two shapes (the
attention runs one head group per shape).

The selection rule is the reference's (`PlanTable.select`,
`miowtion/veda/plan.py:160-188`), which training and inference must share:
the exact geometry; else the same aspect ratio at the nearest latent_t, ties
to the shorter clip; else, only when the aspect has no plan at all, the
mirrored aspect's plan nearest in latent_t, as stored or transposed,
whichever needs fewer tiles on the requested grid (ties and equal distances
keep the plan met first, in the order the table was given its plans).
"""

from __future__ import annotations

import dataclasses
import glob
import json
import os
import tempfile
from collections.abc import Sequence

import torch

from miowtion_amd import geometry as veda_geometry
from miowtion_amd import tiling

MAX_SHAPES_PER_LAYER = 2


@dataclasses.dataclass
class HeadGroup:
    """Heads of one layer that share a tile shape."""

    shape: tiling.TileShape
    heads: torch.Tensor  # [H'] int64


def _aspect_key(name: str) -> str:
    """'16x9' of a plan or geometry name '16x9_t37'."""
    return name.split('_t')[0]


def _mirror_key(aspect_key: str) -> str:
    w, h = aspect_key.split('x')
    return f'{h}x{w}'


@dataclasses.dataclass
class TilePlan:
    """Per-(layer, head) shape choice for one geometry.

    geometry: its name ('16x9_t37'); grid: the (T, H, W) token grid the plan
    was made for; shapes: the distinct shapes; head_shape[layer][head]: an
    index into shapes; provenance: free-form metadata.

    Raises (on construction):
        ValueError: If a layer uses more than two shapes, or an index is
            outside shapes.
    """

    geometry: str
    grid: tuple[int, int, int]
    shapes: list[tiling.TileShape]
    head_shape: list[list[int]]
    provenance: dict = dataclasses.field(default_factory=dict)

    def __post_init__(self):
        self.grid = tuple(self.grid)
        for layer, row in enumerate(self.head_shape):
            used = set(row)
            if len(used) > MAX_SHAPES_PER_LAYER:
                raise ValueError(f'plan {self.geometry}: layer {layer} uses {len(used)} shapes '
                                 f'(at most {MAX_SHAPES_PER_LAYER} per layer are allowed)')
            if used and (min(used) < 0 or max(used) >= len(self.shapes)):
                raise ValueError(f'plan {self.geometry}: layer {layer} indexes a shape outside '
                                 f'the {len(self.shapes)} it lists')
        self._groups: dict = {}

    @property
    def num_layers(self) -> int:
        return len(self.head_shape)

    def layer_shapes(self, layer: int) -> list[tiling.TileShape]:
        return [self.shapes[i] for i in sorted(set(self.head_shape[layer]))]

    def head_groups(self, layer: int, device: torch.device | str) -> list[HeadGroup]:
        """The layer's heads grouped by shape, in shape-index order, each
        group's heads ascending (built once per layer and device)."""
        key = (layer, str(device))
        groups = self._groups.get(key)
        if groups is None:
            members: dict[int, list[int]] = {}
            for head, index in enumerate(self.head_shape[layer]):
                members.setdefault(index, []).append(head)
            groups = [HeadGroup(self.shapes[i], torch.tensor(members[i], dtype=torch.int64,
                                                             device=device))
                      for i in sorted(members)]
            self._groups[key] = groups
        return groups

    # -- plan-file form ------------------------------------------------------
    def to_json(self) -> dict:
        return dict(geometry=self.geometry, grid=list(self.grid),
                    shapes=[str(s) for s in self.shapes],
                    head_shape=[list(row) for row in self.head_shape],
                    provenance=dict(self.provenance))

    @classmethod
    def from_json(cls, data: dict) -> 'TilePlan':
        return cls(data['geometry'], tuple(data['grid']),
                   [tiling.TileShape.parse(s) for s in data['shapes']],
                   [list(row) for row in data['head_shape']], data.get('provenance', {}))

    def save(self, path: str) -> None:
        """Writes the plan file; a reader never sees a partial file."""
        folder = os.path.dirname(os.path.abspath(path))
        fd, tmp = tempfile.mkstemp(prefix='.plan-', suffix='.json', dir=folder)
        try:
            with os.fdopen(fd, 'w') as f:
                json.dump(self.to_json(), f, indent=1)
            # mkstemp creates the file 0600; give it the mode open() would
            # (0666 less the umask), as the reference's writer does
            umask = os.umask(0)
            os.umask(umask)
            os.chmod(tmp, 0o666 & ~umask)
            os.replace(tmp, path)
        except BaseException:
            if os.path.exists(tmp):
                os.unlink(tmp)
            raise

    @classmethod
    def load(cls, path: str) -> 'TilePlan':
        with open(path) as f:
            return cls.from_json(json.load(f))

    # -- derived plans -------------------------------------------------------
    @classmethod
    def uniform(cls, geometry, *args) -> 'TilePlan':
        """One shape for every head of every layer.

        uniform(geometry: Geometry, shape, num_layers, num_heads) or, for a
        grid without a resolved geometry, uniform(name, grid, shape,
        num_layers, num_heads).
        """
        if isinstance(geometry, veda_geometry.Geometry):
            name, grid, (shape, num_layers, num_heads) = geometry.name, geometry.video_grid, args
        else:
            name, (grid, shape, num_layers, num_heads) = geometry, args
        rows = [[0] * num_heads for _ in range(num_layers)]
        return cls(name, tuple(grid), [shape], rows, {'source': 'uniform'})

    def _swapped(self, name: str, provenance_key: str) -> 'TilePlan':
        t, h, w = self.grid
        return TilePlan(name, (t, w, h), [s.transposed() for s in self.shapes],
                        [list(row) for row in self.head_shape],
                        {**self.provenance, provenance_key: self.geometry})

    def mirrored(self) -> 'TilePlan':
        """This plan for the H<->W mirrored aspect (9x16_t37 from
        16x9_t37), under the mirrored geometry's own name.

        Raises:
            ValueError: If the mirrored geometry's grid is not the transpose
                of this grid (the canvas rounding of the two aspects differs).
        """
        aspect, latent_t = self.geometry.split('_t')
        mirror = veda_geometry.geometry_from_latent_t(
            _mirror_key(aspect).replace('x', ':'), int(latent_t))
        t, h, w = self.grid
        if mirror.video_grid != (t, w, h):
            raise ValueError(f'cannot mirror {self.geometry} {self.grid}: {mirror.name} has '
                             f'grid {mirror.video_grid}, not the transpose')
        return self._swapped(mirror.name, 'mirrored_from')

    def transposed(self) -> 'TilePlan':
        """H<->W transposed plan named '<geometry>_T' (the table's last
        resort for an aspect without plans)."""
        return self._swapped(self.geometry + '_T', 'transposed_from')


class PlanTable:
    """All plans of a run, by geometry name, indexed by aspect."""

    def __init__(self, plans: Sequence[TilePlan]):
        self.plans: dict[str, TilePlan] = {}
        for plan in plans:
            self.plans[plan.geometry] = plan
        self._by_aspect: dict[str, list[TilePlan]] = {}
        for plan in self.plans.values():
            self._by_aspect.setdefault(_aspect_key(plan.geometry), []).append(plan)

    @classmethod
    def load_dir(cls, directory: str) -> 'PlanTable':
        """Every '*.json' plan file of a directory, in file-name order.

        Raises:
            FileNotFoundError: If the directory holds no plan file.
        """
        files = sorted(glob.glob(os.path.join(directory, '*.json')))
        if not files:
            raise FileNotFoundError(f'{directory} holds no plan files')
        return cls([TilePlan.load(f) for f in files])

    def select(self, geometry: veda_geometry.Geometry) -> TilePlan:
        """The plan for `geometry` (rule in the module docstring).

        Raises:
            KeyError: If neither the aspect nor its mirror has a plan.
        """
        exact = self.plans.get(geometry.name)
        if exact is not None:
            return exact
        t = geometry.latent_t
        aspect = geometry.aspect.replace(':', 'x')
        same = self._by_aspect.get(aspect)
        if same:
            return min(same, key=lambda p: (abs(p.grid[0] - t), p.grid[0]))
        mirrored = self._by_aspect.get(_mirror_key(aspect))
        if not mirrored:
            raise KeyError(f'no plan for {geometry.name} or its mirrored aspect')
        base = min(mirrored, key=lambda p: abs(p.grid[0] - t))
        grid = geometry.video_grid
        tiles = lambda plan: sum(shape.num_tiles(grid) for shape in plan.shapes)
        flipped = base.transposed()
        return flipped if tiles(flipped) < tiles(base) else base
