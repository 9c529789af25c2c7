"""Writes tests/golden/plan_16x9_t37.json from the reference's released plan
file plans/released/16x9_t37.json (a data file the reference ships; read as
JSON, nothing executed). Only the plan table is kept: geometry, grid, shapes
and the [50 layers][56 heads] shape index; the search provenance is dropped.

Also writes tests/golden/plan_grids.json: for every plan file the reference
ships (plans/*/*.json), its geometry name, token grid, shapes and table
size -- the grids pin the geometry rounding rules.

Run in the build container (the reference is not present on the GPU box):
    python tests/golden/make_plan_fixture.py /root/reference
"""

import json
import pathlib
import sys


def main(ref_root: str) -> None:
    src = pathlib.Path(ref_root) / 'plans' / 'released' / '16x9_t37.json'
    data = json.loads(src.read_text())
    out = {k: data[k] for k in ('geometry', 'grid', 'shapes', 'head_shape')}
    out['provenance'] = {'source': 'plans/released/16x9_t37.json'}
    dst = pathlib.Path(__file__).parent / 'plan_16x9_t37.json'
    dst.write_text(json.dumps(out, separators=(',', ':')) + '\n')
    print(f'wrote {dst}')
    grids = {}
    for path in sorted((pathlib.Path(ref_root) / 'plans').glob('*/*.json')):
        plan = json.loads(path.read_text())
        grids[f'{path.parent.name}/{path.name}'] = {
            'geometry': plan['geometry'], 'grid': plan['grid'], 'shapes': plan['shapes'],
            'layers': len(plan['head_shape']), 'heads': len(plan['head_shape'][0])}
    dst = pathlib.Path(__file__).parent / 'plan_grids.json'
    dst.write_text(json.dumps(grids, indent=1) + '\n')
    print(f'wrote {dst}')


if __name__ == '__main__':
    main(sys.argv[1] if len(sys.argv) > 1 else '/root/reference')
