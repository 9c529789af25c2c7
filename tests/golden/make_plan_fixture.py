"""Writes tests/golden/plan_16x9_t37.json from the reference's released plan
file plans/released/16x9_t37.json (a data file the reference ships; read as
JSON, nothing executed). Only the plan table is kept: geometry, grid, shapes
and the [50 layers][56 heads] shape index; the search provenance is dropped.

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


if __name__ == '__main__':
    main(sys.argv[1] if len(sys.argv) > 1 else '/root/reference')
