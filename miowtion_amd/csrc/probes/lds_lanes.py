"""LDS lane groups of ds_read_b128 / ds_read_b64 on gfx950.

Runs `gfx950_probe lanes` under `rocprofv3 --pmc SQ_LDS_BANK_CONFLICT` (512
one-wave dispatches; in dispatch k two lanes, a and b, read one bank at two
addresses) and prints, per instruction and lane a, the lanes b whose dispatch
counted bank conflicts: the lanes the LDS serves in the same cycle as a.

Usage (from the repository root, after `make -C miowtion_amd/csrc/probes`):
    python miowtion_amd/csrc/probes/lds_lanes.py OUT_DIR
"""

from __future__ import annotations

import csv
import os
import pathlib
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
LANE_A = (0, 5, 17, 42)
MODES = ('ds_read_b128', 'ds_read_b64')


def main(out_dir: str) -> int:
    out = pathlib.Path(out_dir).resolve()
    out.mkdir(parents=True, exist_ok=True)
    env = dict(os.environ, TMPDIR='/tmp')
    cmd = ['rocprofv3', '--pmc', 'SQ_LDS_BANK_CONFLICT', '--output-format', 'csv', '-d', str(out),
           '-o', 'lanes', '--', str(HERE / 'gfx950_probe'), 'lanes']
    rc = subprocess.run(cmd, cwd='/tmp', env=env, timeout=60).returncode
    if rc != 0:
        return rc
    rows = [r for r in csv.DictReader(open(out / 'lanes_counter_collection.csv'))
            if 'lane_kernel' in r['Kernel_Name']]
    per_dispatch: dict[int, float] = {}
    for r in rows:
        d = int(r['Dispatch_Id'])
        per_dispatch[d] = per_dispatch.get(d, 0.0) + float(r['Counter_Value'])
    values = [per_dispatch[d] for d in sorted(per_dispatch)]
    if len(values) != 2 * len(LANE_A) * 64:
        print(f'expected {2 * len(LANE_A) * 64} dispatches, found {len(values)}')
        return 1
    k = 0
    for mode in MODES:
        for a in LANE_A:
            same = [b for b in range(64) if b != a and values[k + b] > 0]
            print(f'{mode}: lane {a:2d} shares its cycle with lanes {same}')
            k += 64
    return 0


if __name__ == '__main__':
    sys.exit(main(sys.argv[1] if len(sys.argv) > 1 else 'gpurun_out/lds_lanes'))
