"""End-to-end GPU parity of the attention plug-ins (the drop-in boundary,
`AttentionFn(q, k, v, layer) -> out`) against the oracle chain:

  SparseStudent: gather + pool -> predictor logits -> top-k -> block mask ->
      lists -> sparse attention -> scatter (miowtion/veda/attention.py:745-794).
      Block lists are bit-exact to the oracle's on the same logits; the
      output matches the fp32 masked-dense oracle.
  Dynamic tile shapes (BASELINE config 3 in miniature): two head groups with
      their own permutations; the permutation round trip is bit-exact.
  OracleStudent: dense LSE -> heat('sum') -> top-k -> sparse (config 5's chain).
"""

import pytest
import torch

from miowtion_amd import attention as pa
from miowtion_amd import mask as pm
from miowtion_amd import plan as pplan
from miowtion_amd import predictor as pp
from miowtion_amd import tiling as pt
from oracle import attention as oa
from oracle import mask as om
from oracle import predictor as op
from oracle import tiling as ot
from tests import helpers
from tests.test_gpu_attention import _close

pytestmark = pytest.mark.gpu


def _oracle_student(q, k, v, olay, heads, logits, ratio):
    """Oracle of one head group given the predictor logits."""
    idx, keep = om.select_video_blocks(logits[:, :olay.n_video_tiles], olay,
                                       om.column_blocks(olay, om.Budget(ratio=ratio)))
    mask = om.dense_block_mask(idx, keep, olay)
    qt, kt, vt = (ot.gather_tiles(t, olay, heads) for t in (q, k, v))
    o = oa.block_sparse_attention(qt, kt, vt, mask, olay.valid_count)
    out = torch.zeros(olay.seq_len + 1, *q.shape[1:], dtype=q.dtype)
    ot.scatter_tiles_(out, o, olay, heads)
    return out[:olay.seq_len], (idx, keep, mask)


def _clip(spans, used, seq_len, ratio):
    layout = pa.PackedLayout(tuple(pa.VideoSpan(s, g) for s, g in spans), used, seq_len)
    return pa.ClipTiling(layout, pa.VedaConfig(target_budget=pm.Budget(ratio=ratio)), 'cuda')


def test_sparse_student_config1():
    spans, used, seq_len, shape = helpers.CONFIGS['C1']
    clip = _clip(spans, used, seq_len, 0.5)
    plan = pplan.TilePlan.uniform('c1', spans[-1][1], pt.TileShape.parse(shape), 1, 8)
    pred = pp.TileScorePredictor([pp.LayerPredictor.random(
        8, 128, std=0.02, generator=torch.Generator().manual_seed(3), device='cuda', fp8=True)])
    student = pa.SparseStudent(clip, plan, pred)
    q, k, v = helpers.qkv(seq_len, 8, 128, seed=5)
    out = student(q.cuda(), k.cuda(), v.cuda(), 0)
    part = student.last['parts'][0]
    olay = helpers.oracle_layout(spans, used, seq_len, shape)
    heads = torch.arange(8)
    want, (idx, keep, mask) = _oracle_student(q, k, v, olay, heads, part['logits'].cpu(), 0.5)
    assert torch.equal(part['selection'].index.cpu(), idx)
    assert torch.equal(part['selection'].keep.cpu(), keep)
    for a, b in zip(part['lists'], om.index_lists(mask, olay)):
        assert torch.equal(a.cpu(), b)
    _close(out, want)
    # the logits themselves follow the oracle predictor to fp32 tolerance
    lp = pred.layers[0]
    oq, ok = ot.gather_tiles(q, olay, heads), ot.gather_tiles(k, olay, heads)
    wl = op.logits(op.pool_tiles(oq, olay), op.pool_tiles(ok, olay),
                   op.dequantize_fp8(lp.proj_q.values.cpu(), lp.proj_q.scale.cpu()),
                   op.dequantize_fp8(lp.proj_k.values.cpu(), lp.proj_k.scale.cpu()), heads)
    assert (part['logits'].cpu() - wl).abs().max() <= 1e-4 * wl.abs().max()


class _NaNBufferStudent(pa.SparseStudent):
    """A student whose scatter buffer starts as NaN: a (real row, head) the
    layer failed to write would show as NaN in its output."""

    def _output_buffer(self, q, rows):
        self.buffer = torch.full((rows, *q.shape[1:]), float('nan'), dtype=q.dtype,
                                 device=q.device)
        return self.buffer


def _oracle_compensated(q, k, v, olay, heads, logits, ratio):
    """Oracle of one head group with zero-order compensation
    (attention.py:591-689 after the selection) given the predictor logits."""
    idx, keep = om.select_video_blocks(logits[:, :olay.n_video_tiles], olay,
                                       om.column_blocks(olay, om.Budget(ratio=ratio)))
    mask = om.dense_block_mask(idx, keep, olay) & olay.kv_ok[None, None, :]
    qt, kt, vt = (ot.gather_tiles(t, olay, heads) for t in (q, k, v))
    o, lse = oa.block_sparse_attention(qt, kt, vt, mask, olay.valid_count, return_lse=True)
    comp = oa.zero_order_compensation(o, lse, qt, kt, vt, mask, olay.valid_count)
    out = torch.zeros(olay.seq_len + 1, *q.shape[1:], dtype=q.dtype)
    ot.scatter_tiles_(out, comp, olay, heads)
    return out[:olay.seq_len], (idx, keep, mask)


@pytest.mark.parametrize('compensation', [False, True])
def test_sparse_student_dynamic_shapes_and_round_trip(compensation):
    """Two tile shapes in one layer (seeded per-head choice), 80% sparsity,
    padded tails as partial tiles; out rows match the oracle (with the
    zero-order compensation when set), padding rows 0, and every real row
    of every head is written (the buffer starts as NaN)."""
    grid = (9, 20, 12)
    start = 200
    used = start + grid[0] * grid[1] * grid[2]
    seq_len = used + 48
    spans = [(start, grid)]
    layout = pa.PackedLayout(tuple(pa.VideoSpan(s, g) for s, g in spans), used, seq_len)
    cfg = pa.VedaConfig(target_budget=pm.Budget(ratio=0.2),
                        zero_order_compensation=compensation)
    clip = pa.ClipTiling(layout, cfg, 'cuda')
    H = 6
    choice = torch.randint(0, 2, (H,), generator=torch.Generator().manual_seed(0)).tolist()
    shapes = [pt.TileShape(1, 8, 16), pt.TileShape(4, 4, 8)]
    plan = pplan.TilePlan('dyn', grid, shapes, [choice])
    assert len(set(choice)) == 2
    pred = pp.TileScorePredictor([pp.LayerPredictor.random(
        H, 128, std=0.02, generator=torch.Generator().manual_seed(4), device='cuda')])
    student = _NaNBufferStudent(clip, plan, pred)
    q, k, v = helpers.qkv(seq_len, H, 128, seed=9)
    q[used:] = 0
    out = student(q.cuda(), k.cuda(), v.cuda(), 0)
    assert out.data_ptr() == student.buffer.data_ptr()      # the NaN buffer was the output
    out = out.cpu()
    assert not torch.isnan(out.float()).any()
    assert (out[used:] == 0).all()
    want = torch.zeros(seq_len, H, 128, dtype=torch.bfloat16)
    oracle = _oracle_compensated if compensation else _oracle_student
    for part in student.last['parts']:
        heads = part['heads'].cpu()
        shape = shapes[choice[int(heads[0])]]
        olay = helpers.oracle_layout(spans, used, seq_len, str(shape))
        o, (idx, keep, _) = oracle(q, k, v, olay, heads, part['logits'].cpu(), 0.2)
        assert torch.equal(part['selection'].index.cpu(), idx)
        assert torch.equal(part['selection'].keep.cpu(), keep)
        want[:, heads] = o[:, heads]
    if compensation:
        _close(out[:used].float(), want[:used].float())
    else:
        _close(out[:used], want[:used])


@pytest.mark.parametrize('fused', [True, False])
def test_oracle_student_matches_oracle_chain(fused):
    spec = helpers.small_layout(grid=(6, 12, 20), shape='2x8x8', text=100, extra=16)
    spans, used, seq_len, shape = spec
    clip = _clip(spans, used, seq_len, 0.3)
    plan = pplan.TilePlan.uniform('o', spans[-1][1], pt.TileShape.parse(shape), 1, 4)
    student = pa.OracleStudent(clip, plan, target='mass', fused=fused)
    q, k, v = helpers.qkv(seq_len, 4, 128, seed=2)
    out = student(q.cuda(), k.cuda(), v.cuda(), 0).cpu()
    olay = helpers.oracle_layout(*spec)
    heads = torch.arange(4)
    _, lse = oa.dense_attention(q, k, v, used, return_lse=True)
    rows = torch.arange(olay.n_video_tiles)
    if fused:
        # the tile-ordered LSE of the fused pass, on the real rows
        got = student.last['parts'][0]['lse_tiles'].cpu()
        want = ot.gather_lse(lse, olay, heads)[:rows.numel() * 128].t()
        real = olay.slot_valid[:rows.numel() * 128].bool()
        torch.testing.assert_close(got[:, real], want[:, real], rtol=0, atol=2e-4)
    else:
        _close(student.last['lse'], lse)
    qt, kt = ot.gather_tiles(q, olay, heads), ot.gather_tiles(k, olay, heads)
    # select on the kernel's heat: the selection is then bit-exact
    heat = student.last['parts'][0]['heat'].cpu()
    ref_heat = oa.teacher_heat(qt, kt, ot.gather_lse(lse, olay, heads), olay, rows, 'sum')
    torch.testing.assert_close(heat, ref_heat, rtol=2e-3, atol=1e-6)
    want, (idx, keep, _) = _oracle_student(q, k, v, olay, heads, heat, 0.3)
    sel = student.last['parts'][0]['selection']
    assert torch.equal(sel.index.cpu(), idx) and torch.equal(sel.keep.cpu(), keep)
    _close(out[:used], want[:used])


@pytest.mark.parametrize('kind', ['sparse', 'compensated', 'oracle', 'oracle_two_pass'])
def test_head_chunks_change_nothing(kind):
    """Splitting every head group into at least three chunks (collect_bytes
    lowered, attention.py:204-206) gives the same bits as one chunk per
    group: heads are independent (the reference pins this for the student,
    tests/unit/test_veda_heatmap_attention.py:210-235, and for the oracle
    path, tests/gpu/test_kernels_gpu.py:159). Two tile shapes, six heads
    each."""
    grid = (9, 20, 12)
    start = 200
    used = start + grid[0] * grid[1] * grid[2]
    seq_len = used + 48
    layout = pa.PackedLayout((pa.VideoSpan(start, grid),), used, seq_len)
    H = 12
    shapes = [pt.TileShape(1, 8, 16), pt.TileShape(4, 4, 8)]
    plan = pplan.TilePlan('chunks', grid, shapes, [[h % 2 for h in range(H)]])
    pred = pp.TileScorePredictor([pp.LayerPredictor.random(
        H, 128, std=0.02, generator=torch.Generator().manual_seed(7), device='cuda')])
    q, k, v = (t.cuda() for t in helpers.qkv(seq_len, H, 128, seed=13))

    def run(collect_bytes):
        cfg = pa.VedaConfig(target_budget=pm.Budget(ratio=0.3), collect_bytes=collect_bytes,
                            zero_order_compensation=kind == 'compensated')
        clip = pa.ClipTiling(layout, cfg, 'cuda')
        if kind.startswith('oracle'):
            student = pa.OracleStudent(clip, plan, fused=kind == 'oracle')
        else:
            student = pa.SparseStudent(clip, plan, pred)
        out = student(q, k, v, 0)
        torch.cuda.synchronize()
        return out.cpu(), student, clip

    whole, s_whole, clip = run(pa.DEFAULT_COLLECT_BYTES)
    slots = max(clip.get(s).num_slots for s in shapes)
    chunked, s_chunked, _ = run(2 * slots * 128 * 2)
    assert len(s_whole.last['parts']) == 2
    per_group: dict = {}
    for part in s_chunked.last['parts']:
        per_group[part['shape'].num_slots] = per_group.get(part['shape'].num_slots, 0) + 1
    assert len(per_group) == 2 and min(per_group.values()) >= 3, per_group
    assert torch.equal(chunked, whole)
    assert not torch.isnan(whole.float()).any() and (whole[used:] == 0).all()
