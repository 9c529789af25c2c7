"""Benchmark of the Veda block-sparse attention hot path on one MI355X.

Workload: one H3-scale layer, video grid 37x30x52 =
57,720 tokens (seq_len 57,728), 48 heads, head_dim 128, bf16 q/k/v ~ N(0,1),
tile shape (1,8,16) -> 592 query / key tiles, uniform random tile scores,
equal-cost budget 0.1 * 451^2 / 592 with Bresenham rounding and the forced
diagonal -> 20,340 kept 128x128 blocks per head (90% sparsity).

A step = one block-sparse attention forward over all 48 heads with the block
lists prebuilt (the reference bench's "kernel" timing,
miowtion/kernels/bench.py:87-126). As the reference bench does
(:313-314, 337-343), the timed loop cycles through several seeded patterns
(distinct uniform random score tensors, each giving 20,340 kept blocks per
head), and before any rate is reported the output of every pattern is
checked against fp32 masked attention of 3 query tiles x 2 heads computed
with plain torch (:129-144, 315-333): the line carries the max error, a
dense-match guard, and no TFLOP/s unless the error is within 2e-2.

Reported beside it: "+prep" (selection, block mask and lists rebuilt per
call), the full Veda layer (pooling of q and k, predictor, selection, lists,
sparse forward reading q, k and v in sequence order with the scatter fused
in) on the same C2 patterns, the same layer with the lists of
its random-weight predictor (labelled as such), the dense baselines at the
same shape, the roofline of the sparse kernel and the CPU baseline (the
oracle's masked-dense attention + predictor on host cores).

Prints ONE JSON line. Effective TFLOP/s counts computed blocks only,
4 * 128 * 128 * D per kept block (miowtion/kernels/bench.py:52-60).
"""

from __future__ import annotations

import argparse
import itertools
import json
import math
import os
import pathlib
import sys
import time

import torch

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = 'block-sparse attn ms/layer + effective TFLOP/s @57.7k tok, 90% sparse, 1 GPU'
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0
GRID = (37, 30, 52)
HEADS = 48
D = 128
RATIO = 0.1
PATTERNS = 4          # distinct seeded block patterns cycled in the timed loop
CHECK_MAX_ERR = 2e-2  # fp32-reference bar a timed kernel must meet for its rate to count


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _events_ms(fn, reps: int) -> list[float]:
    """Per-call durations (ms) measured with events on the current stream,
    which is the stream every op of this package launches on."""
    out = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        b.synchronize()
        out.append(a.elapsed_time(b))
    return out


def build_case(seed: int = 0, patterns: int = 1):
    """The C2 layout, q / k / v and `patterns` seeded score tensors, each with
    its block mask and lists (pattern 0 is the first draw after q, k, v)."""
    from miowtion_amd import kernels, mask as pm, tiling as pt
    used = GRID[0] * GRID[1] * GRID[2]
    seq_len = -(-used // 64) * 64
    lay = pt.build_tile_layout([pt.TiledSpan(0, GRID, pt.TileShape(1, 8, 16))], used, seq_len, 'cuda')
    g = torch.Generator(device='cuda').manual_seed(seed)
    q, k, v = (torch.randn(seq_len, HEADS, D, generator=g, device='cuda').to(torch.bfloat16)
               for _ in range(3))
    for t in (q, k, v):
        t[used:] = 0
    all_scores = [torch.rand(HEADS, lay.n_tiles, lay.n_tiles, generator=g, device='cuda')
                  for _ in range(max(1, patterns))]
    qt, kt, vt = (kernels.gather_tiles(t, lay, None) for t in (q, k, v))
    blocks = pm.column_blocks(lay, pm.Budget(ratio=RATIO))

    def prep(i: int = 0):
        sel = pm.select_video_blocks(all_scores[i], lay, blocks)
        mask = pm.dense_block_mask(sel, lay)
        return mask, kernels.index_lists(mask, lay)

    built = [prep(i) for i in range(len(all_scores))]
    return dict(lay=lay, q=q, k=k, v=v, qt=qt, kt=kt, vt=vt, scores=all_scores[0],
                all_scores=all_scores, prep=prep, mask=built[0][0], lists=built[0][1],
                masks=[b[0] for b in built], all_lists=[b[1] for b in built],
                used=used, seq_len=seq_len)


def check_rows(c: dict, outs: list, tiles: list[int], heads: list[int]) -> dict:
    """fp32 masked attention of query tiles `tiles` x `heads` with plain torch
    (on the device, outside any timed region), against each pattern's
    tile-ordered output in `outs`; also against dense attention (every key
    tile kept), which a correct sparse output must be further from
    (miowtion/kernels/bench.py:129-144, 315-333)."""
    lay = c['lay']
    key_ok = lay.slot_valid.bool()                               # [N] real key slots
    scale = 1.0 / math.sqrt(D)
    err = dense_err = 0.0
    for mask, out in zip(c['masks'], outs):
        for h in heads:
            k = c['kt'][:, h].float()
            v = c['vt'][:, h].float()
            for i in tiles:
                rows = slice(i * 128, (i + 1) * 128)
                s = (c['qt'][rows, h].float() @ k.T) * scale                 # [128, N]
                kept = mask[h, i].repeat_interleave(128) & key_ok
                ref = torch.softmax(s.masked_fill(~kept[None], float('-inf')), -1) @ v
                dense = torch.softmax(s.masked_fill(~key_ok[None], float('-inf')), -1) @ v
                got = out[rows, h].float()
                err = max(err, (got - ref).abs().max().item())
                dense_err = max(dense_err, (got - dense).abs().max().item())
    verdict = 'ok'
    if not err <= CHECK_MAX_ERR:
        verdict = f'WRONG: max_err {err:.3g} above {CHECK_MAX_ERR}'
    elif dense_err < err:
        verdict = 'WRONG: output matches dense attention'
    return {'max_err': err, 'dense_err': dense_err, 'bar': CHECK_MAX_ERR, 'verdict': verdict,
            'query_tiles': tiles, 'heads': heads, 'patterns': len(outs)}


def cpu_baseline(budget_s: float = 20.0) -> dict:
    """The oracle (the reference's CPU torch path restated: predictor pooling +
    logits + top-k, and masked-dense fp32 attention) on host cores, on a
    bounded sample of the C2 workload: 1 head, query tiles taken in order until
    the time budget is spent; scaled to all 592 x 48 query tiles."""
    from oracle import attention as oa, mask as om, predictor as op, tiling as ot
    used = GRID[0] * GRID[1] * GRID[2]
    seq_len = -(-used // 64) * 64
    lay = ot.build_layout([ot.Span(0, GRID, ot.Shape(1, 8, 16))], used, seq_len)
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(seq_len, 1, D, generator=g).to(torch.bfloat16) for _ in range(3))
    qt, kt, vt = (ot.gather_tiles(t, lay, None) for t in (q, k, v))
    t0 = time.perf_counter()
    pq = torch.randn(1, 3 * D, D, generator=g) * 0.02
    pk = torch.randn(1, 3 * D, D, generator=g) * 0.02
    logits = op.logits(op.pool_tiles(qt, lay), op.pool_tiles(kt, lay), pq, pk, torch.tensor([0]))
    idx, keep = om.select_video_blocks(logits, lay, om.column_blocks(lay, om.Budget(ratio=RATIO)))
    mask = om.dense_block_mask(idx, keep, lay)
    t_pred = time.perf_counter() - t0
    n = lay.n_tiles
    done, t_attn, blocks = 0, 0.0, 0
    step = 4
    while done < n and t_attn < budget_s:
        rows = torch.arange(done, min(done + step, n))
        sub_q = qt.view(n, 128, 1, D)[rows].reshape(-1, 1, D)
        t1 = time.perf_counter()
        oa.block_sparse_attention(sub_q, kt, vt, mask[:, rows], lay.valid_count, q_chunk=512)
        t_attn += time.perf_counter() - t1
        blocks += int(mask[:, rows].sum())
        done += rows.numel()
    per_tile = t_attn / done
    layer_s = (per_tile * n + t_pred) * HEADS
    flop = 4.0 * 128 * 128 * D * 20340 * HEADS
    return {'value': round(flop / layer_s / 1e12, 6), 'unit': 'TFLOP/s (effective)',
            'ms_per_layer': round(layer_s * 1e3, 1),
            'cores': torch.get_num_threads(), 'os_cpu_count': os.cpu_count(), 'kind': 'port',
            'sample': (f'C2, 1 of {HEADS} heads: predictor (pool + logits + top-k) on all '
                       f'{n} tiles and masked-dense fp32 attention on {done} of {n} query tiles '
                       f'({t_attn:.1f} s); scaled linearly to {n} tiles x {HEADS} heads')}


def _traffic() -> float | None:
    f = ROOT / 'profiles' / 'sparse_fwd_c2_traffic.json'
    if f.exists():
        try:
            return json.loads(f.read_text()).get('hbm_bytes_per_launch')
        except (ValueError, OSError):
            return None
    return None


def _median_ms(fn, reps: int = 5, batch: int = 1) -> float:
    """Median over `reps` event-timed runs of `batch` back-to-back calls,
    per call. Sub-millisecond kernels are timed in batches of 10, so the
    host's per-call work (allocation, argument checks, the ctypes call)
    overlaps the previous launch instead of being counted as kernel time."""
    fn()
    torch.cuda.synchronize()

    def run():
        for _ in range(batch):
            fn()
    t = sorted(_events_ms(run, reps))
    return t[len(t) // 2] / batch


def _hbm(ms: float, nbytes: float) -> dict:
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {'ms': round(ms, 4), 'bytes': nbytes, 'bound': 'hbm', 'achieved': round(gbs, 1),
            'unit': 'GB/s', 'peak': PEAK_HBM_GBS, 'frac': round(gbs / PEAK_HBM_GBS, 4)}


def _mfma(ms: float, flop: float) -> dict:
    tf = flop / (ms * 1e-3) / 1e12
    return {'ms': round(ms, 4), 'flop': flop, 'bound': 'mfma', 'achieved': round(tf, 1),
            'unit': 'TFLOP/s', 'peak': PEAK_BF16_TFLOPS, 'frac': round(tf / PEAK_BF16_TFLOPS, 4)}


def suite(reps: int = 5) -> dict:
    """Every kernel of the path at its BASELINE configuration, each against
    its own roofline (HBM-bound kernels: algorithmic bytes; MFMA-bound:
    algorithmic FLOP; selection and predictor are small and reported as time).
    Synthetic seeded inputs, resident in HBM before timing."""
    from miowtion_amd import attention as pa, kernels, mask as pm, plan as pplan
    from miowtion_amd import predictor as pp, tiling as pt
    res = {}
    # ---- C2: 57,720 tokens x 48 heads, (1,8,16) tiles
    _log('suite: C2')
    c = build_case()
    lay, q, v = c['lay'], c['q'], c['v']
    n, N, used = lay.n_tiles, lay.num_slots, c['used']
    row = HEADS * D * 2  # bytes of one [H, D] bf16 row
    feats = HEADS * n * 3 * D * 4
    ms = _median_ms(lambda: kernels.gather_and_pool(q, lay, None), reps, 10)
    res['gather_pool_q_c2'] = _hbm(ms, used * row + N * row + feats)
    ms = _median_ms(lambda: kernels.gather_tiles(v, lay, None), reps, 10)
    res['gather_v_c2'] = _hbm(ms, used * row + N * row)
    outbuf = torch.zeros(c['seq_len'] + 1, HEADS, D, dtype=torch.bfloat16, device='cuda')
    ms = _median_ms(lambda: kernels.scatter_tiles_(outbuf, c['qt'], lay, None), reps, 10)
    res['scatter_c2'] = _hbm(ms, 2 * used * row)
    blocks = pm.column_blocks(lay, pm.Budget(ratio=RATIO))
    ms = _median_ms(lambda: pm.select_video_blocks(c['scores'], lay, blocks), reps, 10)
    res['select_topk_c2'] = {'ms': round(ms, 4), 'bound': 'small (reported, not rooflined)'}
    # a ~30 us kernel: through the C-ABI into preallocated lists, since the
    # operator's per-call host work (four allocations, dispatch) takes longer
    # than the kernel and batching cannot hide it
    from miowtion_amd import _native
    lists = [torch.empty(shape, dtype=torch.int32, device='cuda')
             for shape in ((HEADS, n), (HEADS, n, n), (HEADS, n), (HEADS, n, n))]
    stream = torch.cuda.current_stream().cuda_stream
    ms = _median_ms(lambda: _native.call(
        'veda_index_lists', c['mask'].data_ptr(), HEADS, n, n, lay.kv_ok.data_ptr(),
        lay.full_tile.data_ptr(), *(t.data_ptr() for t in lists), stream), reps, 10)
    res['index_lists_c2'] = _hbm(ms, HEADS * n * n * (1 + 2 * 4) + 2 * HEADS * n * 4)
    res['index_lists_c2']['timing'] = 'C-ABI call into preallocated lists'
    del lists
    pred = pp.LayerPredictor.random(HEADS, D, std=0.02, generator=torch.Generator().manual_seed(1),
                                    device='cuda', fp8=True)
    _, fq = kernels.gather_and_pool(q, lay, None)
    _, fk = kernels.gather_and_pool(c['k'], lay, None)
    heads = torch.arange(HEADS, device='cuda')
    ms = _median_ms(lambda: pred(fq, fk, heads), reps, 10)
    pflop = 2 * 2.0 * n * 3 * D * D * HEADS + 2.0 * n * n * D * HEADS
    res['predictor_c2'] = {'ms': round(ms, 4), 'flop': pflop,
                           'tflops_fp32': round(pflop / (ms * 1e-3) / 1e12, 2),
                           'bound': 'small (fp32 GEMMs, reported, not rooflined)'}
    kept = int(c['mask'].sum())
    ms = _median_ms(lambda: kernels.block_sparse_attention_lists(c['qt'], c['kt'], c['vt'],
                                                                 c['lists'], lay), reps)
    res['sparse_fwd_c2'] = _mfma(ms, 4.0 * 128 * 128 * D * kept)
    # block-sparse backward (stage-2 training) given the forward's out and LSE:
    # 5 products of 2 * 128 * 128 * D per kept block (S, dP, dV, dK, dQ; the
    # dQ kernel's recomputation of S and dP is not counted)
    from miowtion_amd import ops
    lists_t = kernels.index_lists(c['mask'], lay, transpose=True)
    o_f, lse_f = kernels.block_sparse_attention_lists(c['qt'], c['kt'], c['vt'], c['lists'], lay,
                                                      return_lse=True)
    dout = torch.randn(o_f.shape, generator=torch.Generator(device='cuda').manual_seed(3),
                       device='cuda').to(torch.bfloat16)
    # the layer's gradient (zero on padding rows, whose outputs the scatter
    # drops), then N(0, 1) on every row
    dout_layer = dout * lay.slot_valid.to(dout.dtype)[:, None, None]
    for key, d in (('sparse_bwd_c2', dout_layer), ('sparse_bwd_c2_every_row', dout)):
        ms_b = _median_ms(lambda: ops.block_sparse_bwd(c['qt'], c['kt'], c['vt'], o_f, d, lse_f,
                                                       None, *c['lists'], *lists_t,
                                                       lay.valid_count,
                                                       lay.n_tiles - lay.n_video_tiles), reps)
        res[key] = _mfma(ms_b, 10.0 * 128 * 128 * D * kept)
        res[key]['vs_sparse_fwd'] = round(ms_b / ms, 3)
    del lists_t, o_f, lse_f, dout, dout_layer
    # zero-order compensation of the dropped tiles (summaries + the virtual-key
    # pass; the reference's Triton form costs 1.14x its sparse kernel)
    o_kept, lse_kept = kernels.block_sparse_attention_lists(c['qt'], c['kt'], c['vt'], c['lists'],
                                                            lay, return_lse=True)
    ms_c = _median_ms(lambda: kernels.zero_order_compensation(o_kept, lse_kept, c['qt'], c['kt'],
                                                              c['vt'], c['mask'], lay), reps)
    res['compensation_c2'] = _mfma(ms_c, 4.0 * c['qt'].shape[0] * n * D * HEADS)
    res['compensation_c2']['vs_sparse_fwd'] = round((ms + ms_c) / ms, 3)
    del o_kept, lse_kept
    # the same in one pass (compensation_triton.attention): kept blocks and
    # virtual keys in one online softmax; summaries included, lists prebuilt
    ms_f = _median_ms(lambda: kernels.compensated_attention(c['qt'], c['kt'], c['vt'], c['mask'],
                                                            lay, c['lists']), reps)
    res['compensated_attention_c2'] = _mfma(ms_f, 4.0 * 128 * 128 * D * kept
                                            + 4.0 * c['qt'].shape[0] * n * D * HEADS)
    res['compensated_attention_c2']['vs_sparse_fwd'] = round(ms_f / ms, 3)
    ms = _median_ms(lambda: kernels.dense_attention(q, c['k'], v, used, return_lse=True), 3)
    res['dense_fwd_lse_c2'] = _mfma(ms, 4.0 * used * used * HEADS * D)
    del c, outbuf, fq, fk
    torch.cuda.empty_cache()

    # ---- C3: 9:16 grid, per-head shape (1,8,16) or (4,4,8), keep 0.2, full layer
    _log('suite: C3')
    grid3 = (37, 52, 30)
    used3 = grid3[0] * grid3[1] * grid3[2]
    seq3 = -(-used3 // 64) * 64
    g = torch.Generator(device='cuda').manual_seed(3)
    q3, k3, v3 = (torch.randn(seq3, HEADS, D, generator=g, device='cuda').to(torch.bfloat16)
                  for _ in range(3))
    layout3 = pa.PackedLayout((pa.VideoSpan(0, grid3),), used3, seq3)
    clip3 = pa.ClipTiling(layout3, pa.VedaConfig(target_budget=pm.Budget(ratio=0.2)), 'cuda')
    choice = torch.randint(0, 2, (HEADS,), generator=torch.Generator().manual_seed(3))
    shapes = [pt.TileShape(1, 8, 16), pt.TileShape(4, 4, 8)]
    plan3 = pplan.TilePlan('9x16_t37_c3', grid3, shapes, [choice.tolist()])
    pred3 = pp.TileScorePredictor([pp.LayerPredictor.random(
        HEADS, D, std=0.02, generator=torch.Generator().manual_seed(4), device='cuda', fp8=True)])
    student3 = pa.SparseStudent(clip3, plan3, pred3)
    ms = _median_ms(lambda: student3(q3, k3, v3, 0), 3)
    res['veda_layer_c3'] = {'ms': round(ms, 4), 'groups': [int((choice == i).sum()) for i in (0, 1)],
                            'bound': 'whole layer (pooling, predictor, selection, lists, '
                                     'sparse forward in sequence order), reported as time'}
    del q3, k3, v3, student3, clip3
    torch.cuda.empty_cache()

    # ---- C5: 2,048 global rows + 102x30x52 video, keep 0.05
    _log('suite: C5')
    grid5 = (102, 30, 52)
    start5 = 2048
    used5 = start5 + grid5[0] * grid5[1] * grid5[2]
    seq5 = -(-used5 // 64) * 64
    lay5 = pt.build_tile_layout([pt.TiledSpan(start5, grid5, pt.TileShape(1, 8, 16))], used5,
                                seq5, 'cuda')
    g = torch.Generator(device='cuda').manual_seed(5)
    q5, k5, v5 = (torch.randn(seq5, HEADS, D, generator=g, device='cuda').to(torch.bfloat16)
                  for _ in range(3))
    for t in (q5, k5, v5):
        t[used5:] = 0
    ms = _median_ms(lambda: kernels.dense_attention(q5, k5, v5, used5, return_lse=True), 3)
    res['dense_fwd_lse_c5'] = _mfma(ms, 4.0 * used5 * used5 * HEADS * D)
    _, lse5 = kernels.dense_attention(q5, k5, v5, used5, return_lse=True)
    qt5, kt5, vt5 = (kernels.gather_tiles(t, lay5, None) for t in (q5, k5, v5))
    lse_t = kernels.gather_lse(lse5, lay5, heads)
    n5, nv5 = lay5.n_tiles, lay5.n_video_tiles
    rows5 = torch.arange(nv5, device='cuda')
    ms = _median_ms(lambda: kernels.teacher_heat(qt5, kt5, lse_t, lay5, rows5, 'sum'), 3)
    res['heat_sum_c5'] = _mfma(ms, 2.0 * 128 * 128 * D * nv5 * n5 * HEADS)
    # the fused teacher pass in tile order: LSE + heat from one QK^T pass
    # (what OracleStudent runs instead of dense_fwd_lse + heat), and the same
    # pass with the dense output as well
    ms_f = _median_ms(lambda: kernels.dense_heat(qt5, kt5, lay5, rows5, 'sum'), 3)
    res['dense_heat_sum_c5'] = _mfma(ms_f, 2.0 * 128 * 128 * D * nv5 * n5 * HEADS)
    res['dense_heat_sum_c5']['two_pass_ms'] = round(res['dense_fwd_lse_c5']['ms'] +
                                                    res['heat_sum_c5']['ms'], 4)
    ms_o = _median_ms(lambda: kernels.dense_heat(qt5, kt5, lay5, rows5, 'sum', v=vt5), 3)
    res['dense_heat_out_sum_c5'] = _mfma(ms_o, 4.0 * 128 * 128 * D * nv5 * n5 * HEADS)
    heat = kernels.teacher_heat(qt5, kt5, lse_t, lay5, rows5, 'sum')
    blocks5 = pm.column_blocks(lay5, pm.Budget(ratio=0.05))
    sel5 = pm.select_video_blocks(heat[:, :, :nv5], lay5, blocks5, rows5)
    mask5 = pm.dense_block_mask(sel5, lay5)
    lists5 = kernels.index_lists(mask5, lay5)
    kept5 = int(mask5.sum())
    ms = _median_ms(lambda: kernels.block_sparse_attention_lists(qt5, kt5, vt5, lists5, lay5), 3)
    res['sparse_fwd_c5'] = _mfma(ms, 4.0 * 128 * 128 * D * kept5)
    res['sparse_fwd_c5']['kept_blocks'] = kept5
    return res


def _backward(c: dict, kept: int, steps: int, warmup: int) -> int:
    """The block-sparse backward at C2 given the forward's out and LSE (one
    veda_block_sparse_bwd call: stats, dQ and dK/dV kernels); TFLOP/s on 5
    products of 2 * 128^3 per kept block. Timed with two output gradients:
    the one a layer's scatter passes back (N(0, 1) on real rows, 0 on the
    padding rows of partial query tiles, whose outputs the scatter drops:
    the line's value), and N(0, 1) on every row, padding included."""
    from miowtion_amd import kernels, ops
    lay = c['lay']
    lists_t = kernels.index_lists(c['mask'], lay, transpose=True)
    o, lse = kernels.block_sparse_attention_lists(c['qt'], c['kt'], c['vt'], c['lists'], lay,
                                                  return_lse=True)
    dout_all = torch.randn(o.shape, generator=torch.Generator(device='cuda').manual_seed(3),
                           device='cuda').to(torch.bfloat16)
    dout_layer = dout_all * lay.slot_valid.to(dout_all.dtype)[:, None, None]

    def timed(dout):
        def step():
            return ops.block_sparse_bwd(c['qt'], c['kt'], c['vt'], o, dout, lse, None, *c['lists'],
                                        *lists_t, lay.valid_count,
                                        lay.n_tiles - lay.n_video_tiles)
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        ms = sorted(_events_ms(step, max(5, steps)))
        return ms[len(ms) // 2], sum(ms) / len(ms)

    _log(f'bench: backward, warmup {warmup}, timing {steps} steps, layer gradient')
    med, avg = timed(dout_layer)
    _log('bench: backward, gradient on every row')
    med_all, avg_all = timed(dout_all)
    flop = 10.0 * 128 * 128 * D * kept
    tf = lambda ms: round(flop / (ms * 1e-3) / 1e12, 2)
    print(json.dumps({'metric': 'block-sparse attention backward TFLOP/s @C2 (5 products per '
                                'kept block)',
                      'value': tf(med), 'ms_per_step': round(med, 4),
                      'avg_launch_ms': round(avg, 4), 'flop_per_launch': flop,
                      'frac_of_bf16_peak': round(tf(med) / PEAK_BF16_TFLOPS, 4),
                      'kept_blocks': kept,
                      'dout': 'layer gradient: N(0,1) on real rows, 0 on padding rows (the '
                              'scatter drops their outputs)',
                      'dout_every_row': {'value': tf(med_all), 'ms_per_step': round(med_all, 4),
                                         'avg_launch_ms': round(avg_all, 4),
                                         'frac_of_bf16_peak': round(tf(med_all) / PEAK_BF16_TFLOPS,
                                                                    4)}}), flush=True)
    return 0


class _PatternScores:
    """A predictor layer whose kernels run as usual and whose logits are then
    overwritten with the next of the C2 pattern scores (so a full layer walks
    the same block lists the kernel timing cycles through)."""

    def __init__(self, base, scores: list, order):
        self.base, self.scores, self.order = base, scores, order
        self.second_order_rank = base.second_order_rank
        self.count_gain = base.count_gain

    def __call__(self, *args, **kw):
        logits = self.base(*args, **kw)
        return logits.copy_(self.scores[next(self.order) % len(self.scores)])


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=3)
    ap.add_argument('--patterns', type=int, default=PATTERNS,
                    help='distinct seeded C2 block patterns cycled in the timed loop')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--no-dense', action='store_true')
    ap.add_argument('--cpu-budget', type=float, default=20.0)
    ap.add_argument('--only-kernel', action='store_true',
                    help='time the sparse forward only (for rocprofv3 runs)')
    ap.add_argument('--backward', action='store_true',
                    help='time the block-sparse backward at C2 only (for rocprofv3 runs)')
    ap.add_argument('--suite', action='store_true',
                    help='time every kernel of the path at its BASELINE config against its '
                         'roofline and print that JSON instead of the headline line')
    ap.add_argument('--copy-bytes', type=int, default=0,
                    help='first run 3 device-to-device copies of this many bytes: the known-size '
                         'reference that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings')
    args = ap.parse_args()
    if args.gpus != 1:
        print(f'bench.py measures one GPU only (asked for --gpus {args.gpus}); the Veda path '
              'shards by head with no exchange inside the layer, so N GPUs run N independent '
              'shares -- run with --gpus 1', file=sys.stderr)
        return 2
    from miowtion_amd import kernels, mask as pm
    if args.copy_bytes:
        n = args.copy_bytes // 4
        src = torch.ones(n, dtype=torch.float32, device='cuda')
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        _log(f'bench: copied {args.copy_bytes} bytes x 3 (counter calibration)')
    if args.suite:
        print(json.dumps({'suite': suite(), 'gpu': torch.cuda.get_device_name(0)}), flush=True)
        return 0
    _log('bench: building C2 case')
    patterns = 1 if args.backward else args.patterns
    c = build_case(patterns=patterns)
    lay = c['lay']
    kept_each = [int(m.sum()) for m in c['masks']]
    assert all(k == 20340 * HEADS for k in kept_each), kept_each
    kept = kept_each[0]
    if args.backward:
        return _backward(c, kept, args.steps, args.warmup)
    flop = 4.0 * 128 * 128 * D * kept
    # What the kernel executes: the valid keys of every kept block (padding
    # rows of partial key tiles are neither loaded nor multiplied), for all
    # 128 query rows in the P.V products and for the 32-row groups that hold
    # a real row in the Q.K^T products (a group of padding rows, all zero,
    # skips them); averaged over the patterns.
    vc = lay.valid_count.float()
    live_groups = torch.ceil(vc / 32.0)                                     # per query tile
    exec_flop = 0.0
    for m in c['masks']:
        keys_per_row = (m.float() * vc[None, None, :]).sum(-1)              # [H, R]
        exec_flop += float((keys_per_row * (2.0 * 128 * D
                                            + 2.0 * 32 * D * live_groups[None, :])).sum())
    exec_flop /= len(c['masks'])
    dense_flop = 4.0 * c['used'] * c['used'] * HEADS * D
    order = itertools.count()

    def step():
        i = next(order) % patterns
        return kernels.block_sparse_attention_lists(c['qt'], c['kt'], c['vt'], c['all_lists'][i],
                                                    lay)

    _log(f'bench: warmup {args.warmup}')
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    _log(f'bench: timing {args.steps} steps')
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    kernel_ms = sorted(_events_ms(step, max(5, args.steps)))
    k_ms = kernel_ms[len(kernel_ms) // 2]
    k_avg = sum(kernel_ms) / len(kernel_ms)
    achieved = flop / (k_avg * 1e-3) / 1e12
    # the check runs after the timed region on each pattern's own output
    _log('bench: checking every pattern against fp32 rows')
    n = lay.n_tiles
    check = check_rows(c, [kernels.block_sparse_attention_lists(c['qt'], c['kt'], c['vt'], li, lay)
                           for li in c['all_lists']], [0, n // 3, n - 1], [0, HEADS - 1])
    valid = check['verdict'] == 'ok'
    if not valid:
        _log(f"bench: {check['verdict']}: no rate is reported")
    if args.only_kernel:
        print(json.dumps({'metric': METRIC,
                          'value': round(flop / (k_ms * 1e-3) / 1e12, 2) if valid else None,
                          'ms_per_step': round(k_ms, 4), 'avg_launch_ms': round(k_avg, 4),
                          'check': check, 'only_kernel': True}), flush=True)
        return 0 if valid else 1

    _log('bench: +prep and full layer')
    prep_ms = sorted(_events_ms(lambda: c['prep'](next(order) % patterns), 5))[2]
    from miowtion_amd import attention as pa, plan as pplan, predictor as pp, tiling as pt
    layout = pa.PackedLayout((pa.VideoSpan(0, GRID),), c['used'], c['seq_len'])
    clip = pa.ClipTiling(layout, pa.VedaConfig(target_budget=pm.Budget(ratio=RATIO)), 'cuda')
    plan = pplan.TilePlan.uniform('16x9_t37_c2', GRID, pt.TileShape(1, 8, 16), 1, HEADS)
    base = pp.LayerPredictor.random(HEADS, D, std=0.02, generator=torch.Generator().manual_seed(1),
                                    device='cuda', fp8=True)
    # The whole layer on the timed C2 patterns: the predictor's kernels run
    # as in the real layer, then its logits are overwritten with the next C2
    # pattern's scores (one 67 MB device copy more than the real layer), so
    # the sparse forward walks the same lists as the kernel timing above.
    student = pa.SparseStudent(clip, plan, pp.TileScorePredictor(
        [_PatternScores(base, c['all_scores'], order)]))
    layer_ms = sorted(_events_ms(lambda: student(c['q'], c['k'], c['v'], 0), 7))[3]
    # the same layer on its random-weight predictor's own lists
    student_p = pa.SparseStudent(clip, plan, pp.TileScorePredictor([base]))
    layer_pred_ms = sorted(_events_ms(lambda: student_p(c['q'], c['k'], c['v'], 0), 7))[3]

    dense = {}
    if not args.no_dense:
        _log('bench: dense baselines')
        qd, kd, vd = (t[:c['used']].transpose(0, 1)[None] for t in (c['q'], c['k'], c['v']))
        try:
            sdpa = sorted(_events_ms(lambda: torch.nn.functional.scaled_dot_product_attention(
                qd, kd, vd), 3))[1]
            dense['torch_sdpa_ms'] = round(sdpa, 3)
        except RuntimeError as e:  # a backend refusal is reported, not hidden
            dense['torch_sdpa_error'] = str(e)[:200]
        own = sorted(_events_ms(lambda: kernels.dense_attention(c['q'], c['k'], c['v'], c['used']), 3))[1]
        dense['own_dense_ms'] = round(own, 3)
        best = min(v for k_, v in dense.items() if k_.endswith('_ms'))
        dense['speedup_vs_best_dense'] = round(best / k_ms, 2)
        dense['efficiency'] = round(best * (kept / (HEADS * 592 * 592)) / k_ms, 3)

    cpu = None
    if not args.no_cpu_baseline:
        _log('bench: cpu baseline')
        cpu = cpu_baseline(args.cpu_budget)

    line = {
        'metric': METRIC,
        'value': round(flop / (k_ms * 1e-3) / 1e12, 2) if valid else None,
        'unit': 'TFLOP/s (effective, computed blocks)',
        'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup,
        'ms_per_step': round(k_ms, 4),
        'ms_per_step_wall': round(wall_ms, 4),
        'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None,
        'dtype': 'bf16', 'data': 'synthetic (seeded N(0,1) q/k/v, uniform random tile scores)',
        'config': {'workload': 'BASELINE C2: 57,720 tok (37x30x52) x 48 heads x d128, tiles '
                               '(1,8,16) -> 592, keep 0.1 -> 20,340 blocks/head, forced diagonal, '
                               'sparse forward with prebuilt lists',
                   'kept_blocks': kept, 'flop_per_launch': flop,
                   'executed_flop_per_launch': exec_flop,
                   'dense_equivalent_flop': dense_flop},
        'n_patterns': patterns,
        'check': check,
        'ms_per_layer': {'kernel': round(k_ms, 4), 'plus_prep': round(k_ms + prep_ms, 4),
                         'prep': round(prep_ms, 4), 'full_veda_layer': round(layer_ms, 4),
                         'full_veda_layer_predictor_lists': round(layer_pred_ms, 4),
                         'note': 'full_veda_layer: pooling of q and k, predictor, '
                                 'selection, lists, sparse forward reading q, k and v in '
                                 'sequence order with the scatter fused in, on the timed C2 '
                                 'patterns; '
                                 'full_veda_layer_predictor_lists: the same layer on the lists '
                                 'of its random-weight predictor, which are far more alike '
                                 'across query tiles than C2 uniform random scores'},
        'dense_equivalent_tflops': round(dense_flop / (k_ms * 1e-3) / 1e12, 2),
        'dense': dense,
        'roofline': {'bound': 'mfma', 'achieved': round(achieved, 2) if valid else None,
                     'peak': PEAK_BF16_TFLOPS,
                     'unit': 'TFLOP/s',
                     'frac': round(achieved / PEAK_BF16_TFLOPS, 4) if valid else None,
                     'traffic': _traffic(), 'kernel': 'sfwd_kernel (veda_block_sparse_fwd)',
                     'avg_launch_ms': round(k_avg, 4),
                     'achieved_on_executed_flop': round(exec_flop / (k_avg * 1e-3) / 1e12, 2),
                     'frac_on_executed_flop': round(exec_flop / (k_avg * 1e-3) / 1e12
                                                    / PEAK_BF16_TFLOPS, 4)},
        'cpu_baseline': cpu,
    }
    print(json.dumps(line), flush=True)
    return 0 if valid else 1


if __name__ == '__main__':
    sys.exit(main())
