"""Pins the oracle's pooling, predictor, fp8 weights, attention and heat
(oracle/predictor.py, oracle/attention.py) against naive loops, library
routines (torch SDPA / softmax) and the reference's known identities."""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oa
from oracle import predictor as op
from oracle import tiling as ot


def _layout(grid=(7, 6, 10), shape='8x4x4', text=90, extra=0):
    target = ot.Span(text + 40, grid, ot.Shape.parse(shape))
    used = target.start + target.rows
    return ot.build_layout([target], used, used + extra)


def test_pooling_matches_naive_masked_stats():
    # reference test_veda_predictor_mask.py:25-37 (+ second moments :200-215)
    lay = _layout()
    x = torch.randn(lay.seq_len, 3, 16, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    tiles = ot.gather_tiles(x, lay, None)
    feats = op.pool_tiles(tiles, lay)
    sq = op.pool_tiles(tiles, lay, 'raw')
    var = op.pool_tiles(tiles, lay, 'central')
    assert feats.shape == (3, lay.n_tiles, 48)
    view = tiles.view(lay.n_tiles, 128, 3, 16).float()
    for j in range(lay.n_tiles):
        n = int(lay.valid_count[j])
        rows = view[j, :n]
        want = torch.cat([rows.mean(0), rows.amax(0), rows.amin(0)], -1)
        torch.testing.assert_close(feats[:, j], want, rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(sq[:, j], (rows * rows).mean(0), rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(var[:, j], rows.var(0, unbiased=False), rtol=1e-4, atol=1e-5)


def test_pooling_empty_tile_is_zero_not_nan():
    # reference test_veda_predictor_mask.py:40-47
    lay = _layout()
    lay.valid_count[0] = 0
    lay.kv_ok[0] = False
    tiles = torch.randn(lay.num_slots, 2, 8).to(torch.bfloat16)
    for second in (None, 'raw', 'central'):
        feats = op.pool_tiles(tiles, lay, second)
        assert torch.isfinite(feats).all() and (feats[:, 0] == 0).all()


def test_untrained_predictor_is_mean_pooled_qk():
    # reference test_veda_predictor_mask.py:50-62: P ~ N(0, 1e-4)
    lay = _layout()
    g = torch.Generator().manual_seed(3)
    q = torch.randn(lay.seq_len, 4, 16, generator=g).to(torch.bfloat16)
    k = torch.randn(lay.seq_len, 4, 16, generator=g).to(torch.bfloat16)
    heads = torch.tensor([0, 2])
    pq = torch.randn(4, 48, 16, generator=g) * 1e-4
    pk = torch.randn(4, 48, 16, generator=g) * 1e-4
    fq = op.pool_tiles(ot.gather_tiles(q, lay, heads), lay)
    fk = op.pool_tiles(ot.gather_tiles(k, lay, heads), lay)
    logits = op.logits(fq, fk, pq, pk, heads)
    mq, mk = fq[..., :16], fk[..., :16]
    torch.testing.assert_close(logits, mq @ mk.transpose(1, 2) / 4.0, rtol=1e-2, atol=1e-2)
    # a dropped residual (mean) term fails: embeddings ~ 0 then
    assert (logits.abs().amax() > 1e-3)


def test_count_and_second_order_terms_by_loops():
    lay = _layout()
    g = torch.Generator().manual_seed(4)
    H, D, r = 2, 8, 3
    fq, fk = torch.randn(H, lay.n_tiles, 3 * D, generator=g), torch.randn(H, lay.n_tiles, 3 * D, generator=g)
    pq, pk = torch.randn(H, 3 * D, D, generator=g), torch.randn(H, 3 * D, D, generator=g)
    sq, vk = torch.rand(H, lay.n_tiles, D, generator=g), torch.rand(H, lay.n_tiles, D, generator=g)
    soq, sok = torch.randn(H, D, r, generator=g), torch.randn(H, D, r, generator=g)
    gain = torch.tensor([0.5, 2.0])
    lc = torch.log(lay.valid_count.clamp(min=1).float())
    heads = torch.tensor([1, 0])
    got = op.logits(fq, fk, pq, pk, heads, gain=gain, log_count=lc, sq_q=sq, var_k=vk, so_q=soq, so_k=sok)
    for hp, h in enumerate(heads.tolist()):
        for i in range(lay.n_tiles):
            for j in range(lay.n_tiles):
                qh = sum(fq[hp, i, c] * pq[h, c] for c in range(3 * D)) + fq[hp, i, :D]
                kh = sum(fk[hp, j, c] * pk[h, c] for c in range(3 * D)) + fk[hp, j, :D]
                u = sum(sq[hp, i, c] * soq[h, c] for c in range(D))
                w = sum(vk[hp, j, c] * sok[h, c] for c in range(D))
                want = (qh @ kh) / math.sqrt(D) + gain[h] * lc[j] + u @ w
                assert abs(float(got[hp, i, j] - want)) < 1e-3 * (1 + abs(float(want)))


def test_count_term_adds_exactly_log_b_at_init():
    """The reference's identity (tests/unit/test_veda_predictor_mask.py:325):
    with the gain at its initial 1 the count term adds log B_j of the KEY
    tile j to every row, nothing else (a term indexed by the query tile, or
    a dropped gain, fails)."""
    lay = _layout()
    assert len(set(lay.valid_count.tolist())) > 2        # counts differ per tile
    g = torch.Generator().manual_seed(8)
    D = 16
    q = torch.randn(lay.seq_len, 4, D, generator=g).to(torch.bfloat16)
    k = torch.randn(lay.seq_len, 4, D, generator=g).to(torch.bfloat16)
    heads = torch.tensor([0, 2])
    fq = op.pool_tiles(ot.gather_tiles(q, lay, heads), lay)
    fk = op.pool_tiles(ot.gather_tiles(k, lay, heads), lay)
    pq, pk = (torch.randn(4, 3 * D, D, generator=g) * 1e-2 for _ in range(2))
    plain = op.logits(fq, fk, pq, pk, heads)
    lc = torch.log(lay.valid_count.clamp(min=1).float())
    counted = op.logits(fq, fk, pq, pk, heads, gain=torch.ones(4), log_count=lc)
    delta = counted - plain
    torch.testing.assert_close(delta, lc.expand_as(delta), rtol=1e-5, atol=1e-5)


def test_exact_warm_start_equals_the_diagonal_cumulant():
    """The reference's identity (tests/unit/test_veda_predictor_mask.py:240):
    with the base projections zero and the full-rank second-order head at
    its exact warm start (so_q = so_k = I sqrt(1 / 2D), predictor.py:232-249)
    the logits are mean_q . mean_k / sqrt(D) + E[q^2] . Var(k) / (2D), with
    the tile statistics taken here by per-tile loops over the real rows."""
    lay = _layout()
    g = torch.Generator().manual_seed(9)
    D = 16
    q = torch.randn(lay.seq_len, 4, D, generator=g).to(torch.bfloat16)
    k = torch.randn(lay.seq_len, 4, D, generator=g).to(torch.bfloat16)
    heads = torch.tensor([1, 3])
    qt, kt = ot.gather_tiles(q, lay, heads), ot.gather_tiles(k, lay, heads)
    zero = torch.zeros(4, 3 * D, D)
    eye = torch.eye(D).expand(4, D, D) * math.sqrt(0.5 / D)
    got = op.logits(op.pool_tiles(qt, lay), op.pool_tiles(kt, lay), zero, zero, heads,
                    sq_q=op.pool_tiles(qt, lay, 'raw'), var_k=op.pool_tiles(kt, lay, 'central'),
                    so_q=eye, so_k=eye)
    n = lay.n_tiles
    mq, mk, sq, vk = (torch.zeros(2, n, D) for _ in range(4))
    for j in range(n):
        c = int(lay.valid_count[j])
        if not c:
            continue
        rq = qt.view(n, 128, 2, D)[j, :c].float()
        rk = kt.view(n, 128, 2, D)[j, :c].float()
        mq[:, j], mk[:, j] = rq.mean(0), rk.mean(0)
        sq[:, j] = (rq * rq).mean(0)
        vk[:, j] = ((rk - rk.mean(0)) ** 2).mean(0)
    want = mq @ mk.transpose(1, 2) / math.sqrt(D) + sq @ vk.transpose(1, 2) / (2 * D)
    torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-5)


def test_fp8_per_head_quantisation():
    # bundle.py:71-93: per-head amax maps to 448, values round-trip within e4m3
    g = torch.Generator().manual_seed(5)
    w = torch.randn(3, 384, 128, generator=g) * 0.02
    w[1] *= 10
    vals, scale = op.quantize_fp8(w)
    assert vals.dtype == torch.float8_e4m3fn and scale.shape == (3,)
    torch.testing.assert_close(scale, w.abs().amax(dim=(1, 2)) / 448.0)
    assert torch.equal(vals.float().abs().amax(dim=(1, 2)), torch.full((3,), 448.0))
    deq = op.dequantize_fp8(vals, scale, torch.float32)
    # e4m3 has 3 mantissa bits: relative error <= 2^-4 for normal values
    big = w.abs() > scale.view(-1, 1, 1) * 2 ** -6
    rel = ((deq - w).abs() / w.abs())[big]
    assert rel.max() <= 2 ** -4 + 1e-6
    assert op.dequantize_fp8(vals, scale).dtype == torch.bfloat16


def _qkv(n, heads, dim, seed=0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(n, heads, dim, generator=g).to(torch.bfloat16) for _ in range(3)]


def test_keep_all_sparse_equals_sdpa_with_key_mask():
    lay = _layout(extra=20)
    H = 2
    q, k, v = _qkv(lay.seq_len, H, 32)
    qt, kt, vt = (ot.gather_tiles(t, lay, None) for t in (q, k, v))
    mask = torch.ones(H, lay.n_tiles, lay.n_tiles, dtype=torch.bool)
    out, lse = oa.block_sparse_attention(qt, kt, vt, mask, lay.valid_count, return_lse=True, q_chunk=128)
    keyv = lay.slot_valid.bool()
    ref = F.scaled_dot_product_attention(qt.float().transpose(0, 1), kt.float().transpose(0, 1),
                                         vt.float().transpose(0, 1), attn_mask=keyv[None, None, :])
    torch.testing.assert_close(out.float(), ref.transpose(0, 1).to(torch.bfloat16).float(),
                               rtol=0, atol=1e-2)
    s = torch.einsum('qhd,khd->hqk', qt.float(), kt.float()) / math.sqrt(32)
    torch.testing.assert_close(lse, torch.logsumexp(s.masked_fill(~keyv, float('-inf')), -1))


def test_sparse_rows_by_python_loop_and_empty_rows():
    lay = _layout(grid=(4, 6, 10), shape='2x8x8')
    H, D = 2, 16
    q, k, v = _qkv(lay.seq_len, H, D, seed=1)
    qt, kt, vt = (ot.gather_tiles(t, lay, None) for t in (q, k, v))
    g = torch.Generator().manual_seed(9)
    mask = torch.rand(H, lay.n_tiles, lay.n_tiles, generator=g) < 0.5
    mask[0, 0] = False  # a query tile with no key at all
    out, lse = oa.block_sparse_attention(qt, kt, vt, mask, lay.valid_count, return_lse=True, q_chunk=96)
    assert (out[:128, 0] == 0).all() and torch.isinf(lse[0, :128]).all()
    for h in range(H):
        for row in range(0, lay.num_slots, 37):
            keys = [c for c in range(lay.num_slots)
                    if mask[h, row // 128, c // 128] and (c % 128) < lay.valid_count[c // 128]]
            if not keys:
                continue
            s = torch.stack([(qt[row, h].float() * kt[c, h].float()).sum() for c in keys]) / math.sqrt(D)
            p = torch.exp(s - s.max())
            p = p / p.sum()
            want = sum(p[i] * vt[c, h].float() for i, c in enumerate(keys))
            torch.testing.assert_close(out[row, h].float(), want.to(torch.bfloat16).float(), rtol=0, atol=1e-2)
            torch.testing.assert_close(lse[h, row], torch.logsumexp(s, 0), rtol=1e-5, atol=1e-5)


def test_dense_attention_matches_sdpa_and_zero_padding():
    S, used, H, D = 300, 270, 2, 32
    q, k, v = _qkv(S, H, D, seed=2)
    out, lse = oa.dense_attention(q, k, v, used, return_lse=True, q_chunk=100)
    ref = F.scaled_dot_product_attention(q[:used].float().transpose(0, 1), k[:used].float().transpose(0, 1),
                                         v[:used].float().transpose(0, 1))
    torch.testing.assert_close(out[:used].float(), ref.transpose(0, 1).to(torch.bfloat16).float(), rtol=0, atol=1e-2)
    assert (out[used:] == 0).all() and (lse[used:] == 0).all()
    s = torch.einsum('qhd,khd->hqk', q[:used].float(), k[:used].float()) / math.sqrt(D)
    torch.testing.assert_close(lse[:used], torch.logsumexp(s, -1).T)
    # a sample of rows (the form the BASELINE-size GPU checks use): the same
    # values as the full call, padding rows 0, in the order asked
    rows = torch.tensor([269, 0, 280, 131, 299, 1])
    o_s, l_s = oa.dense_attention(q, k, v, used, return_lse=True, q_chunk=4, rows=rows)
    assert torch.equal(o_s, out[rows]) and torch.equal(l_s, lse[rows])
    assert (o_s[[2, 4]] == 0).all() and (l_s[[2, 4]] == 0).all()


@pytest.mark.parametrize('reduce', ['max', 'sum'])
def test_heat_matches_brute_force_from_dense_softmax(reduce):
    # reference test_veda_heatmap_attention.py:50-74 and :383-407
    target = ot.Span(70, (6, 6, 12), ot.Shape(2, 4, 16))
    used = target.start + target.rows
    lay = ot.build_layout([target], used, used + 20)
    q, k, v = _qkv(lay.seq_len, 2, 32)
    _, lse = oa.dense_attention(q, k, v, lay.used, return_lse=True)
    heads = torch.tensor([0, 1])
    qt, kt = (ot.gather_tiles(t, lay, heads) for t in (q, k))
    lse_t = ot.gather_lse(lse, lay, heads)
    rows = torch.tensor([0, 2, lay.n_tiles - 1])
    s = torch.einsum('qhd,khd->hqk', q[:used].float(), k[:used].float()) / 32 ** 0.5
    probs = torch.softmax(s, -1)
    for dtype, tol in ((torch.float32, 1e-4), (torch.bfloat16, 3e-2)):
        heat = oa.teacher_heat(qt, kt, lse_t, lay, rows, reduce, score_dtype=dtype)
        for ri, r in enumerate(rows.tolist()):
            for j in range(lay.n_tiles):
                qi, kj = lay.perm[r * 128:(r + 1) * 128], lay.perm[j * 128:(j + 1) * 128]
                qi, kj = qi[qi >= 0], kj[kj >= 0]
                if not qi.numel() or not kj.numel():
                    assert (heat[:, ri, j] == 0).all()
                    continue
                blk = probs[:, qi][:, :, kj]
                want = blk.amax(dim=(1, 2)) if reduce == 'max' else blk.sum((1, 2))
                torch.testing.assert_close(heat[:, ri, j], want, rtol=tol, atol=1e-6)
        if reduce == 'sum':  # every row's probabilities sum to 1
            torch.testing.assert_close(heat.sum(-1), lay.valid_count[rows].float().expand(2, -1),
                                       rtol=tol, atol=tol)
