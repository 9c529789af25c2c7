"""Oracle: masked-dense block-sparse attention, dense attention with LSE and
the teacher block heat (CPU torch, fp32 math, test-only).

Restates:
  * block_sparse_attention  -> `miowtion/kernels/reference.py:23-56`
  * _math_attention / dense_attention (math backend)
                            -> `miowtion/h3/attention.py:18-25,80-102`
  * teacher_heat_reference  -> `miowtion/veda/heatmap.py:36-99`
  * zero_order_compensation -> `miowtion/veda/attention.py:591-689`
  * block_sparse_attention_grads -> autograd through
      `miowtion/kernels/reference.py:23-56`, the expected gradients of
      `tests/gpu/test_kernels_gpu.py:200-250` (and a per-tile form of the
      same autograd that scales with the kept blocks)

The reference materialises [H', N, N]; this restatement does the same math
per head and per chunk of query rows so that C2-sized heads fit in memory.
Heads and query rows are independent, so chunking changes no value.
"""

from __future__ import annotations

import math

import torch

from oracle.tiling import TILE, Layout


def block_sparse_attention(q, k, v, block_mask, valid_count, return_lse=False,
                           q_chunk: int = 1024, compute_dtype=torch.float32):
    """q [R*128, H', D], k/v [N, H', D], block_mask [H', R, n] -> out in
    q.dtype (and lse [H', R*128] in compute_dtype, -inf for rows with no
    key). The reference computes in fp32; float64 serves the
    finite-difference checks of the gradients."""
    Rq, H, D = q.shape
    N = k.shape[0]
    scale = 1.0 / math.sqrt(D)
    key_valid = (torch.arange(TILE)[None, :] < valid_count[:, None]).reshape(-1)[:N]
    out = torch.empty(Rq, H, D, dtype=compute_dtype)
    lse = torch.empty(H, Rq, dtype=compute_dtype)
    kf, vf = k.to(compute_dtype), v.to(compute_dtype)
    for h in range(H):
        bm = block_mask[h]
        for q0 in range(0, Rq, q_chunk):
            q1 = min(q0 + q_chunk, Rq)
            rows = torch.arange(q0, q1) // TILE
            tok = bm[rows].repeat_interleave(TILE, 1)[:, :N] & key_valid[None, :]
            s = (q[q0:q1, h].to(compute_dtype) @ kf[:, h].T) * scale
            s = s.masked_fill(~tok, float('-inf'))
            p = torch.softmax(s, -1).nan_to_num(0.0)
            out[q0:q1, h] = p @ vf[:, h]
            lse[h, q0:q1] = torch.logsumexp(s, -1)
    o = out.to(q.dtype)
    return (o, lse) if return_lse else o


def block_sparse_attention_grads(q, k, v, block_mask, valid_count, dout, dlse=None,
                                 dtype=torch.float32):
    """dq, dk, dv of block_sparse_attention for the loss
    sum(out * dout) (+ sum(lse * dlse) over rows that have a key), by
    autograd through the same masked softmax, one head at a time, computed in
    `dtype` (float64 for the finite-difference checks). Returns them in
    `dtype`; a row with no key gets no gradient."""
    Rq, H, D = q.shape
    N = k.shape[0]
    scale = 1.0 / math.sqrt(D)
    key_valid = (torch.arange(TILE)[None, :] < valid_count[:, None]).reshape(-1)[:N]
    grads = [torch.zeros(t.shape, dtype=dtype) for t in (q, k, v)]
    for h in range(H):
        qh, kh, vh = (t[:, h].to(dtype).requires_grad_(True) for t in (q, k, v))
        tok = (block_mask[h].repeat_interleave(TILE, 0)[:Rq].repeat_interleave(TILE, 1)[:, :N]
               & key_valid[None, :])
        s = ((qh @ kh.T) * scale).masked_fill(~tok, float('-inf'))
        p = torch.softmax(s, -1).nan_to_num(0.0)
        loss = ((p @ vh) * dout[:, h].to(dtype)).sum()
        if dlse is not None:
            rows = tok.any(-1)
            loss = loss + (torch.logsumexp(s[rows], -1) * dlse[h, rows].to(dtype)).sum()
        gq, gk, gv = torch.autograd.grad(loss, (qh, kh, vh))
        grads[0][:, h], grads[1][:, h], grads[2][:, h] = gq, gk, gv
    return tuple(grads)


def block_sparse_attention_grads_by_tile(q, k, v, block_mask, valid_count, dout, dlse=None,
                                         dtype=torch.float32):
    """Same gradients as block_sparse_attention_grads, one (head, query tile)
    at a time over only its kept key tiles' valid keys: every row's softmax
    is over exactly those keys, so the restriction is exact, and the key
    gradients of the tiles are summed. Cost scales with the kept blocks, so
    it runs at the BASELINE sizes; block_mask may hold a subset of query
    tiles only if dout covers the same rows (then dk, dv are that subset's
    share)."""
    Rq, H, D = q.shape
    scale = 1.0 / math.sqrt(D)
    vc = valid_count.tolist()
    grads = [torch.zeros(t.shape, dtype=dtype) for t in (q, k, v)]
    for h in range(H):
        kh_all, vh_all = k[:, h].to(dtype), v[:, h].to(dtype)
        for i in range(Rq // TILE):
            cols = torch.nonzero(block_mask[h, i]).flatten().tolist()
            rows = [torch.arange(j * TILE, j * TILE + vc[j]) for j in cols if vc[j] > 0]
            if not rows:
                continue
            idx = torch.cat(rows)
            qi = q[i * TILE:(i + 1) * TILE, h].to(dtype).requires_grad_(True)
            ki = kh_all[idx].requires_grad_(True)
            vi = vh_all[idx].requires_grad_(True)
            s = (qi @ ki.T) * scale
            loss = ((torch.softmax(s, -1) @ vi) * dout[i * TILE:(i + 1) * TILE, h].to(dtype)).sum()
            if dlse is not None:
                loss = loss + (torch.logsumexp(s, -1)
                               * dlse[h, i * TILE:(i + 1) * TILE].to(dtype)).sum()
            gq, gk, gv = torch.autograd.grad(loss, (qi, ki, vi))
            grads[0][i * TILE:(i + 1) * TILE, h] = gq
            grads[1][:, h].index_add_(0, idx, gk)
            grads[2][:, h].index_add_(0, idx, gv)
    return tuple(grads)


def dense_attention(q, k, v, used: int, return_lse=False, q_chunk: int = 1024, rows=None):
    """h3/attention.py 'math' backend: rows [0, used) attend among themselves;
    out zero and lse 0 on padding rows. q/k/v [S, H, D]; lse [S, H].

    rows: optional 1-D index of the query rows to compute (the sampled
    checks at BASELINE sizes); out / lse then hold only those rows, in that
    order, a row at or past `used` giving 0 as a padding row does. Rows are
    independent, so a sample has the same values as the full call."""
    S, H, D = q.shape
    scale = 1.0 / math.sqrt(D)
    if rows is None:
        rows = torch.arange(S)
    rows = torch.as_tensor(rows, dtype=torch.int64)
    out = torch.zeros(rows.numel(), H, D, dtype=torch.float32)
    lse = torch.zeros(rows.numel(), H, dtype=torch.float32)
    real = torch.nonzero(rows < used).flatten()
    kf, vf = k[:used].float(), v[:used].float()
    for h in range(H):
        for c0 in range(0, real.numel(), q_chunk):
            pos = real[c0:c0 + q_chunk]
            s = (q[rows[pos], h].float() @ kf[:, h].T) * scale
            l = torch.logsumexp(s, -1)
            out[pos, h] = torch.exp(s - l[:, None]) @ vf[:, h]
            lse[pos, h] = l
    o = out.to(q.dtype)
    return (o, lse) if return_lse else (o, None)


def teacher_heat(q, k, lse, lay: Layout, q_tiles, reduce='sum', score_dtype=torch.float32):
    """heatmap.py:36-99 -> [H', R, n] fp32.

    score_dtype=torch.bfloat16 reproduces the reference's torch path, whose
    bf16 `bmm` rounds every score; torch.float32 keeps the scores in fp32
    (what an MFMA kernel with fp32 accumulation computes).
    """
    if reduce not in ('max', 'sum'):
        raise ValueError(f"reduce must be 'max' or 'sum': {reduce!r}")
    H, D = q.shape[1], q.shape[2]
    scale = 1.0 / math.sqrt(D)
    valid = lay.slot_valid.bool()
    n = lay.n_tiles
    heat = torch.zeros(H, q_tiles.numel(), n, dtype=torch.float32)
    kf = k.float()
    for ri, r in enumerate(q_tiles.tolist()):
        rows = torch.arange(r * TILE, (r + 1) * TILE)
        row_ok = valid[rows]
        for h in range(H):
            s = q[rows, h].float() @ kf[:, h].T
            s = s.to(score_dtype).float()
            s = s.masked_fill(~valid[None, :], float('-inf'))
            blocks = s.view(TILE, n, TILE)
            l = lse[rows, h]
            if reduce == 'max':
                m = torch.exp(blocks.amax(-1) * scale - l[:, None])
                m = m.masked_fill(~row_ok[:, None], 0.0)
                heat[h, ri] = m.amax(0)
            else:
                p = torch.exp(blocks * scale - l[:, None, None]).sum(-1)
                p = p.masked_fill(~row_ok[:, None], 0.0)
                heat[h, ri] = p.sum(0)
    return heat


def tile_summaries(k, v, valid_count, dtype=torch.float32):
    """Per key tile and head: mean of K over its real rows (sum / max(count,
    1)) and sum of V over them, [n, H', D] in `dtype`
    (compensation_triton.py:80-99 stores bf16; attention.py:654-663 fp32)."""
    n = valid_count.numel()
    H, D = k.shape[1], k.shape[2]
    real = (torch.arange(TILE)[None, :] < valid_count[:, None]).reshape(-1)[:, None, None]
    ks = (k.float() * real).view(n, TILE, H, D).sum(1)
    vs = (v.float() * real).view(n, TILE, H, D).sum(1)
    counts = valid_count.float().clamp(min=1.0)
    return (ks / counts[:, None, None]).to(dtype), vs.to(dtype)


def zero_order_compensation(o_kept, lse_kept, q, k, v, block_mask, valid_count,
                            summary_dtype=torch.float32):
    """attention.py:591-689: every dropped key tile j (mask False, at least
    one real row) stands for one virtual key mean_j(k) with value sum_j(v)
    and weight B_j = its real row count; with the reference lse_kept (0 for
    a row that kept nothing) the kept denominator is 1, so

        out = (o_kept + sum_j p_j sum_j(v)) / (1 + sum_j p_j B_j),
        p_j = exp(q . mean_j(k) / sqrt(D) - lse_kept).

    summary_dtype=torch.bfloat16 rounds the summaries as the reference's
    Triton kernel does (its one deliberate numeric difference)."""
    Rq, H, D = q.shape
    n = valid_count.numel()
    scale = 1.0 / math.sqrt(D)
    kc, vc = tile_summaries(k, v, valid_count, summary_dtype)
    kc, vc = kc.float(), vc.float()
    counts = valid_count.float()
    out = torch.empty(Rq, H, D, dtype=torch.float32)
    rows = torch.arange(Rq) // TILE
    for h in range(H):
        drop = (~block_mask[h][rows]) & (valid_count > 0)[None, :]      # [Rq, n]
        ref = lse_kept[h]
        ref = torch.where(torch.isfinite(ref), ref, torch.zeros_like(ref))
        s = (q[:, h].float() @ kc[:, h].T) * scale
        p = torch.exp(s - ref[:, None]) * drop.float()
        num = p @ vc[:, h]
        den = p @ counts
        out[:, h] = (o_kept[:, h].float() + num) / (1.0 + den)[:, None]
    return out.to(o_kept.dtype)
