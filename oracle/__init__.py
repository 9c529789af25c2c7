"""CPU oracle of the Veda sparse-attention hot path (TEST INFRASTRUCTURE ONLY).

This package restates, in plain CPU torch, the reference algorithms of
veda-sparse/Miowtion's Veda path. It is the checker the HIP kernels are
measured against and nothing else: only `tests/`, `__graft_entry__.smoke()`
and the `cpu_baseline` leg of `bench.py` may import it. The product package
`miowtion_amd` never imports it and has no CPU fallback.

Modules and what pins each function (a check that a plausible mistake --
a dropped term, a wrong index, a transposed operand -- would fail):

  tiling     span_tiles / build_tile_layout (`miowtion/veda/tiling.py:43-312`)
             pinned by the reference's known answers (36 shapes, 333 / 330
             tiles, padded (40,24,44), 3D-box membership, contiguous cut),
             bijection + valid-prefix invariants, and a brute-force
             per-slot recomputation from the grid on small spans.
  mask       Budget / split_budget / Bresenham / select_video_blocks /
             dense_block_mask (`miowtion/veda/mask.py:38-317`) pinned by the
             known answer 0.1*292^2/330, the Bresenham mean bound, the
             selection rules (diagonal kept and costs budget, global rows and
             columns dense), and `torch.topk` (a library routine) on scores
             with distinct values.
  lists      index_lists / _pack_lists (`miowtion/kernels/fa4.py:266-296`)
             pinned by rebuilding the mask from the lists and sortedness.
  predictor  pool_tiles (+ second moments), LayerPredictor.embed/forward, the
             fp8 bundle (de)quantisation (`miowtion/veda/predictor.py:82-338`,
             `miowtion/veda/bundle.py:71-93`) pinned by naive per-tile loops,
             the empty-tile rule, the untrained-predictor identity and e4m3
             round-trip bounds.
  attention  masked-dense block-sparse attention + LSE
             (`miowtion/kernels/reference.py:23-56`) and dense attention with
             LSE (`miowtion/h3/attention.py:18-102`) pinned by keep-all ==
             torch SDPA, a per-row Python loop on tiny inputs and chunk
             invariance.
  heat       teacher_heat_reference (`miowtion/veda/heatmap.py:36-99`),
             in the reference's bf16-score form and in an fp32-score form,
             pinned by brute force from dense softmax and the row-mass
             identity sum_j heat[i, j] = valid_count[i].

No function here is "parity unpinned".

Tie order of the top-k: the reference calls `torch.topk`, whose order among
exactly equal scores is backend-defined (CPU and CUDA differ, and CPU is not
stable). The oracle fixes it as "higher score first, lower column first on
equal scores" (a stable descending sort); on scores whose values at the cut
are distinct this is exactly `torch.topk`'s result, which the tests check.
"""
