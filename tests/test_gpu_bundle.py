"""A loaded predictor bundle on the GPU: an e4m3 bundle kept resident as
e4m3 + per-head scale gives the same logit bits as its bf16 materialisation
(the reference's resident form, miowtion/veda/bundle.py:296-312), and a
SparseStudent driven by a bundle's plan and predictor reproduces the one
built from the same weights in memory."""

import pytest
import torch

from miowtion_amd import attention as pa
from miowtion_amd import bundle
from miowtion_amd import geometry
from miowtion_amd import kernels
from miowtion_amd import mask as pm
from miowtion_amd import plan as pplan
from miowtion_amd import tiling as pt
from tests import helpers

pytestmark = pytest.mark.gpu


def test_fp8_resident_logits_equal_bf16_materialised(tmp_path):
    w = {}
    g = torch.Generator().manual_seed(0)
    for i in range(2):
        for name in ('proj_q', 'proj_k'):
            w[f'layers.{i}.{name}'] = torch.randn(4, 384, 128, generator=g) * 0.02
    plans = pplan.PlanTable([pplan.TilePlan.uniform(geometry.geometry_from_latent_t('16:9', 37),
                                                    pt.TileShape(1, 8, 16), 2, 4)])
    path = str(tmp_path / 'b.safetensors')
    bundle.save(path, w, plans, num_layers=2, num_heads=4, head_dim=128, keep_ratio=0.1,
                source='t', source_weights='live', step=0, dtype=torch.float8_e4m3fn)
    b8 = bundle.load(path, 'cuda')
    b16 = bundle.load(path, 'cuda', keep_fp8=False)
    assert b8.predictor.layers[0].proj_q.values.dtype == torch.float8_e4m3fn
    assert b16.predictor.layers[0].proj_q.values.dtype == torch.bfloat16
    fq = torch.randn(4, 37, 384, generator=g).cuda()
    fk = torch.randn(4, 37, 384, generator=g).cuda()
    heads = torch.arange(4, device='cuda')
    for layer in range(2):
        a = b8.predictor.layers[layer](fq, fk, heads)
        c = b16.predictor.layers[layer](fq, fk, heads)
        assert torch.equal(a, c)


def test_sparse_student_from_a_bundle(tmp_path):
    spec = helpers.small_layout(grid=(4, 16, 16), shape='2x8x8', text=0, extra=0)
    spans, used, seq_len, shape = spec
    grid = spans[0][1]
    H = 4
    plan = pplan.TilePlan('t', grid, [pt.TileShape.parse(shape)], [[0] * H])
    pred = bundle.random_bundle(1, H, 128, [], 0.5, seed=2, device='cuda').predictor
    path = str(tmp_path / 'b.safetensors')
    bundle.save(path, bundle.state_dict(pred), pplan.PlanTable([plan]), num_layers=1, num_heads=H,
                head_dim=128, keep_ratio=0.5, source='t', source_weights='live', step=0,
                dtype=torch.bfloat16)
    loaded = bundle.load(path, 'cuda')
    layout = pa.PackedLayout((pa.VideoSpan(spans[0][0], grid),), used, seq_len)
    q, k, v = (t.cuda() for t in helpers.qkv(seq_len, H, 128, seed=4))
    outs = []
    for p_, table in ((pred, plan), (loaded.predictor, loaded.plans.plans['t'])):
        clip = pa.ClipTiling(layout, pa.VedaConfig(target_budget=loaded.target_budget), 'cuda')
        outs.append(pa.SparseStudent(clip, table, p_)(q, k, v, 0))
    assert loaded.target_budget == pm.Budget(ratio=0.5)
    assert torch.equal(outs[0], outs[1])
