"""An fc in the N-D batched MatMul form (an ONNX MatMul on a (3, 7) input
with W (16, 7), output (3, 16); verify_zono_bnb.py:3145-3168 and
4382-4401) on the GPU against the oracle: zonotope bounds, centre and
generators, CROWN intermediate bounds, the spec bound with its input
linearization, and one BaB step.  The reference's interval forward has no
N-D form (it fails on the shapes), and the drop-in raises there; a width
that does not chain raises before any launch.  Tolerances as in
test_gpu_parity."""
import copy

import pytest
import torch

from oracle import ref_bab as rbab
from oracle import ref_bound as rb
from vibecheck_amd import verify_graph as vg
from vibecheck_amd import verify_zono_bnb as vz

import _util
from test_gpu_parity import assert_bounds, assert_interval, cpu, d64, spec_scale

pytestmark = pytest.mark.gpu
F32 = torch.float32


def _boxes(B, seed, r=0.1):
    g = torch.Generator().manual_seed(seed)
    c = torch.rand(B, 21, generator=g) * 2 - 1
    rad = torch.rand(B, 21, generator=g) * r + 0.005
    return c - rad, c + rad


def _nets(gpu, seed=3):
    gg_c = _util.nd_mlp_gg(seed=seed, dtype=F32)
    return gg_c, _util.to_dev(gg_c, gpu)


def test_nd_fc_zonotope(gpu):
    gg_c, gg_g = _nets(gpu)
    xl, xh = _boxes(200, seed=1)
    ref, (rc, rG) = rb.zono_forward_batched(xl, xh, gg_c)
    ref64, _ = rb.zono_forward_batched(xl.double(), xh.double(), d64(gg_c))
    got, (gc, gG) = vz._forward_zonotope_graph_batched(xl.to(gpu), xh.to(gpu), gg_g, gpu, F32)
    for L in ref:
        assert_interval(got[L], ref[L], f'nd zono L{L}', ref64=ref64[L])
    assert gG.shape == rG.shape, (gG.shape, rG.shape)
    assert_bounds(gc, rc, 'nd zono centre', scale=rG.abs().sum(-1))
    rad = rG.abs().sum(-1, keepdim=True).double().expand_as(rG)
    assert_bounds(gG, rG, 'nd zono generators', scale=rad)


def test_nd_fc_crown_and_spec_bound(gpu):
    gg_c, gg_g = _nets(gpu, seed=4)
    xl, xh = _boxes(128, seed=2)
    sb, _ = rb.zono_forward_batched(xl, xh, gg_c)
    sb64 = {L: (a.double(), b.double()) for L, (a, b) in sb.items()}
    tight = rb.crown_intermediate_batched(gg_c, xl, xh, sb=sb)
    tight64 = rb.crown_intermediate_batched(d64(gg_c), xl.double(), xh.double(), sb=sb64)
    sbg = {L: (a.to(gpu), b.to(gpu)) for L, (a, b) in sb.items()}
    got = vz._crown_intermediate_batched(gg_g, xl.to(gpu), xh.to(gpu), gpu, F32, sb=sbg)
    for L in tight:
        assert_interval(got[L], tight[L], f'nd crown L{L}', ref64=tight64[L])
    se_c, _ = _util.spec_for(3, dtype=F32)
    se_g = {k: (w.to(gpu), b) for k, (w, b) in se_c.items()}
    lb, A, acc = rb.spec_backward_batched(tight, xl, xh, gg_c, se_c, return_input_linear=True)
    lb64, A64, acc64 = rb.spec_backward_batched(d64(tight), xl.double(), xh.double(),
                                                d64(gg_c), d64(se_c), return_input_linear=True)
    tg = {L: (a.to(gpu), b.to(gpu)) for L, (a, b) in tight.items()}
    glb, gA, gacc = vz._spec_backward_graph_batched(tg, xl.to(gpu), xh.to(gpu), gg_g, se_g,
                                                    gpu, F32, return_input_linear=True)
    s = spec_scale(A, acc, xl, xh)
    assert_bounds(glb, lb, 'nd spec lb', ref64=lb64, scale=s)
    assert_bounds(gacc, acc, 'nd spec acc', ref64=acc64, scale=s)
    assert_bounds(gA, A, 'nd spec A', ref64=A64, scale=A.abs().amax(-1, keepdim=True))


def test_nd_fc_bab_step(gpu):
    """The BaB step on the N-D net (layer-wise path) against the oracle's:
    closure exact outside the tolerance band of 0, and with no flip the
    unclosed leaves, feasibility and split dimensions exact."""
    gg_c, gg_g = _nets(gpu, seed=5)
    xl, xh = _boxes(512, seed=4, r=0.02)
    se_c, dq = _util.spec_for(3, dtype=F32)
    se_g = {k: (w.to(gpu), b) for k, (w, b) in se_c.items()}
    ref = rbab.bab_step(xl, xh, gg_c, se_c, dq)
    got = vg.bab_step(xl.to(gpu), xh.to(gpu), gg_g, se_g, vg.DisjunctTable(dq, gpu))
    near0 = (ref['lb'].double().abs()
             <= 1e-6 + 1e-5 * spec_scale(ref['A'], ref['acc'], xl, xh)).any(1)
    d = cpu(got['closed']) != ref['closed']
    print(f'nd step: closed gpu {int(got["closed"].sum())} oracle {int(ref["closed"].sum())}, '
          f'near-zero {int(near0.sum())}, differing {int(d.sum())}')
    assert 0 < int(ref['closed'].sum()) < 512
    assert not bool((d & ~near0).any())
    if not bool(d.any()):
        assert torch.equal(cpu(got['unclosed']), ref['unclosed'])
        assert torch.equal(cpu(got['feasible']), ref['feasible'])
        assert torch.equal(cpu(got['ax']), ref['ax'])


def test_nd_fc_refusals(gpu):
    """Interval forward: NotImplementedError (the reference's mid @ W.T
    has no N-D form).  Backward without out_shape_nd: NotImplementedError
    (the reference's backward takes the N-D form only with it).  A width
    that does not chain: ValueError before any launch.  alpha-CROWN's
    gradient sweep takes fc/relu chains without the N-D form:
    NotImplementedError."""
    gg_c, gg_g = _nets(gpu, seed=6)
    xl, xh = (t.to(gpu) for t in _boxes(8, seed=5))
    with pytest.raises(NotImplementedError):
        vz._ibp_forward_graph_batched(xl, xh, gg_g, gpu, F32)
    se_c, _ = _util.spec_for(3, dtype=F32)
    se_g = {k: (w.to(gpu), b) for k, (w, b) in se_c.items()}
    no_out = _util.to_dev(_util.nd_mlp_gg(seed=6, dtype=F32, out_nd=False), gpu)
    sb, _ = vz._forward_zonotope_graph_batched(xl, xh, no_out, gpu, F32)
    with pytest.raises(NotImplementedError):
        vz._spec_backward_graph_batched(sb, xl, xh, no_out, se_g, gpu, F32)
    bad = copy.copy(gg_g)
    bad['ops'] = [dict(op) for op in gg_g['ops']]
    del bad['ops'][0]['in_shapes_nd']
    with pytest.raises(ValueError):
        vz._forward_zonotope_graph_batched(xl, xh, bad, gpu, F32)
    with pytest.raises(ValueError):
        vz._spec_backward_graph_batched(sb, xl, xh, bad, se_g, gpu, F32)
    with pytest.raises(ValueError):
        vz._forward_zonotope_graph_batched(xl[:, :20], xh[:, :20], gg_g, gpu, F32)
    with pytest.raises(NotImplementedError):
        vz._run_alpha_crown_inputsplit_batched(xl, xh, gg_g, se_g, gpu, F32, n_iters=3)
