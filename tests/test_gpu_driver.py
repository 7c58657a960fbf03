"""The driver and the step's options on the GPU, against the oracle:

  - a zero-width root box left open is a degenerate leaf: 'unknown' with
    batched_open_degenerate = 1 and an empty worklist
    (verify_graph.py:13366-13369, 13452-13464);
  - a failure inside alpha-CROWN keeps the CROWN bound
    (verify_graph.py:12962-12969);
  - the clip loop (input_split_batched_clip_iters, verify_graph.py:
    13036-13081) against the oracle's on the same boxes.
"""
import os

import pytest
import torch

from oracle import ref_bab as rbab
from vibecheck_amd import onnx_net, vnnlib
from vibecheck_amd import verify_graph as vg
from vibecheck_amd import workloads as wk
from vibecheck_amd.spec import VNNSpec

from test_formats import GOLD, NET, WITNESS_X
import _util

pytestmark = pytest.mark.gpu
F32 = torch.float32


def test_zero_width_root_box_is_a_degenerate_leaf(gpu):
    """prop_2 of the bundled ACAS-Xu example is violated at the README's
    witness: a zero-width box there cannot close, and it has no width to
    split."""
    gg = onnx_net.load_onnx(NET, device=gpu, dtype=F32)
    p2 = vnnlib.load_vnnlib(os.path.join(GOLD, 'prop_2.vnnlib'))
    spec = VNNSpec(WITNESS_X, WITNESS_X, p2.disjuncts)
    settings = {'input_split_crown_intermediate': True, 'total_timeout': 60.0}
    verdict, det = vg._input_split_batched(None, spec, settings, gg, gpu, F32)
    print(verdict, det)
    assert verdict == 'unknown'
    assert det['phase'] == 'batched_timeout'
    assert det['batched_open_degenerate'] == 1 and det['batched_worklist_left'] == 0
    assert det['batched_n_leaves'] == 1 and det['batched_n_iters'] == 1


def test_alpha_failure_keeps_the_crown_bound(gpu, monkeypatch):
    gg = wk.acas_gg(device=gpu, dtype=F32)
    xl, xh = wk.acas_boxes(2048, seed=3, device=gpu, dtype=F32)
    c, r = (xl + xh) / 2, (xh - xl) / 2
    xl, xh = (c - 3 * r).contiguous(), (c + 3 * r).contiguous()
    se_c, dq = _util.spec_for(5, dtype=F32)
    se = {k: (w.to(gpu), b) for k, (w, b) in se_c.items()}
    table = vg.DisjunctTable(dq, gpu)
    plain = vg.bab_step(xl, xh, gg, se, table, alpha_iters=0, clip_iters=2)

    def broken(*a, **k):
        raise RuntimeError('alpha-CROWN failed')
    monkeypatch.setattr(vg, '_run_alpha_crown_inputsplit_batched', broken)
    got = vg.bab_step(xl, xh, gg, se, table, alpha_iters=5, alpha_all=True, clip_iters=2)
    assert got['n_alpha_leaves'] > 0 and got['n_alpha_iters'] == 0
    assert torch.equal(got['lb'], plain['lb'])
    assert torch.equal(got['closed'], plain['closed'])
    assert torch.equal(got['xl_split'], plain['xl_split'])


def _halfspaces(B, Q, n, seed):
    """Boxes and halfspaces A x + b <= 0 whose minimum over each box is just
    below 0 (-0.01 * |A|_1 * width): the clips cut, and cut again once
    another halfspace has shrunk the box."""
    g = torch.Generator().manual_seed(seed)
    xl = torch.rand(B, n, generator=g) * 2 - 1
    xh = xl + 0.05 + torch.rand(B, n, generator=g) * 0.5
    A = torch.randn(B, Q, n, generator=g)
    mn = (A.clamp(min=0) * xl.unsqueeze(1) + A.clamp(max=0) * xh.unsqueeze(1)).sum(-1)
    b = -mn - 0.01 * (A.abs() * (xh - xl).unsqueeze(1)).sum(-1)
    return xl, xh, A, b


@pytest.mark.parametrize('n_disj', [1, 2])
def test_clip_loop_parity(gpu, n_disj):
    # two halfspaces per disjunct: more, and nearly every intersection is empty
    B, Q, n = 4096, 2 * n_disj, 5
    xl, xh, A, b = _halfspaces(B, Q, n, seed=3 + n_disj)
    dq = {0: [0, 1]} if n_disj == 1 else {0: [0, 1], 1: [2, 3]}
    table = vg.DisjunctTable(dq, gpu)
    args = [t.to(gpu).contiguous() for t in (xl, xh, A, b)]
    widths = []
    for clip_iters in (1, 2, 6):
        rl, rh_, rf = rbab.clip_iterated(xl, xh, A, b, dq, clip_iters)
        gl, gh, gf = vg._clip_iterated(*args, table, clip_iters)
        assert torch.equal(gf.cpu(), rf), clip_iters
        # the feasible leaves' boxes (the others are dropped), each
        # coordinate within the rounding its clip thresholds carry
        tol = _util.clip_tolerance(A[rf], b[rf], xl[rf], xh[rf])
        for got, ref, k in ((gl, rl, 'xl'), (gh, rh_, 'xh')):
            err = (got.cpu()[rf].double() - ref[rf].double()).abs()
            assert bool((err <= tol).all()), (clip_iters, k, int((err > tol).sum()))
        widths.append(float((rh_ - rl)[rf].sum()))
        print(f'{n_disj} disjunct(s), clip_iters={clip_iters}: feasible {int(rf.sum())}, '
              f'total width {widths[-1]:.4f}', flush=True)
    # the loop tightens beyond one clip on this batch
    assert widths[1] < widths[0] and widths[2] <= widths[1]


def test_bab_step_clip_iters_parity(gpu):
    gg_c = wk.acas_gg(dtype=F32)
    gg_g = wk.acas_gg(device=gpu, dtype=F32)
    xl, xh = wk.acas_boxes(4096, seed=7)
    c, r = (xl + xh) / 2, (xh - xl) / 2
    xl, xh = c - 4 * r, c + 4 * r
    se_c, dq = _util.spec_for(5, dtype=F32)
    se_g = {k: (w.to(gpu), b) for k, (w, b) in se_c.items()}
    ref = rbab.bab_step(xl, xh, gg_c, se_c, dq, clip_iters=3)
    got = vg.bab_step(xl.to(gpu), xh.to(gpu), gg_g, se_g, vg.DisjunctTable(dq, gpu),
                      clip_iters=3)
    assert torch.equal(got['closed'].cpu(), ref['closed'])
    assert torch.equal(got['unclosed'].cpu(), ref['unclosed'])
    assert torch.equal(got['feasible'].cpu(), ref['feasible'])
    assert torch.equal(got['ax'].cpu(), ref['ax'])
    fidx = ref['unclosed'][ref['feasible']]
    tol = _util.clip_tolerance(ref['A'][fidx], ref['acc'][fidx], xl[fidx], xh[fidx])
    for k in ('xl_split', 'xh_split'):
        err = (got[k].cpu().double() - ref[k].double()).abs()
        assert bool((err <= tol).all()), (k, int((err > tol).sum()))


def test_native_rounds_from_two_host_threads(gpu):
    """Two host threads run BaB rounds at once, each on its own stream: the
    counts the native round polls and alpha's stop word are per thread, and
    the domain-queue counters per call, so each thread's round equals the
    same round run alone."""
    import threading
    gg = wk.acas_gg(device=gpu, dtype=F32)
    se_c, dq = _util.spec_for(5, dtype=F32)
    se = {k: (w.to(gpu), b) for k, (w, b) in se_c.items()}
    batches = []
    for seed in (11, 12):
        xl, xh = wk.acas_boxes(3000, seed=seed, device=gpu, dtype=F32)
        c, r = (xl + xh) / 2, (xh - xl) / 2
        batches.append(((c - 3 * r).contiguous(), (c + 3 * r).contiguous()))
    kw = dict(alpha_iters=8, alpha_all=True, alpha_lr=0.1)
    alone = [vg.bab_step(xl, xh, gg, se, vg.DisjunctTable(dq, gpu), **kw)
             for xl, xh in batches]
    got = [None, None]
    errors = []

    def run(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for _ in range(3):
                    got[i] = vg.bab_step(*batches[i], gg, se, vg.DisjunctTable(dq, gpu), **kw)
            s.synchronize()
        except Exception as e:  # reported below
            errors.append(repr(e))
    ts = [threading.Thread(target=run, args=(i,)) for i in (0, 1)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    assert not errors, errors
    for a, b in zip(alone, got):
        assert b is not None
        assert torch.equal(a['closed'], b['closed']) and torch.equal(a['lb'], b['lb'])
        assert torch.equal(a['unclosed'], b['unclosed'])
        assert a['n_alpha_iters'] == b['n_alpha_iters']
