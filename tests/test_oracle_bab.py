"""Pins the CPU oracle's BaB-step logic (oracle/ref_bab.py): closure,
halfspace clipping, widest-axis choice, bisection, compaction order, LIFO
chunk worklist, query dedup.  Hand-computed cases and brute force."""
import numpy as np
import torch

from oracle import ref_bab as rbab
from oracle import ref_bound as rb
from vibecheck_amd import workloads as wk
from vibecheck_amd.spec import (Conjunct, Constraint, PairwiseConstraint,
                                VNNSpec, dedup_queries)

import _util

DT = torch.float64


def _t(v, dt=DT):
    return torch.tensor(v, dtype=dt)


def test_closure_any_within_all_across():
    lb = _t([[1.0, -1.0, -1.0], [-1.0, 2.0, 2.0], [-1.0, -1.0, -1.0],
             [0.0, 3.0, 0.0]])
    one = {0: [0, 1, 2]}
    assert rbab.closure(lb, one).tolist() == [True, True, False, True]
    each = {0: [0], 1: [1], 2: [2]}
    assert rbab.closure(lb, each).tolist() == [False, False, False, False]
    two = {0: [0, 1], 1: [2]}
    assert rbab.closure(lb, two).tolist() == [False, True, False, False]
    lb2 = _t([[0.5, 0.1, 0.2]])
    assert rbab.closure(lb2, each).tolist() == [True]


def test_clip_hand_computed():
    # x0 + 0.5 <= 0 on [0,1]^2 is empty (min 0.5 > 0); x0 - 0.5 <= 0 gives x0 <= 0.5
    xl, xh = _t([[0.0, 0.0]]), _t([[1.0, 1.0]])
    A = _t([[[1.0, 0.0]]])
    l, h, f = rbab.clip_box_by_halfspaces_batched(xl, xh, A, _t([[0.5]]))
    assert not bool(f[0])
    l, h, f = rbab.clip_box_by_halfspaces_batched(xl, xh, A, _t([[-0.5]]))
    assert bool(f[0])
    torch.testing.assert_close(h, _t([[0.5, 1.0]]))
    torch.testing.assert_close(l, _t([[0.0, 0.0]]))
    # -x0 - x1 + 1.5 <= 0 -> x0 >= 0.5 and x1 >= 0.5
    l, h, f = rbab.clip_box_by_halfspaces_batched(xl, xh, _t([[[-1.0, -1.0]]]),
                                                  _t([[1.5]]))
    torch.testing.assert_close(l, _t([[0.5, 0.5]]))


def test_clip_brute_force_contains_feasible_points():
    g = torch.Generator().manual_seed(3)
    B, Q, n = 64, 3, 3
    xl = torch.rand(B, n, generator=g, dtype=DT) - 1
    xh = xl + torch.rand(B, n, generator=g, dtype=DT) + 0.1
    A = torch.randn(B, Q, n, generator=g, dtype=DT)
    b = torch.randn(B, Q, generator=g, dtype=DT)
    l, h, f = rbab.clip_box_by_halfspaces_batched(xl, xh, A, b)
    pts = _util.sample_box(xl, xh, 4000, seed=2)
    val = torch.einsum('bqn,bpn->bpq', A, pts) + b.unsqueeze(1)
    ok = (val <= 0).all(-1)                                    # (B, P)
    for i in range(B):
        inside = pts[i][ok[i]]
        if inside.numel():
            assert bool(f[i])
            assert bool((inside >= l[i] - 1e-12).all() and (inside <= h[i] + 1e-12).all())
    assert bool((l >= xl).all() and (h <= xh).all())


def test_clip_multi_disjunct_union():
    xl, xh = _t([[0.0, 0.0]]), _t([[1.0, 1.0]])
    A = _t([[[1.0, 0.0], [-1.0, 0.0]]])
    b = _t([[-0.25, 0.75]])          # d0: x0 <= 0.25 ; d1: x0 >= 0.75
    l, h, f = rbab.clip_leaves(xl, xh, A, b, {0: [0], 1: [1]})
    assert bool(f[0])
    torch.testing.assert_close(l, _t([[0.0, 0.0]]))
    torch.testing.assert_close(h, _t([[1.0, 1.0]]))
    b2 = _t([[0.5, 0.75]])           # d0 empty -> union is d1's box
    l, h, f = rbab.clip_leaves(xl, xh, A, b2, {0: [0], 1: [1]})
    torch.testing.assert_close(l, _t([[0.75, 0.0]]))
    torch.testing.assert_close(h, _t([[1.0, 1.0]]))
    b3 = _t([[0.5, 1.5]])            # both empty -> infeasible, box kept
    l, h, f = rbab.clip_leaves(xl, xh, A, b3, {0: [0], 1: [1]})
    assert not bool(f[0])
    torch.testing.assert_close(l, xl)


def test_widest_axis_first_max():
    xl = _t([[0.0, 0.0, 0.0], [0.0, 0.0, 0.0]])
    xh = _t([[1.0, 2.0, 2.0], [3.0, 1.0, 3.0]])
    assert rbab.widest_axis(xl, xh).tolist() == [1, 0]


def test_bisect_children_partition_parent():
    g = torch.Generator().manual_seed(0)
    xl = torch.rand(20, 4, generator=g)
    xh = xl + torch.rand(20, 4, generator=g)
    xh[3] = xl[3]                                    # degenerate leaf
    ax = rbab.widest_axis(xl, xh)
    n_deg, (lxl, lxh), (hxl, hxh) = rbab.bisect(xl, xh, ax)
    assert n_deg == 1
    keep = [i for i in range(20) if i != 3]
    for r, i in enumerate(keep):
        a = int(ax[i])
        mid = (xl[i, a] + xh[i, a]) * 0.5
        assert torch.equal(lxl[r], xl[i]) and torch.equal(hxh[r], xh[i])
        assert float(lxh[r, a]) == float(mid) == float(hxl[r, a])
        others = [k for k in range(4) if k != a]
        assert torch.equal(lxh[r, others], xh[i, others])
        assert torch.equal(hxl[r, others], xl[i, others])


def test_worklist_lifo_chunks():
    wl = rbab.ChunkWorklist(_t([0.0]), _t([1.0]))
    wl.pop(1)
    a = torch.arange(6, dtype=DT).reshape(3, 2)
    b = torch.arange(6, 10, dtype=DT).reshape(2, 2)
    wl.push(a, a)
    wl.push(b, b)
    xl, _ = wl.pop(3)                   # all of b (last pushed) then last row of a
    assert xl.tolist() == [[6, 7], [8, 9], [4, 5]]
    assert wl.size() == 2
    xl, _ = wl.pop(2)
    assert xl.tolist() == [[0, 1], [2, 3]]
    assert not wl


def test_step_compaction_order_and_clipped_rows():
    """bab_step's leaf bookkeeping against a per-leaf brute force on a C0
    batch: ``unclosed`` lists exactly the open leaves in ascending order,
    ``feasible`` and the split rows follow that order (each row the clip of
    its own leaf alone), and the low/high children pair up row by row.  A
    descending or closed-leaf compaction, or a clip over the wrong rows,
    fails here."""
    gg = wk.acas_gg(dtype=DT)
    xl, xh = wk.acas_boxes(48, seed=4, dtype=DT)
    c, r = (xl + xh) / 2, (xh - xl) / 2
    xl, xh = c - 6 * r, c + 6 * r                 # wide enough to leave some open
    spec_ew, dq = _util.spec_for(5)
    st = rbab.bab_step(xl, xh, gg, spec_ew, dq)
    closed = st['closed']
    want = [i for i in range(48) if not bool(closed[i])]
    assert 0 < len(want) < 48
    assert st['unclosed'].tolist() == want
    rows_l, rows_h, feas = [], [], []
    for i in want:
        l1, h1, f1 = rbab.clip_box_by_halfspaces_batched(
            xl[i:i + 1], xh[i:i + 1], st['A'][i:i + 1], st['acc'][i:i + 1])
        feas.append(bool(f1[0]))
        if f1[0]:
            rows_l.append(l1[0])
            rows_h.append(h1[0])
    assert st['feasible'].tolist() == feas
    assert torch.equal(st['xl_split'], torch.stack(rows_l))
    assert torch.equal(st['xh_split'], torch.stack(rows_h))
    (lxl, lxh), (hxl, hxh) = st['low'], st['high']
    assert torch.equal(lxl, st['xl_split']) and torch.equal(hxh, st['xh_split'])
    for k in range(lxl.shape[0]):
        a = int(st['ax'][k])
        assert lxh[k, a] == hxl[k, a]


def test_band_select_hand_computed():
    """Boundary-band alpha leaves (verify_graph.py:12938-12950): worst
    disjunct's best bound > -eps, unclosed only, best first, ties in leaf
    order, truncated to max_leaves."""
    lb = _t([[-0.1, -0.3, -0.2],     # d0 -0.1, d1 -0.2 -> worst -0.2
             [-0.6, -0.7, 0.1],      # worst -0.6: outside the band
             [-0.4, -0.05, -0.2],    # d0 -0.05, d1 -0.2 -> -0.2 (tie with leaf 0)
             [0.3, -1.0, -0.01],     # d0 0.3, d1 -0.01 -> -0.01 (best)
             [0.2, 0.1, 0.3],        # closed
             [-0.45, -0.5, -0.3],    # -0.45
             [-0.5, -0.9, -0.5]])    # exactly -eps: outside (strict)
    dq = {0: [0, 1], 1: [2]}
    closed = rbab.closure(lb, dq)
    assert closed.tolist() == [False, False, False, False, True, False, False]
    assert rbab.band_select(lb, closed, dq, 0.5, 200).tolist() == [3, 0, 2, 5]
    assert rbab.band_select(lb, closed, dq, 0.5, 3).tolist() == [3, 0, 2]
    assert rbab.band_select(lb, closed, dq, 0.5, 2).tolist() == [3, 0]
    assert rbab.band_select(lb, closed, dq, 0.7, 200).tolist() == [3, 0, 2, 5, 6, 1]
    assert rbab.band_select(lb, closed, dq, 0.005, 200).tolist() == []


def test_clip_loop_repeats_until_nothing_shrinks():
    """x0 - x1 <= 0 and x1 - 0.3 <= 0 on [0, 1]^2: the first clip gives
    x1 <= 0.3 but keeps x0 <= 1; the second, on the smaller box, gives
    x0 <= 0.3; the third changes nothing and ends the loop
    (verify_graph.py:13036-13081)."""
    xl, xh = _t([[0.0, 0.0]]), _t([[1.0, 1.0]])
    A = _t([[[1.0, -1.0], [0.0, 1.0]]])
    b = _t([[0.0, -0.3]])
    dq = {0: [0, 1]}
    l1, h1, f1 = rbab.clip_iterated(xl, xh, A, b, dq, 1)
    torch.testing.assert_close(h1, _t([[1.0, 0.3]]))
    l2, h2, f2 = rbab.clip_iterated(xl, xh, A, b, dq, 2)
    torch.testing.assert_close(h2, _t([[0.3, 0.3]]))
    l9, h9, f9 = rbab.clip_iterated(xl, xh, A, b, dq, 9)
    torch.testing.assert_close(h9, _t([[0.3, 0.3]]))
    assert bool(f1[0] and f2[0] and f9[0])
    torch.testing.assert_close(l9, xl)
    # an emptied box stays infeasible on later iterations
    b_e = _t([[0.0, 0.1]])                      # x1 <= -0.1: empty on x1 >= 0
    _, _, fe = rbab.clip_iterated(xl, xh, A, b_e, dq, 5)
    assert not bool(fe[0])


def test_spec_queries_and_dedup():
    spec = VNNSpec([0.0], [1.0], [
        Conjunct([PairwiseConstraint(0, 1), Constraint(2, '>=', 0.5)]),
        Conjunct([PairwiseConstraint(0, 1), Constraint(1, '<=', -2.0)])])
    q = spec.as_linear_queries(3)
    assert [d for d, _, _ in q] == [0, 0, 1, 1]
    np.testing.assert_array_equal(q[0][1], [1.0, -1.0, 0.0])
    np.testing.assert_array_equal(q[1][1], [0.0, 0.0, -1.0])
    assert q[1][2] == 0.5
    np.testing.assert_array_equal(q[3][1], [0.0, 1.0, 0.0])
    assert q[3][2] == 2.0
    uq, dq = dedup_queries(q)
    assert len(uq) == 3 and dq == {0: [0, 1], 1: [0, 2]}


def test_bab_step_sound_split_of_unclosed_only():
    """One C0-shaped step: closed leaves are never split; every child box
    lies inside its parent; the children of a leaf partition it."""
    gg = wk.acas_gg(dtype=DT)
    xl, xh = wk.acas_boxes(64, seed=1, dtype=DT)
    spec_ew, dq = _util.spec_for(5)
    st = rbab.bab_step(xl, xh, gg, spec_ew, dq)
    closed = st['closed']
    pts = _util.sample_box(xl, xh, 300, seed=9)
    Wq = torch.stack([spec_ew[q][0] for q in sorted(spec_ew)])
    for b in range(64):
        y, _ = rb.point_forward(pts[b], gg)
        if bool(closed[b]):            # verified: every sample is safe
            assert bool(((y @ Wq.T) > 0).any(1).all())
    n_u = st['unclosed'].numel()
    assert n_u == int((~closed).sum())
    (lxl, lxh), (hxl, hxh) = st['low'], st['high']
    assert lxl.shape[0] + st['n_degenerate'] <= n_u
    assert bool((lxh >= lxl).all() and (hxh >= hxl).all())


def test_input_split_driver_known_answers():
    """The oracle's driver on the reference's bundled ACAS-Xu example
    (README.md:42-80): prop_1 is unsat -- verified, here after 253 leaves in
    11 iterations (the counts the GPU driver must reproduce); prop_2 is
    violated and is never verified; a box around a point where the spec
    holds strictly closes at the root."""
    import os
    from vibecheck_amd import onnx_net, vnnlib
    from test_formats import GOLD, NET
    gg = onnx_net.load_onnx(NET, dtype=torch.float32)

    def run(spec, **kw):
        uq, dq = dedup_queries(spec.as_linear_queries(5))
        se = {i: (torch.tensor(w, dtype=torch.float32), b) for i, (w, b) in enumerate(uq)}
        return rbab.input_split_batched(torch.tensor(spec.x_lo, dtype=torch.float32),
                                        torch.tensor(spec.x_hi, dtype=torch.float32), gg,
                                        se, dq, **kw)
    p1 = vnnlib.load_vnnlib(os.path.join(GOLD, 'prop_1.vnnlib'))
    verdict, det, trace = run(p1)
    assert verdict == 'verified', det
    assert (det['batched_n_leaves'], det['batched_n_iters']) == (253, 11), det
    assert sum(t['B'] for t in trace) == 253 and trace[0]['B'] == 1
    # every popped leaf is closed or split: children = 2 (B - closed)
    assert all(t['n_children'] == 2 * (t['B'] - t['n_closed']) for t in trace)
    p2 = vnnlib.load_vnnlib(os.path.join(GOLD, 'prop_2.vnnlib'))
    verdict, det, _ = run(p2, max_iters=12)
    assert verdict == 'unknown', det
    # a tiny box around a point whose spec margin (the largest query value,
    # one disjunct: any query > 0 closes) is clearly positive closes at the
    # root
    gg64 = wk.acas_gg(dtype=DT)
    gg32 = wk.acas_gg(dtype=torch.float32)
    se64, _ = _util.spec_for(5)
    Wq = torch.stack([se64[q][0] for q in sorted(se64)])
    g = torch.Generator().manual_seed(11)
    pts = torch.rand(400, 5, generator=g, dtype=DT) * 2 - 1
    margins = torch.stack([(Wq @ rb.point_forward(p, gg64)[0].reshape(-1)).max() for p in pts])
    for k, want in ((int(margins.argmax()), 'verified'),):
        assert float(margins[k]) > 1e-2, float(margins[k])
        spec = wk.acas_spec((pts[k] - 1e-4).tolist(), (pts[k] + 1e-4).tolist())
        uq, dq = dedup_queries(spec.as_linear_queries(5))
        se = {i: (torch.tensor(w, dtype=torch.float32), b) for i, (w, b) in enumerate(uq)}
        v, det, _ = rbab.input_split_batched(torch.tensor(spec.x_lo, dtype=torch.float32),
                                             torch.tensor(spec.x_hi, dtype=torch.float32),
                                             gg32, se, dq, max_iters=6)
        assert v == want, (float(margins[k]), det)
        if want == 'verified':
            assert det['batched_n_iters'] == 1 and det['batched_n_leaves'] == 1


# ----------------------------------------------------------- SB and K > 1
def test_sb_scores_known_answer():
    """widths (1, 2, 0.5); A rows (1, -1, 4), (2, 0.5, -2); lb (-1, -0.5).
    sum form: (1 * 3, 2 * 1.5, 0.5 * 6) = (3, 3, 3); margin form (thr 0.6,
    mw 1): q0 (1*1/2 - 1, 1*2/2 - 1, 4*0.5/2 - 1) = (-0.5, 0, 0),
    q1 (2*1/2 - 0.5, 0.6*2/2 - 0.5, 2*0.5/2 - 0.5) = (0.5, 0.1, 0), max over
    q = (0.5, 0.1, 0)."""
    xl = _t([[0.0, 0.0, 0.0]])
    xh = _t([[1.0, 2.0, 0.5]])
    A = _t([[[1.0, -1.0, 4.0], [2.0, 0.5, -2.0]]])
    lb = _t([[-1.0, -0.5]])
    s = rbab.sb_scores(xl, xh, A, lb)
    assert s.tolist() == [[3.0, 3.0, 3.0]]
    m = rbab.sb_scores(xl, xh, A, lb, margin=True, thr=0.6, mw=1.0)
    assert torch.allclose(m, _t([[0.5, 0.1, 0.0]]), rtol=0, atol=1e-15)
    # ties: the first maximum (torch.argmax), a stable order for K > 1
    assert rbab.top_dims(s, 1).tolist() == [[0]]
    assert rbab.top_dims(_t([[1.0, 3.0, 3.0, 2.0]]), 1).tolist() == [[1]]
    assert rbab.top_dims(_t([[1.0, 3.0, 3.0, 2.0]]), 3).tolist() == [[1, 2, 3]]


def test_split_multi_partitions_each_leaf():
    """Brute force: the children of a leaf are its 2^K_u sub-boxes (K_u =
    dimensions wider than 1e-12 among the K), in combo-bit order, and every
    sample of the parent box lies in exactly one child (off the split
    planes); leaves with no usable dimension are dropped and counted."""
    g = torch.Generator().manual_seed(3)
    xl = torch.rand(4, 5, generator=g, dtype=DT)
    xh = xl + torch.rand(4, 5, generator=g, dtype=DT)
    xh[1, 2] = xl[1, 2]                      # one zero-width split dimension
    xh[3] = xl[3]                            # a leaf with nothing to split
    dims = torch.tensor([[4, 0, 2], [2, 1, 3], [0, 1, 2], [1, 2, 3]])
    n_deg, (cl, ch) = rbab.split_multi(xl, xh, dims)
    assert n_deg == 1
    counts = [8, 4, 8]
    assert cl.shape[0] == sum(counts)
    row = 0
    for b, cnt in zip(range(3), counts):
        usable = [int(d) for d in dims[b] if float(xh[b, d] - xl[b, d]) > 1e-12]
        assert cnt == 1 << len(usable)
        kids_l, kids_h = cl[row:row + cnt], ch[row:row + cnt]
        for c in range(cnt):
            for k, d in enumerate(usable):
                mid = (xl[b, d] + xh[b, d]) / 2
                if (c >> k) & 1:
                    assert kids_l[c, d] == mid and kids_h[c, d] == xh[b, d]
                else:
                    assert kids_l[c, d] == xl[b, d] and kids_h[c, d] == mid
        pts = xl[b] + torch.rand(500, 5, generator=g, dtype=DT) * (xh[b] - xl[b])
        inside = ((pts.unsqueeze(1) > kids_l) & (pts.unsqueeze(1) < kids_h)) | \
            (kids_l == kids_h)
        assert bool((inside.all(-1).sum(1) == 1).all())
        row += cnt


def test_bab_step_sb_and_multi_split():
    """One step with SB branching and K = 3: every feasible split leaf gives
    2^K_u children inside its clipped box, the split dimensions are the
    top-3 SB scores of that leaf's A rows, and the driver grows the queue."""
    gg = wk.acas_gg(dtype=DT)
    xl, xh = wk.acas_boxes(32, seed=2, dtype=DT)
    c, r = (xl + xh) / 2, (xh - xl) / 2
    xl, xh = c - 8 * r, c + 8 * r
    spec_ew, dq = _util.spec_for(5)
    st = rbab.bab_step(xl, xh, gg, spec_ew, dq, branch_sb=True, split_depth=3)
    xs, hs = st['xl_split'], st['xh_split']
    assert xs.shape[0] > 0 and len(st['chunks']) == 1
    A_s = st['A'][st['unclosed']][st['feasible']]
    lb_s = st['lb'][st['unclosed']][st['feasible']]
    dims = rbab.top_dims(rbab.sb_scores(xs, hs, A_s, lb_s), 3)
    assert torch.equal(st['dims'], dims)
    kl, kh = st['chunks'][0]
    row = 0
    for b in range(xs.shape[0]):
        ku = sum(float(hs[b, d] - xs[b, d]) > 1e-12 for d in dims[b].tolist())
        n = 1 << ku if ku else 0
        assert bool((kl[row:row + n] >= xs[b]).all() and (kh[row:row + n] <= hs[b]).all())
        row += n
    assert row == kl.shape[0]


# --------------------------------------------------- alpha on the BaB leaves
def _one_neuron_net():
    """x -> z = x -> h = relu(z) -> (y0, y1) = (h + 0.1, h - 10), in fp64.

    On a box [l, u] with l < 0 < u, CROWN's lower relaxation h >= alpha z
    gives lb(y0) = alpha l + 0.1 and lb(y1) = alpha l - 10 (alpha in [0, 1]);
    the adaptive slope is alpha = 1 iff u > -l.  The exact minimum of y0 is
    0.1, reached by alpha = 0, and alpha-CROWN's Adam walks alpha down from 1
    by lr_t each step (a constant gradient makes every Adam step lr_t, to
    1e-8 relative), clamped at 0."""
    gg = wk.mlp_gg([_t([[1.0]]), _t([[1.0], [1.0]])], [_t([0.0]), _t([0.1, -10.0])],
                   dtype=DT)
    se2 = {0: (_t([1.0, 0.0]), 0.0), 1: (_t([0.0, 1.0]), 0.0)}
    se1 = {0: (_t([1.0, 0.0]), 0.0)}
    # leaves: A [-0.5, 1] open (lb0 -0.4); B [-1, 0.5] closed (alpha 0: 0.1);
    # C [0.2, 0.3] stable, closed (0.3); D [-0.05, 1] closed (0.05, alpha 1);
    # E [-2, 3] open (-1.9)
    xl = _t([[-0.5], [-1.0], [0.2], [-0.05], [-2.0]])
    xh = _t([[1.0], [0.5], [0.3], [1.0], [3.0]])
    return gg, se1, se2, xl, xh


def _alpha_walk(n, g):
    """alpha after n Adam steps from 1 at lr 0.25, decay 0.98, clamped at 0,
    under a constant gradient of magnitude g: Adam's bias-corrected moments
    are g and g^2, so each step is lr_t g / (g + 1e-8)."""
    a = 1.0
    for t in range(n):
        a = max(0.0, a - 0.25 * 0.98 ** t * g / (g + 1e-8))
    return a


def test_alpha_on_leaves_closed_form():
    """``alpha_on_leaves`` (verify_graph.py:12927-12975) on the one-neuron
    net, every number by hand.  alpha_all runs on the CROWN-open leaves A, E
    only; the closed leaves' bounds stay bit for bit (alpha on D would raise
    its 0.05 to 0.1); the open leaves' bounds are max(CROWN, alpha) entry by
    entry (a min merge keeps -0.4); the closure is recomputed from the merged
    bound (a stale one leaves A, E open); the iteration count is the loop's
    own: the global max of the best bound stops improving (it stays 0.1
    once alpha is clamped at 0) after 7 evaluations."""
    gg, _, se2, xl, xh = _one_neuron_net()
    dq = {0: [0, 1]}
    lb, _, _ = rbab.bound_batch(xl, xh, gg, se2)
    torch.testing.assert_close(lb, _t([[-0.4, -10.5], [0.1, -10.0], [0.3, -9.8],
                                       [0.05, -10.05], [-1.9, -12.0]]), rtol=0, atol=1e-12)
    closed = rbab.closure(lb, dq)
    assert closed.tolist() == [False, True, True, True, False]
    lb_in = lb.clone()
    out, cl, n_l, n_it = rbab.alpha_on_leaves(lb, xl, xh, gg, se2, dq, closed, 20,
                                              True, 0.0, 200)
    assert torch.equal(lb, lb_in)                       # input not mutated
    assert (n_l, n_it) == (2, 7)
    for i in (1, 2, 3):
        assert torch.equal(out[i], lb[i])
    # alpha reaches 0 after 5 steps: best y0 = 0.1, best y1 = -10
    torch.testing.assert_close(out[[0, 4]], _t([[0.1, -10.0], [0.1, -10.0]]),
                               rtol=0, atol=1e-9)
    assert cl.tolist() == [True] * 5
    # the count alone, from the alpha loop on the two open leaves
    _, n = rb.alpha_crown_batched(xl[[0, 4]], xh[[0, 4]], gg, se2, n_iters=20,
                                  return_trace=True)
    assert n == 7
    # an iteration budget below the stop: 3 evaluations, alpha 1, 0.75, 0.505
    out3, cl3, _, n3 = rbab.alpha_on_leaves(lb, xl, xh, gg, se2, dq, closed, 3,
                                            True, 0.0, 200)
    # (gradient of -(lb0 + lb1) in alpha: -2 l, so 1 for A and 4 for E)
    aA, aE = _alpha_walk(2, 1.0), _alpha_walk(2, 4.0)
    assert n3 == 3 and abs(aA - 0.505) < 1e-7 and abs(aE - 0.505) < 1e-7
    torch.testing.assert_close(out3[[0, 4]], _t([[-0.5 * aA + 0.1, -0.5 * aA - 10],
                                                 [-2 * aE + 0.1, -2 * aE - 10]]),
                               rtol=0, atol=1e-12)
    assert cl3.tolist() == [False, True, True, True, False]


def test_alpha_on_leaves_all_positive_stop():
    """With the single query y0 the loop stops on every best bound > 0
    (verify_zono_bnb.py:5258-5259) at the 5th evaluation, where alpha =
    1 - 0.25 (1 + 0.98 + 0.98^2 + 0.98^3) = 0.029602 gives y0 bounds
    0.085199 (A) and 0.040796 (E): the bound of the evaluation that stopped
    the loop, not the 0.1 that further steps would reach."""
    gg, se1, _, xl, xh = _one_neuron_net()
    dq = {0: [0]}
    lb, _, _ = rbab.bound_batch(xl, xh, gg, se1)
    closed = rbab.closure(lb, dq)
    out, cl, n_l, n_it = rbab.alpha_on_leaves(lb, xl, xh, gg, se1, dq, closed, 20,
                                              True, 0.0, 200)
    # (gradient of -lb0 in alpha: -l, so 0.5 for A and 2 for E)
    aA, aE = _alpha_walk(4, 0.5), _alpha_walk(4, 2.0)
    assert abs(aA - 0.029602) < 1e-7 and abs(aE - 0.029602) < 1e-7
    assert (n_l, n_it) == (2, 5)
    torch.testing.assert_close(out[[0, 4], 0], _t([-0.5 * aA + 0.1, -2 * aE + 0.1]),
                               rtol=0, atol=1e-12)
    assert cl.tolist() == [True] * 5


def test_alpha_on_leaves_band_and_multi_disjunct():
    """Band selection (alpha_all off): eps 1 takes A (worst -0.4) and not E
    (-1.9); eps 3 with max_leaves 1 takes the best, A.  With two one-query
    disjuncts no leaf ever closes (y1 < 0), alpha_all takes all five, and the
    loop stops at its 2nd evaluation, because leaf C's constant 0.3 holds
    the global max (a per-leaf stop would run on); D rises to
    -0.75 * 0.05 + 0.1 = 0.0625."""
    gg, _, se2, xl, xh = _one_neuron_net()
    dq = {0: [0, 1]}
    lb, _, _ = rbab.bound_batch(xl, xh, gg, se2)
    closed = rbab.closure(lb, dq)
    for eps, mx in ((1.0, 200), (3.0, 1)):
        out, cl, n_l, n_it = rbab.alpha_on_leaves(lb, xl, xh, gg, se2, dq, closed, 20,
                                                  False, eps, mx)
        assert (n_l, n_it) == (1, 7)
        torch.testing.assert_close(out[0], _t([0.1, -10.0]), rtol=0, atol=1e-9)
        assert torch.equal(out[1:], lb[1:])
        assert cl.tolist() == [True, True, True, True, False]
    # nothing in the band: no alpha, nothing changes
    out, cl, n_l, n_it = rbab.alpha_on_leaves(lb, xl, xh, gg, se2, dq, closed, 20,
                                              False, 0.3, 200)
    assert (n_l, n_it) == (0, 0) and torch.equal(out, lb)
    # off: zero iterations, or neither alpha_all nor a band
    for it, al, eps in ((0, True, 0.0), (20, False, 0.0)):
        assert rbab.alpha_on_leaves(lb, xl, xh, gg, se2, dq, closed, it, al, eps,
                                    200)[2:] == (0, 0)
    dq2 = {0: [0], 1: [1]}
    closed2 = rbab.closure(lb, dq2)
    assert closed2.tolist() == [False] * 5
    out, cl, n_l, n_it = rbab.alpha_on_leaves(lb, xl, xh, gg, se2, dq2, closed2, 20,
                                              True, 0.0, 200)
    assert (n_l, n_it) == (5, 2)
    # one step each: alpha 0.75 to 1e-8 relative (gradients 1, 0.1, 4)
    want = lb.clone()
    for i, l in ((0, -0.5), (3, -0.05), (4, -2.0)):
        a = _alpha_walk(1, -2 * l)
        assert abs(a - 0.75) < 1e-7
        want[i] = _t([a * l + 0.1, a * l - 10])
    torch.testing.assert_close(want[[0, 3, 4]], _t([[-0.275, -10.375], [0.0625, -10.0375],
                                                    [-1.4, -11.5]]), rtol=0, atol=1e-7)
    torch.testing.assert_close(out, want, rtol=0, atol=1e-12)
    assert cl.tolist() == [False] * 5


def test_bab_step_alpha_branch():
    """bab_step with alpha (verify_graph.py:12927-12986): ``crown_lb`` /
    ``crown_closed`` are the bound phase's, ``lb`` / ``closed`` the merged
    ones, ``unclosed`` lists the leaves still open after alpha, and the clip
    of that leaf uses the CROWN pass's linear bound: E = [-2, 3] with
    y0 >= x + 0.1 and y1 >= x - 10 (one disjunct: both <= 0 on the clip)
    clips to [-2, -0.1] and bisects at -1.05."""
    gg, _, se2, xl, xh = _one_neuron_net()
    dq = {0: [0, 1]}
    st = rbab.bab_step(xl, xh, gg, se2, dq, alpha_iters=20, alpha_eps=1.0)
    st0 = rbab.bab_step(xl, xh, gg, se2, dq)
    assert torch.equal(st['crown_lb'], st0['lb'])
    assert torch.equal(st['crown_closed'], st0['closed'])
    assert (st['n_alpha_leaves'], st['n_alpha_iters']) == (1, 7)
    assert st['closed'].tolist() == [True, True, True, True, False]
    assert st['unclosed'].tolist() == [4] and st0['unclosed'].tolist() == [0, 4]
    torch.testing.assert_close(st['lb'][0], _t([0.1, -10.0]), rtol=0, atol=1e-9)
    assert st['feasible'].tolist() == [True]
    torch.testing.assert_close(st['xl_split'], _t([[-2.0]]), rtol=0, atol=1e-12)
    torch.testing.assert_close(st['xh_split'], _t([[-0.1]]), rtol=0, atol=1e-12)
    (lxl, lxh), (hxl, hxh) = st['low'], st['high']
    torch.testing.assert_close(lxh, _t([[-1.05]]), rtol=0, atol=1e-12)
    assert torch.equal(lxh, hxl) and torch.equal(lxl, st['xl_split'])
    stall = rbab.bab_step(xl, xh, gg, se2, dq, alpha_iters=20, alpha_all=True)
    assert stall['unclosed'].numel() == 0 and stall['chunks'] == []
