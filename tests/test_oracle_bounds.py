"""Pins the CPU oracle's bound primitives (oracle/ref_bound.py).

Checks are closed forms, the reference's own known-answer tests
(tests/test_bnb.py:159-199 and tests/test_ibp_crown.py of the reference),
hand-computed small cases, and sampled ground truth: each is chosen so that
a dropped term, a sign error or a transposed operand in the oracle fails.
All CPU, float64 unless stated.
"""
import numpy as np
import pytest
import torch

from oracle import ref_bound as rb
from vibecheck_amd import workloads as wk

import _util

DT = torch.float64


def _t(v):
    return torch.tensor(v, dtype=DT)


# ---------------------------------------------------------------- slopes
class TestMakeSlopes:
    """Known answers of the reference's TestMakeSlopes."""

    def test_active(self):
        lo_s, up_s, up_t, a, d, u = rb.make_slopes(_t([1.0, 2.0]), _t([3.0, 4.0]))
        assert a.all() and not d.any() and not u.any()
        assert torch.equal(lo_s, _t([1.0, 1.0]))

    def test_dead(self):
        lo_s, up_s, up_t, a, d, u = rb.make_slopes(_t([-3.0, -2.0]), _t([-1.0, -0.5]))
        assert d.all() and not a.any()
        assert torch.equal(lo_s, _t([0.0, 0.0]))

    def test_unstable(self):
        lo_s, up_s, up_t, a, d, u = rb.make_slopes(_t([-1.0]), _t([3.0]))
        assert u.all()
        torch.testing.assert_close(up_s, _t([0.75]))
        torch.testing.assert_close(up_t, _t([0.75]))
        torch.testing.assert_close(lo_s, _t([1.0]))

    def test_mixed(self):
        lo_s, up_s, up_t, a, d, u = rb.make_slopes(_t([1.0, -1.0, -3.0]),
                                                   _t([2.0, 1.0, -1.0]))
        assert a.tolist() == [True, False, False]
        assert d.tolist() == [False, False, True]
        assert u.tolist() == [False, True, False]

    def test_upper_line_is_chord(self):
        # the upper relaxation passes through (lo, 0) and (hi, hi)
        g = torch.Generator().manual_seed(0)
        lo = -torch.rand(1000, generator=g, dtype=DT) * 5 - 1e-3
        hi = torch.rand(1000, generator=g, dtype=DT) * 5 + 1e-3
        _, up_s, up_t, _, _, u = rb.make_slopes(lo, hi)
        assert u.all()
        torch.testing.assert_close(up_s * lo + up_t, torch.zeros_like(lo),
                                   atol=1e-12, rtol=0)
        torch.testing.assert_close(up_s * hi + up_t, hi)

    def test_lower_slope_minimises_area(self):
        # lo_s = 1 iff hi > -lo (the relaxation of smaller area)
        lo_s, *_ = rb.make_slopes(_t([-1.0, -3.0, -2.0]), _t([3.0, 1.0, 2.0]))
        assert lo_s.tolist() == [1.0, 0.0, 0.0]

    def test_zero_interval_is_active_and_dead(self):
        lo_s, up_s, up_t, a, d, u = rb.make_slopes(_t([0.0]), _t([0.0]))
        assert bool(a[0]) and bool(d[0]) and not bool(u[0])
        assert float(lo_s[0]) == 1.0

    def test_tiny_negative_dead_edge(self):
        # lb_r + 1e-8 > 0 gives a dead neuron a non-zero upper slope
        lo_s, up_s, up_t, a, d, u = rb.make_slopes(_t([-5e-9]), _t([-1e-9]))
        assert bool(d[0]) and float(lo_s[0]) == 0.0
        assert float(up_s[0]) == pytest.approx(0.5, rel=1e-9)


# ---------------------------------------------------------------- IBP
def _box(n, B, eps, seed):
    g = torch.Generator().manual_seed(seed)
    c = torch.rand(B, n, generator=g, dtype=DT) * 2 - 1
    return c - eps, c + eps


@pytest.mark.parametrize('net', ['mlp', 'cnn'])
def test_ibp_sound_and_first_layer_exact(net):
    gg = _util.tiny_mlp([4, 8, 8, 3], seed=3) if net == 'mlp' else _util.tiny_cnn()
    n = gg['input_n']
    xl, xh = _box(n, 3, 0.3, 1)
    sb = rb.ibp_forward_batched(xl, xh, gg)
    pts = _util.sample_box(xl, xh, 200, seed=7)
    for b in range(3):
        _, pre = rb.point_forward(pts[b], gg)
        for L, (lo, hi) in sb.items():
            assert bool((pre[L] >= lo[b] - 1e-9).all())
            assert bool((pre[L] <= hi[b] + 1e-9).all())
    # exactness of the first affine layer: endpoint-wise interval sum
    op = gg['ops'][0]
    if op['type'] == 'fc':
        W, bias = op['W'], op['bias']
        lo_ex = (torch.minimum(W * xl[:, None, :], W * xh[:, None, :])).sum(-1) + bias
        hi_ex = (torch.maximum(W * xl[:, None, :], W * xh[:, None, :])).sum(-1) + bias
    else:
        # dense matrix of the conv from the unit basis
        basis = torch.eye(n, dtype=DT)
        y0 = torch.nn.functional.conv2d(torch.zeros(1, *op['in_shape'], dtype=DT),
                                        op['kernel'], op['bias'], stride=op['stride'],
                                        padding=op['padding']).reshape(-1)
        Wd = (torch.nn.functional.conv2d(basis.reshape(n, *op['in_shape']),
                                         op['kernel'], op['bias'], stride=op['stride'],
                                         padding=op['padding']).reshape(n, -1) - y0).T
        lo_ex = torch.minimum(Wd * xl[:, None, :], Wd * xh[:, None, :]).sum(-1) + y0
        hi_ex = torch.maximum(Wd * xl[:, None, :], Wd * xh[:, None, :]).sum(-1) + y0
    torch.testing.assert_close(sb[0][0], lo_ex)
    torch.testing.assert_close(sb[0][1], hi_ex)


def test_ibp_clamps_root_and_repair():
    gg = _util.tiny_mlp([4, 8, 8, 3], seed=3)
    xl, xh = _box(4, 1, 0.5, 2)
    sb = rb.ibp_forward_batched(xl, xh, gg)
    B = 3
    xlb, xhb = xl.expand(B, -1).clone(), xh.expand(B, -1).clone()
    lo0, hi0 = sb[0][0][0], sb[0][1][0]
    j = int(((lo0 < 0) & (hi0 > 0)).nonzero()[0])
    n0 = lo0.numel()
    cl = torch.full((B, n0), -np.inf, dtype=DT)
    ch = torch.full((B, n0), np.inf, dtype=DT)
    ch[1, j] = 0.0
    root = {L: (lo[0], hi[0]) for L, (lo, hi) in sb.items()}
    sbc = rb.ibp_forward_batched(xlb, xhb, gg, relu_clamps={0: (cl, ch)}, root_sb=root)
    assert float(sbc[0][1][1, j]) == 0.0
    torch.testing.assert_close(sbc[0][1][0], hi0)
    assert bool((sbc[1][0][1] >= sb[1][0][0] - 1e-12).all())
    assert bool((sbc[1][1][1] <= sb[1][1][0] + 1e-12).all())
    jp = (lo0 > 0).nonzero()
    if jp.numel():
        ch2 = torch.full((B, n0), np.inf, dtype=DT)
        ch2[2, int(jp[0])] = 0.0
        sbe = rb.ibp_forward_batched(xlb, xhb, gg, relu_clamps={0: (cl, ch2)}, root_sb=root)
        assert bool((sbe[0][1][2] >= sbe[0][0][2]).all())


def test_ibp_unsupported_raises():
    gg = _util.tiny_mlp([2, 2, 1], seed=0)
    gg['ops'].insert(0, {'name': 's', 'type': 'sigmoid', 'inputs': ['X']})
    with pytest.raises(NotImplementedError):
        rb.ibp_forward_batched(torch.zeros(1, 2, dtype=DT), torch.ones(1, 2, dtype=DT), gg)


# ---------------------------------------------------------------- zonotope
def _chain(ws, bs):
    return wk.mlp_gg([torch.tensor(w, dtype=DT) for w in ws],
                     [torch.tensor(b, dtype=DT) for b in bs], dtype=DT)


def test_zono_hand_computed():
    # x in [-1, 1]; z0 = x -> relu: lam = 1/2, mu = 1/4 -> zonotope of the
    # relu output: c = 1/4, G = [1/2, 1/4] -> z1 = y0 in [-1/2, 1].
    gg = _chain([[[1.0]], [[1.0]], [[1.0]]], [[0.0], [0.0], [0.0]])
    sb, (c, G) = rb.zono_forward_batched(_t([[-1.0]]), _t([[1.0]]), gg)
    torch.testing.assert_close(sb[0][0], _t([[-1.0]]))
    torch.testing.assert_close(sb[0][1], _t([[1.0]]))
    torch.testing.assert_close(sb[1][0], _t([[-0.5]]))
    torch.testing.assert_close(sb[1][1], _t([[1.0]]))
    # second relu on [-1/2, 1]: lam = 2/3, mu = 1/6; c' = 2/3*1/4 + 1/6 = 1/3
    torch.testing.assert_close(c, _t([[1.0 / 3.0]]))
    torch.testing.assert_close(G.abs().sum(-1), _t([[2.0 / 3.0 * 0.75 + 1.0 / 6.0]]))


def test_zono_hand_computed_two_dims():
    # z0 = [x0 + x1, x0 - x1], x in [0,1]x[-1,1]; z0a in [-1, 2], z0b in [-1, 2]
    # relu: lam = 2/3, mu = 1/3 each; z1 = z0a' + z0b' has centre
    # 2/3*(0.5+0.5) + 2/3 = 4/3, generators x0: 2/3*(0.5+0.5) = 2/3,
    # x1: 2/3*(1-1) = 0, new: 1/3 + 1/3 -> radius 4/3 -> [0, 8/3]
    gg = _chain([[[1.0, 1.0], [1.0, -1.0]], [[1.0, 1.0]], [[1.0]]],
                [[0.0, 0.0], [0.0], [0.0]])
    sb, _ = rb.zono_forward_batched(_t([[0.0, -1.0]]), _t([[1.0, 1.0]]), gg)
    torch.testing.assert_close(sb[0][0], _t([[-1.0, -1.0]]))
    torch.testing.assert_close(sb[0][1], _t([[2.0, 2.0]]))
    torch.testing.assert_close(sb[1][0], _t([[0.0]]))
    torch.testing.assert_close(sb[1][1], _t([[8.0 / 3.0]]))


def test_zono_generator_layout_rank_and_padding():
    """The new generator columns of a ReLU (verify_zono_bnb.py:3190-3210):
    one per unstable neuron, in neuron order (the cumulative-count rank),
    padded with zero columns to the batch's largest unstable count.
    z = [x, x + 0.5, x - 0.5]; domain 0: x in [-1, 1], all three unstable;
    domain 1: x in [-0.1, 0.3], only neuron 0 unstable (1 active, 2 dead).
    An identity fc after the ReLU keeps G as the ReLU leaves it."""
    gg = _chain([[[1.0], [1.0], [1.0]], [[1.0, 0.0, 0.0], [0.0, 1.0, 0.0], [0.0, 0.0, 1.0]]],
                [[0.0, 0.5, -0.5], [0.0, 0.0, 0.0]])
    _, (c, G) = rb.zono_forward_batched(_t([[-1.0], [-0.1]]), _t([[1.0], [0.3]]), gg)
    assert G.shape == (2, 3, 4)
    # domain 0: lam = (1/2, 3/4, 1/4), mu = (1/4, 3/16, 3/16)
    torch.testing.assert_close(c[0], _t([0.25, 0.5625, 0.0625]))
    torch.testing.assert_close(G[0], _t([[0.5, 0.25, 0.0, 0.0],
                                         [0.75, 0.0, 0.1875, 0.0],
                                         [0.25, 0.0, 0.0, 0.1875]]))
    # domain 1: centre 0.1, radius 0.2; neuron 0 on [-0.1, 0.3]: lam = 3/4,
    # mu = 0.0375 in column 0 of the new block, columns 1 and 2 padding
    torch.testing.assert_close(c[1], _t([0.1125, 0.6, 0.0]))
    torch.testing.assert_close(G[1], _t([[0.15, 0.0375, 0.0, 0.0],
                                         [0.2, 0.0, 0.0, 0.0],
                                         [0.0, 0.0, 0.0, 0.0]]))


def test_zono_contains_samples_and_matches_ibp_at_first_layer():
    gg = wk.acas_gg(dtype=DT)
    xl, xh = wk.acas_boxes(16, seed=5, dtype=DT)
    xl, xh = xl * 4, xh * 4  # wider boxes: many unstable neurons
    sb, _ = rb.zono_forward_batched(xl, xh, gg)
    sbi = rb.ibp_forward_batched(xl, xh, gg)
    torch.testing.assert_close(sb[0][0], sbi[0][0])
    torch.testing.assert_close(sb[0][1], sbi[0][1])
    pts = _util.sample_box(xl, xh, 300, seed=3)
    for b in range(16):
        _, pre = rb.point_forward(pts[b], gg)
        for L, (lo, hi) in sb.items():
            assert bool((pre[L] >= lo[b] - 1e-9).all())
            assert bool((pre[L] <= hi[b] + 1e-9).all())


# ---------------------------------------------------------------- CROWN
def test_crown_hand_computed():
    # y = relu(x), x in [-1, 3]: lower line y >= x (up_s = 3/4 > 1/2),
    # upper line y <= 3/4 x + 3/4.  min y bound = -1, min(-y) bound = -3.
    gg = _chain([[[1.0]], [[1.0]]], [[0.0], [0.0]])
    xl, xh = _t([[-1.0]]), _t([[3.0]])
    sb = rb.ibp_forward_batched(xl, xh, gg)
    spec = {0: (_t([1.0]), 0.0), 1: (_t([-1.0]), 0.0)}
    lb, A, acc = rb.spec_backward_batched(sb, xl, xh, gg, spec, return_input_linear=True)
    torch.testing.assert_close(lb, _t([[-1.0, -3.0]]))
    torch.testing.assert_close(A, _t([[[1.0], [-0.75]]]))
    torch.testing.assert_close(acc, _t([[0.0, -0.75]]))


def test_crown_sound_and_linear_bound_pointwise():
    gg = wk.acas_gg(dtype=DT)
    xl, xh = wk.acas_boxes(8, seed=2, dtype=DT)
    xl, xh = xl * 3, xh * 3
    spec_ew, _ = _util.spec_for(5)
    sb, _ = rb.zono_forward_batched(xl, xh, gg)
    lb, A, acc = rb.spec_backward_batched(sb, xl, xh, gg, spec_ew, return_input_linear=True)
    Wq = torch.stack([spec_ew[q][0] for q in sorted(spec_ew)])
    pts = _util.sample_box(xl, xh, 500, seed=4)
    for b in range(8):
        y, _ = rb.point_forward(pts[b], gg)
        val = y @ Wq.T                                   # (P, Q)
        lin = pts[b] @ A[b].T + acc[b]                   # (P, Q)
        assert bool((lin <= val + 1e-9).all())           # linear lower bound holds
        assert bool((lb[b] <= val.min(0).values + 1e-9).all())
        assert bool((lb[b] <= lin.min(0).values + 1e-9).all())


def _conv_as_dense(gg):
    """Same network with every conv replaced by its dense fc matrix."""
    ops = []
    for op in gg['ops']:
        if op['type'] == 'conv':
            n = int(np.prod(op['in_shape']))
            y0 = torch.nn.functional.conv2d(torch.zeros(1, *op['in_shape'], dtype=DT),
                                            op['kernel'], op['bias'], stride=op['stride'],
                                            padding=op['padding']).reshape(-1)
            basis = torch.eye(n, dtype=DT).reshape(n, *op['in_shape'])
            Wd = (torch.nn.functional.conv2d(basis, op['kernel'], op['bias'],
                                             stride=op['stride'],
                                             padding=op['padding']).reshape(n, -1) - y0).T
            ops.append({'name': op['name'], 'type': 'fc', 'inputs': op['inputs'],
                        'W': Wd.contiguous(), 'bias': y0})
        else:
            ops.append(op)
    out = dict(gg)
    out['ops'] = ops
    return out


def test_crown_conv_equals_dense_equivalent():
    gg = _util.tiny_cnn(seed=4)
    for op in gg['ops']:
        if op['type'] == 'conv':
            op['bias'] = torch.randn(op['bias'].shape, dtype=DT,
                                     generator=torch.Generator().manual_seed(1)) * 0.2
    dense = _conv_as_dense(gg)
    xl, xh = _box(gg['input_n'], 2, 0.2, 3)
    spec_ew, _ = _util.spec_for(2)
    sb = rb.ibp_forward_batched(xl, xh, gg)
    sbd = rb.ibp_forward_batched(xl, xh, dense)
    for L in sb:
        torch.testing.assert_close(sb[L][0], sbd[L][0])
    lb, A, acc = rb.spec_backward_batched(sb, xl, xh, gg, spec_ew, return_input_linear=True)
    lbd, Ad, accd = rb.spec_backward_batched(sb, xl, xh, dense, spec_ew,
                                             return_input_linear=True)
    torch.testing.assert_close(lb, lbd)
    torch.testing.assert_close(A, Ad)
    torch.testing.assert_close(acc, accd)


def test_beta_zero_is_plain_and_beta_sound():
    """tests/test_ibp_crown.py:246-288 of the reference, on an MLP."""
    gg = _util.tiny_mlp([2, 6, 6, 2], seed=11)
    xl, xh = _t([[-1.0, -1.0]]), _t([[1.0, 1.0]])
    sb = rb.ibp_forward_batched(xl, xh, gg)
    spec = {0: (_t([1.0, -1.0]), 0.0)}
    lb_plain = rb.spec_backward_batched(sb, xl, xh, gg, spec)
    n0 = sb[0][0].shape[1]
    lb_b0 = rb.spec_backward_batched(sb, xl, xh, gg, spec,
                                     relu_split_beta={0: torch.zeros(1, n0, dtype=DT)})
    torch.testing.assert_close(lb_plain, lb_b0)
    lo0, hi0 = sb[0][0][0], sb[0][1][0]
    j = int(((lo0 < 0) & (hi0 > 0)).nonzero()[0])
    cl = torch.full((1, n0), -np.inf, dtype=DT)
    ch = torch.full((1, n0), np.inf, dtype=DT)
    ch[0, j] = 0.0
    root = {L: (lo[0], hi[0]) for L, (lo, hi) in sb.items()}
    sbc = rb.ibp_forward_batched(xl, xh, gg, relu_clamps={0: (cl, ch)}, root_sb=root)
    g = np.linspace(-1, 1, 201)
    X = torch.tensor(np.stack(np.meshgrid(g, g), -1).reshape(-1, 2), dtype=DT)
    y, pre = rb.point_forward(X, gg)
    inside = pre[0][:, j] <= 0
    true_min = float((y[inside] @ spec[0][0]).min())
    sgn = torch.zeros(1, n0, dtype=DT)
    sgn[0, j] = 1.0
    for beta in (0.0, 0.05, 0.5, 5.0):
        lb = float(rb.spec_backward_batched(sbc, xl, xh, gg, spec,
                                            relu_split_beta={0: sgn * beta})[0, 0])
        assert lb <= true_min + 1e-6


# ------------------------------------------------ ReLU-split alpha/beta bound
def test_split_domain_bounds_no_reforward_hand_computed():
    """Root bounds broadcast, clamps intersected, crossings repaired, layers
    without clamps left as the root (verify_milp.py:2706-2717)."""
    inf = float('inf')
    root = {0: (_t([-1.0, -2.0, 0.5]), _t([1.0, 3.0, 1.0])),
            1: (_t([-4.0]), _t([2.0]))}
    cl = _t([[-inf, 0.0, -inf], [-inf, -inf, -inf]])
    ch = _t([[0.0, inf, 0.0], [inf, inf, inf]])
    x = torch.zeros(2, 1, dtype=DT)
    sb = rb.split_domain_bounds(x, x, None, root, {0: (cl, ch)}, no_reforward=True)
    # domain 0: OFF on j0, ON on j1, OFF on the root-active j2 (crossing -> point)
    torch.testing.assert_close(sb[0][0], _t([[-1.0, 0.0, 0.5], [-1.0, -2.0, 0.5]]))
    torch.testing.assert_close(sb[0][1], _t([[0.0, 3.0, 0.5], [1.0, 3.0, 1.0]]))
    torch.testing.assert_close(sb[1][0], _t([[-4.0], [-4.0]]))
    torch.testing.assert_close(sb[1][1], _t([[2.0], [2.0]]))


def beta_known_answer_net():
    """x in [-1,1]^2; h1 = relu(x1 + x2) (the split neuron), h2 = relu(x1 +
    x2 + 2) (active on the box); y = -h2 + 2.4 = 0.4 - (x1 + x2).
    On the OFF side (x1 + x2 <= 0) min y = 0.4; on the ON side -1.6."""
    return _chain([[[1.0, 1.0], [1.0, 1.0]], [[0.0, -1.0]]], [[0.0, 2.0], [2.4]])


def test_beta_crown_bound_known_answer():
    """The OFF child closes only through beta: lb(beta) = 2 beta - 1.6 for
    beta < 1, and Adam moves beta by ~lr per step from 0, so the 5th
    evaluation (beta ~ 1) is the first with lb > 0, at ~0.4.  The ON child
    is exact at its true min -1.6: its gradient pushes beta below 0 and the
    clamp beta >= 0 holds it there (without the clamp the bound would pass
    the true min).  Without beta (sign 0) the OFF child stays at -1.6."""
    gg = beta_known_answer_net()
    inf = float('inf')
    xl = _t([[-1.0, -1.0], [-1.0, -1.0]])
    xh = _t([[1.0, 1.0], [1.0, 1.0]])
    root = rb.ibp_forward_batched(xl[:1], xh[:1], gg)
    root = {L: (lo[0], hi[0]) for L, (lo, hi) in root.items()}
    cl = _t([[-inf, -inf], [0.0, -inf]])                 # domain 1: ON
    ch = _t([[0.0, inf], [inf, inf]])                    # domain 0: OFF
    clamps = {0: (cl, ch)}
    sb = rb.split_domain_bounds(xl, xh, gg, root, clamps)
    sgn = rb.beta_signs_from_clamps(clamps)
    torch.testing.assert_close(sgn[0], _t([[1.0, 0.0], [-1.0, 0.0]]))
    spec = {0: (_t([1.0]), 0.0)}
    best, n = rb.beta_crown_bound(sb, xl, xh, gg, spec, sgn, n_iters=20, lr=0.25,
                                  return_trace=True)
    assert n == 20                                       # the ON child never closes
    assert abs(float(best[1, 0]) + 1.6) < 1e-12
    assert 0.39 < float(best[0, 0]) <= 0.4 + 1e-12
    sb_off = {L: (lo[:1], hi[:1]) for L, (lo, hi) in sb.items()}
    best5, n5 = rb.beta_crown_bound(sb_off, xl[:1], xh[:1], gg, spec, {0: sgn[0][:1]},
                                    n_iters=20, lr=0.25, return_trace=True)
    assert n5 == 5
    assert 0.39 < float(best5[0, 0]) <= 0.4 + 1e-12
    nob = rb.beta_crown_bound(sb, xl, xh, gg, spec, {0: torch.zeros_like(sgn[0])},
                              n_iters=20, lr=0.25)
    assert abs(float(nob[0, 0]) + 1.6) < 1e-12


def test_beta_crown_bound_first_iteration_monotone_and_sound():
    """First evaluation = plain CROWN on the split bounds (alpha init is the
    adaptive slope, beta = 0); the best bound is non-decreasing in the
    iteration count; it never exceeds the true min over the points of the
    box that satisfy the domain's split constraints."""
    gg = _util.tiny_mlp([2, 8, 8, 3], seed=23)
    inf = float('inf')
    x0l, x0h = _t([[-1.0, -1.0]]), _t([[1.0, 1.0]])
    root = rb.ibp_forward_batched(x0l, x0h, gg)
    un = [(L, int(j)) for L in sorted(root)
          for j in ((root[L][0][0] < 0) & (root[L][1][0] > 0)).nonzero().flatten()]
    assert len(un) >= 3
    picks = [un[0], un[len(un) // 2], un[-1]]
    doms = [[(picks[0], s0), (picks[1], s1), (picks[2], s2)]
            for s0 in (0, 1) for s1 in (0, 1) for s2 in (0, 1)]
    B = len(doms)
    clamps = {}
    for b, dom in enumerate(doms):
        for (L, j), side in dom:
            if L not in clamps:
                n_L = root[L][0].shape[1]
                clamps[L] = (torch.full((B, n_L), -inf, dtype=DT),
                             torch.full((B, n_L), inf, dtype=DT))
            clamps[L][1 if side == 0 else 0][b, j] = 0.0
    xl, xh = x0l.expand(B, -1).clone(), x0h.expand(B, -1).clone()
    rootv = {L: (lo[0], hi[0]) for L, (lo, hi) in root.items()}
    sb = rb.split_domain_bounds(xl, xh, gg, rootv, clamps)
    sgn = rb.beta_signs_from_clamps(clamps)
    spec, _ = _util.spec_for(3)
    plain = rb.spec_backward_batched(sb, xl, xh, gg, spec)
    b1, n1 = rb.beta_crown_bound(sb, xl, xh, gg, spec, sgn, n_iters=1, return_trace=True)
    assert n1 == 1
    torch.testing.assert_close(b1, plain)
    prev = b1
    for k in (3, 8, 20):
        bk = rb.beta_crown_bound(sb, xl, xh, gg, spec, sgn, n_iters=k)
        assert bool((bk >= prev - 1e-12).all())
        prev = bk
    g = np.linspace(-1, 1, 161)
    X = torch.tensor(np.stack(np.meshgrid(g, g), -1).reshape(-1, 2), dtype=DT)
    y, pre = rb.point_forward(X, gg)
    Wq = torch.stack([spec[q][0] for q in sorted(spec)])
    vals = y @ Wq.T
    for b, dom in enumerate(doms):
        m = torch.ones(X.shape[0], dtype=torch.bool)
        for (L, j), side in dom:
            m &= (pre[L][:, j] <= 0) if side == 0 else (pre[L][:, j] >= 0)
        if bool(m.any()):
            assert bool((prev[b] <= vals[m].min(0).values + 1e-9).all())


# ------------------------------------------------ CROWN intermediate bounds
def test_crown_intermediate_chunk_invariant_brackets_and_tightens():
    gg = wk.acas_gg(dtype=DT)
    xl, xh = wk.acas_boxes(6, seed=9, dtype=DT)
    xl, xh = xl * 3, xh * 3
    sb, _ = rb.zono_forward_batched(xl, xh, gg)
    t1 = rb.crown_intermediate_batched(gg, xl, xh, chunk=1)
    t2 = rb.crown_intermediate_batched(gg, xl, xh, chunk=4096)
    pts = _util.sample_box(xl, xh, 300, seed=1)
    for L in sb:
        torch.testing.assert_close(t1[L][0], t2[L][0], atol=1e-9, rtol=0)
        torch.testing.assert_close(t1[L][1], t2[L][1], atol=1e-9, rtol=0)
        assert bool((t2[L][0] >= sb[L][0] - 1e-12).all())
        assert bool((t2[L][1] <= sb[L][1] + 1e-12).all())
    assert any(bool((t2[L][1] - t2[L][0] < sb[L][1] - sb[L][0] - 1e-9).any()) for L in sb)
    for b in range(6):
        _, pre = rb.point_forward(pts[b], gg)
        for L in sb:
            assert bool((pre[L] >= t2[L][0][b] - 1e-9).all())
            assert bool((pre[L] <= t2[L][1][b] + 1e-9).all())


def test_crown_intermediate_all_stable_layer_unchanged():
    # positive weights/biases and a positive box: every neuron active
    gg = _chain([np.full((3, 2), 0.5), np.full((3, 3), 0.5), np.full((1, 3), 1.0)],
                [[0.1] * 3, [0.1] * 3, [0.0]])
    xl, xh = _t([[0.5, 0.5]]), _t([[1.0, 1.0]])
    sb, _ = rb.zono_forward_batched(xl, xh, gg)
    t = rb.crown_intermediate_batched(gg, xl, xh)
    for L in sb:
        assert torch.equal(t[L][0], sb[L][0]) and torch.equal(t[L][1], sb[L][1])


def test_crown_intermediate_union_seeding():
    """A neuron unstable in only one domain is re-derived in every domain:
    the batch result differs from per-domain runs only on stable neurons,
    and never in the spec bound."""
    gg = wk.acas_gg(dtype=DT)
    xl, xh = wk.acas_boxes(4, seed=12, dtype=DT)
    xl[0] *= 6
    xh[0] *= 6
    spec_ew, _ = _util.spec_for(5)
    tb = rb.crown_intermediate_batched(gg, xl, xh)
    lb_b = rb.spec_backward_batched(tb, xl, xh, gg, spec_ew)
    for b in range(4):
        ts = rb.crown_intermediate_batched(gg, xl[b:b + 1], xh[b:b + 1])
        lb_s = rb.spec_backward_batched(ts, xl[b:b + 1], xh[b:b + 1], gg, spec_ew)
        torch.testing.assert_close(lb_b[b:b + 1], lb_s, atol=1e-9, rtol=1e-9)
        for L in ts:
            ust = (ts[L][0][0] < 0) & (ts[L][1][0] > 0)
            torch.testing.assert_close(tb[L][0][b][ust], ts[L][0][0][ust], atol=1e-9, rtol=0)


# ---------------------------------------------------------------- alpha
def test_alpha_first_iteration_is_crown_and_best_monotone():
    gg = wk.acas_gg(dtype=DT)
    xl, xh = wk.acas_boxes(8, seed=21, dtype=DT)
    xl, xh = xl * 3, xh * 3
    spec_ew, _ = _util.spec_for(5)
    sb, _ = rb.zono_forward_batched(xl, xh, gg)
    plain = rb.spec_backward_batched(sb, xl, xh, gg, spec_ew)
    b1, n1 = rb.alpha_crown_batched(xl, xh, gg, spec_ew, n_iters=1, return_trace=True)
    torch.testing.assert_close(b1, plain)
    prev = b1
    for k in (3, 6, 12):
        bk = rb.alpha_crown_batched(xl, xh, gg, spec_ew, n_iters=k, early_stop_eps=-1.0)
        assert bool((bk >= prev - 1e-12).all())
        prev = bk
    assert bool((prev > plain + 1e-6).any())
    pts = _util.sample_box(xl, xh, 400, seed=5)
    Wq = torch.stack([spec_ew[q][0] for q in sorted(spec_ew)])
    for b in range(8):
        y, _ = rb.point_forward(pts[b], gg)
        assert bool((prev[b] <= (y @ Wq.T).min(0).values + 1e-9).all())


def test_alpha_early_stop_on_global_max():
    """A batch whose best bound cannot move stops after two iterations
    (verify_zono_bnb.py:5283: global max improvement below eps)."""
    gg = _chain([[[1.0]], [[1.0]]], [[0.5], [0.0]])
    xl, xh = _t([[1.0]]), _t([[2.0]])                    # all stable
    spec = {0: (_t([-1.0]), 0.0)}
    _, n = rb.alpha_crown_batched(xl, xh, gg, spec, n_iters=20, return_trace=True)
    assert n == 2


# ---------------------------------------------------------------- add / sub / mul
def _affine_gg(ops, n_in):
    return wk._finish(ops, n_in, (1, n_in))


def _fc(name, inp, W, b):
    return {'name': name, 'type': 'fc', 'inputs': [inp], 'W': _t(W), 'bias': _t(b)}


def test_affine_ops_hand_computed():
    """x in [1, 3]; z = (-2 x + 5) - 0.5 = -2 x + 4.5 in [-1.5, 2.5]; y =
    relu(z).  IBP and the zonotope give [-1.5, 2.5] (the zonotope: c = 2,
    G = 1, then -4 / -2, +5, -0.5).  The CROWN bound of y uses the lower
    slope 1 (2.5 > 1.5): y >= z = -2 x + 4.5, so A = -2, acc = 4.5,
    lb = -1.5; of -y the upper line 0.625 z + 0.9375: A = 1.25,
    acc = -3.75, lb = -2.5 = -max y (verify_zono_bnb.py:1136-1148,
    3235-3265, 3501-3536, 4470-4518, 4686-4712)."""
    ops = [{'name': 'm', 'type': 'mul', 'inputs': [wk.INPUT_NAME], 'scale': np.array([-2.0])},
           {'name': 'a', 'type': 'add', 'inputs': ['m'], 'is_merge': False,
            'bias': np.array([5.0])},
           {'name': 's', 'type': 'sub', 'inputs': ['a'], 'bias': np.array([0.5])},
           {'name': 'r', 'type': 'relu', 'inputs': ['s'], 'layer_idx': 0},
           _fc('f', 'r', [[1.0]], [0.0])]
    gg = _affine_gg(ops, 1)
    xl, xh = _t([[1.0]]), _t([[3.0]])
    sb = rb.ibp_forward_batched(xl, xh, gg)
    assert torch.equal(sb[0][0], _t([[-1.5]])) and torch.equal(sb[0][1], _t([[2.5]]))
    sbz, (c, G) = rb.zono_forward_batched(xl, xh, gg)
    assert torch.equal(sbz[0][0], _t([[-1.5]])) and torch.equal(sbz[0][1], _t([[2.5]]))
    spec = {0: (_t([1.0]), 0.0), 1: (_t([-1.0]), 0.0)}
    lb, A, acc = rb.spec_backward_batched(sb, xl, xh, gg, spec, return_input_linear=True)
    torch.testing.assert_close(lb, _t([[-1.5, -2.5]]))
    torch.testing.assert_close(A, _t([[[-2.0], [1.25]]]))
    torch.testing.assert_close(acc, _t([[4.5, -3.75]]))


def test_residual_merge_shares_the_fork_generators():
    """z = x + (-1) x over x in [-1, 1]: the input is the fork point, so the
    merge's one generator column is shared and cancels (zonotope [0, 0]);
    interval arithmetic cannot see it ([-2, 2]); the CROWN rows reaching
    the input from both branches sum to 0 (A = 0, lb = 0).  A merge that
    took no shared column, or a backward that kept one branch, fails
    (verify_zono_bnb.py:2387-2428, 3213-3234, 1133-1135, 4462-4469)."""
    ops = [{'name': 'ra', 'type': 'reshape', 'inputs': [wk.INPUT_NAME]},
           {'name': 'nb', 'type': 'mul', 'inputs': [wk.INPUT_NAME], 'scale': np.array([-1.0])},
           {'name': 'z', 'type': 'add', 'inputs': ['ra', 'nb'], 'is_merge': True, 'bias': None},
           {'name': 'r', 'type': 'relu', 'inputs': ['z'], 'layer_idx': 0},
           _fc('f', 'r', [[1.0]], [0.0])]
    gg = _affine_gg(ops, 1)
    assert wk.INPUT_NAME in gg['fork_points']
    xl, xh = _t([[-1.0]]), _t([[1.0]])
    sb = rb.ibp_forward_batched(xl, xh, gg)
    assert torch.equal(sb[0][0], _t([[-2.0]])) and torch.equal(sb[0][1], _t([[2.0]]))
    sbz, _ = rb.zono_forward_batched(xl, xh, gg)
    assert torch.equal(sbz[0][0], _t([[0.0]])) and torch.equal(sbz[0][1], _t([[0.0]]))
    seed = {'z': _t([[[1.0], [-1.0]]])}
    lb, A, acc = rb.spec_backward_batched(sbz, xl, xh, gg, None, return_input_linear=True,
                                          seed_ew_at=seed, seed_acc=_t([[0.0, 0.0]]))
    assert torch.equal(A, _t([[[0.0], [0.0]]])) and torch.equal(lb, _t([[0.0, 0.0]]))


def test_merge_shared_count_at_a_deeper_fork():
    """A fork after a ReLU: both branches carry the ReLU's new generator
    columns as the shared prefix.  _find_shared_gens_count returns the
    fork's count, and the merge's width is K_a + K_b - shared."""
    gg = wk.residual_mlp_gg(3, 6, 2, seed=4, dtype=DT, n_blocks=1)
    xl, xh = _box(3, 5, 0.3, seed=2)
    # the generator counts the forward records, op by op
    counts = {}
    orig = rb.shared_gens_count

    def spy(a, b, gg_, gc):
        counts.update(gc)
        return orig(a, b, gg_, gc)
    rb.shared_gens_count = spy
    try:
        _, (c, G) = rb.zono_forward_batched(xl, xh, gg)
    finally:
        rb.shared_gens_count = orig
    assert orig('b0_fb', 'relu0', gg, counts) == counts['relu0'] > counts[wk.INPUT_NAME]
    # the block's merge: a = b0_fb (relu0's columns, then b0_ra's), b = relu0
    # (exactly the shared ones): the fast path, K_out = K_a
    assert counts['b0_fb'] >= counts['relu0']


def test_affine_ops_equal_the_folded_network():
    """Input normalisation ((x - m) / s), a constant add after a hidden fc
    and a scalar mul by -1 before the last fc, against the same network
    with the constants folded into the fc weights and biases: IBP, the
    zonotope, CROWN intermediate bounds and the spec bound agree to fp64
    rounding.  A wrong sign of sub or mul, or a constant left out of the
    backward's acc, fails here."""
    g = torch.Generator().manual_seed(9)
    n_in, h, n_out = 4, 7, 3
    W0, b0 = torch.randn(h, n_in, generator=g, dtype=DT), torch.randn(h, generator=g, dtype=DT)
    W1, b1 = torch.randn(h, h, generator=g, dtype=DT), torch.randn(h, generator=g, dtype=DT)
    W2, b2 = torch.randn(n_out, h, generator=g, dtype=DT), torch.randn(n_out, generator=g, dtype=DT)
    m = torch.rand(n_in, generator=g, dtype=DT) - 0.5
    s = 0.5 + torch.rand(n_in, generator=g, dtype=DT)
    cst = torch.randn(h, generator=g, dtype=DT) * 0.3
    ops = [{'name': 'ns', 'type': 'sub', 'inputs': [wk.INPUT_NAME], 'bias': m.numpy()},
           {'name': 'nm', 'type': 'mul', 'inputs': ['ns'], 'scale': (1.0 / s).numpy()},
           {'name': 'f0', 'type': 'fc', 'inputs': ['nm'], 'W': W0, 'bias': b0},
           {'name': 'r0', 'type': 'relu', 'inputs': ['f0'], 'layer_idx': 0},
           {'name': 'f1', 'type': 'fc', 'inputs': ['r0'], 'W': W1, 'bias': b1},
           {'name': 'c1', 'type': 'add', 'inputs': ['f1'], 'is_merge': False,
            'bias': cst.numpy()},
           {'name': 'r1', 'type': 'relu', 'inputs': ['c1'], 'layer_idx': 1},
           {'name': 'ng', 'type': 'mul', 'inputs': ['r1'], 'scale': np.array([-1.0])},
           {'name': 'f2', 'type': 'fc', 'inputs': ['ng'], 'W': W2, 'bias': b2}]
    gg = _affine_gg(ops, n_in)
    Wf0 = W0 / s
    folded = wk.mlp_gg([Wf0, W1, -W2], [b0 - Wf0 @ m, b1 + cst, b2], dtype=DT)
    xl, xh = _box(n_in, 6, 0.4, seed=5)
    for f in (lambda g_: rb.ibp_forward_batched(xl, xh, g_),
              lambda g_: rb.zono_forward_batched(xl, xh, g_)[0],
              lambda g_: rb.crown_intermediate_batched(g_, xl, xh)):
        a, b = f(gg), f(folded)
        for L in a:
            for k in (0, 1):
                torch.testing.assert_close(a[L][k], b[L][k], rtol=1e-10, atol=1e-10)
    spec, _ = _util.spec_for(n_out)
    t = rb.crown_intermediate_batched(gg, xl, xh)
    la, Aa, ca = rb.spec_backward_batched(t, xl, xh, gg, spec, return_input_linear=True)
    lb_, Ab, cb = rb.spec_backward_batched(t, xl, xh, folded, spec, return_input_linear=True)
    torch.testing.assert_close(la, lb_, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(Aa, Ab, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(ca, cb, rtol=1e-10, atol=1e-10)


def test_residual_net_bounds_contain_samples():
    """The residual MLP (normalisation constants, two skip blocks, offset,
    negation, output offset): every pre-activation sample lies inside the
    IBP, zonotope and CROWN bounds, CROWN is at least as tight as the
    zonotope, and the spec bound's linear form A x + acc lies below the
    spec value at every sample."""
    gg = wk.residual_mlp_gg(5, 10, 4, seed=3, dtype=DT)
    xl, xh = _box(5, 3, 0.2, seed=6)
    ibp = rb.ibp_forward_batched(xl, xh, gg)
    zono, _ = rb.zono_forward_batched(xl, xh, gg)
    crown = rb.crown_intermediate_batched(gg, xl, xh)
    spec, _ = _util.spec_for(4)
    lb, A, acc = rb.spec_backward_batched(crown, xl, xh, gg, spec, return_input_linear=True)
    X = _util.sample_box(xl, xh, 400, seed=7)
    Wq = torch.stack([spec[q][0] for q in sorted(spec)])
    for b in range(xl.shape[0]):
        y, pre = rb.point_forward(X[b], gg)
        for L in crown:
            for bounds in (ibp, zono, crown):
                assert bool((pre[L] >= bounds[L][0][b] - 1e-9).all())
                assert bool((pre[L] <= bounds[L][1][b] + 1e-9).all())
            assert bool((crown[L][1][b] - crown[L][0][b] <= zono[L][1][b] - zono[L][0][b]
                         + 1e-12).all())
        val = y @ Wq.T
        lin = X[b] @ A[b].T + acc[b]
        assert bool((lin <= val + 1e-9).all())
        assert bool((lb[b] <= val.min(0).values + 1e-9).all())


# ------------------------------------------------ N-D batched MatMul fc
def _nd_boxes(B, seed):
    g = torch.Generator().manual_seed(seed)
    c = torch.rand(B, 21, generator=g, dtype=DT) * 2 - 1
    r = torch.rand(B, 21, generator=g, dtype=DT) * 0.2 + 0.01
    return c - r, c + r


def test_nd_fc_equals_block_diagonal_fc():
    """An fc in the N-D MatMul form (W (16, 7) on a (3, 7) input,
    verify_zono_bnb.py:3145-3168 and 4382-4401) is the plain fc of the
    block-diagonal kron(I_3, W) with the bias repeated: point forward,
    zonotope bounds, generators, CROWN-intermediate bounds and the spec
    bound with its linear form all agree.  A slice order that takes the
    prefix as the inner dim, or a bias summed once instead of per slice,
    fails here."""
    gg = _util.nd_mlp_gg(seed=1)
    gb = _util.nd_as_block_diag(gg)
    xl, xh = _nd_boxes(16, 2)
    pts = _util.sample_box(xl, xh, 50, seed=3).reshape(-1, 21)
    y_nd, pre_nd = rb.point_forward(pts, gg)
    y_bd, pre_bd = rb.point_forward(pts, gb)
    torch.testing.assert_close(y_nd, y_bd, rtol=0, atol=1e-12)
    torch.testing.assert_close(pre_nd[0], pre_bd[0], rtol=0, atol=1e-12)
    sb_nd, (c_nd, G_nd) = rb.zono_forward_batched(xl, xh, gg)
    sb_bd, (c_bd, G_bd) = rb.zono_forward_batched(xl, xh, gb)
    for L in sb_bd:
        for a, b in zip(sb_nd[L], sb_bd[L]):
            torch.testing.assert_close(a, b, rtol=0, atol=1e-12)
    torch.testing.assert_close(G_nd, G_bd, rtol=0, atol=1e-12)
    t_nd = rb.crown_intermediate_batched(gg, xl, xh)
    t_bd = rb.crown_intermediate_batched(gb, xl, xh)
    spec_ew, _ = _util.spec_for(3)
    lb_nd, A_nd, acc_nd = rb.spec_backward_batched(t_nd, xl, xh, gg, spec_ew,
                                                   return_input_linear=True)
    lb_bd, A_bd, acc_bd = rb.spec_backward_batched(t_bd, xl, xh, gb, spec_ew,
                                                   return_input_linear=True)
    for L in t_bd:
        for a, b in zip(t_nd[L], t_bd[L]):
            torch.testing.assert_close(a, b, rtol=0, atol=1e-10)
    torch.testing.assert_close(lb_nd, lb_bd, rtol=0, atol=1e-10)
    torch.testing.assert_close(A_nd, A_bd, rtol=0, atol=1e-10)
    torch.testing.assert_close(acc_nd, acc_bd, rtol=0, atol=1e-10)
    # and the bounds contain the sampled outputs
    Wq = torch.stack([spec_ew[q][0] for q in sorted(spec_ew)])
    val = (y_nd @ Wq.T).reshape(16, 50, -1)
    assert bool((val >= lb_nd.unsqueeze(1) - 1e-9).all())
    for L, (lo, hi) in t_nd.items():
        p = pre_nd[L].reshape(16, 50, -1)
        assert bool((p >= lo.unsqueeze(1) - 1e-9).all() and (p <= hi.unsqueeze(1) + 1e-9).all())


def test_nd_fc_interval_forward_has_no_nd_form():
    """The reference's interval fc is mid @ W.T (verify_zono_bnb.py:
    1108-1113): an N-D fc fails there with torch's shape error, and so
    does the oracle."""
    gg = _util.nd_mlp_gg(seed=1)
    xl, xh = _nd_boxes(4, 2)
    with pytest.raises(RuntimeError):
        rb.ibp_forward_batched(xl, xh, gg)


def test_validate_gg_widths_and_mismatches():
    """The drop-in checks every node's width before any launch
    (vibecheck_amd.verify_zono_bnb.validate_gg, shapes only, no device):
    the N-D fc form gives 3 x 16; an input, fc, conv or merge width that
    does not chain raises ValueError (the kernels would otherwise read a
    wider tensor as rows of W.shape[1]); an unknown op raises
    NotImplementedError."""
    import copy
    from vibecheck_amd.verify_zono_bnb import validate_gg
    gg = _util.nd_mlp_gg(seed=1)
    w = validate_gg(gg)
    assert w == {'input': 21, 'fc0': 48, 'relu0': 48, 'flat': 48, 'fc1': 6,
                 'relu1': 6, 'fc2': 3}
    with pytest.raises(ValueError):
        validate_gg(gg, n_in=20)
    bad = copy.deepcopy(gg)
    bad['ops'][0]['in_shapes_nd'] = [(7, 3)]           # last dim is not W's 7
    with pytest.raises(ValueError):
        validate_gg(bad)
    bad = copy.deepcopy(gg)
    del bad['ops'][0]['in_shapes_nd']                   # 21 values read as rows of 7
    with pytest.raises(ValueError):
        validate_gg(bad)
    bad = copy.deepcopy(gg)
    bad['ops'][3]['W'] = torch.zeros(6, 47, dtype=DT)
    with pytest.raises(ValueError):
        validate_gg(bad)
    assert validate_gg(wk.acas_gg(dtype=DT))['fc6'] == 5
    cnn = _util.tiny_cnn()
    wc = validate_gg(cnn)
    assert wc[cnn['ops'][-1]['name']] == 2
    bad = copy.deepcopy(cnn)
    conv = next(op for op in bad['ops'] if op['type'] == 'conv')
    conv['in_shape'] = (2, 6, 5)
    with pytest.raises(ValueError):
        validate_gg(bad)
    res = wk.residual_mlp_gg(4, 8, 3, seed=0, dtype=DT)
    validate_gg(res)
    bad = copy.deepcopy(res)
    merge = next(op for op in bad['ops'] if op['type'] == 'add' and op.get('is_merge'))
    merge['inputs'] = [merge['inputs'][0], bad['input_name']]
    with pytest.raises(ValueError):
        validate_gg(bad)
    bad = copy.deepcopy(gg)
    bad['ops'][2]['type'] = 'softmax'
    with pytest.raises(NotImplementedError):
        validate_gg(bad)
