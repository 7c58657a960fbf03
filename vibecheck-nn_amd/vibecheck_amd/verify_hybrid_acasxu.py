"""Hybrid per-query alpha-CROWN freeze / replay verifier on the HIP library
(verify_hybrid_acasxu.py:164-539).

  - ``_full_freeze`` (verify_hybrid_acasxu.py:164-257): a batch of leaves
    gets alpha-optimized intermediate bounds, layer by layer.  For ReLU
    layer L the rows [+I; -I] (Q = 2 n_L) are seeded at the op feeding the
    ReLU; every ReLU k below L has its own alpha per (leaf, row, neuron),
    initialised to the CROWN lower slopes; Adam on -sum(lb) with the slopes
    clamped to [0, 1], the learning rate decayed by 0.98 per iteration and
    the early stop on the sum of the running best; the layer's bounds are
    then intersected with the best seeded bounds.  The same per-query loop
    then runs for the spec rows, with the deadline checked per iteration.
  - ``_replay_batched`` (verify_hybrid_acasxu.py:260-318): the frozen layer
    alphas re-tighten every layer of a batch of leaves without optimisation,
    then the spec alpha, warm-started from the frozen one, takes
    ``spec_iters`` Adam steps; the best bound per (leaf, query) and, per
    leaf, the input linearization of its last improving evaluation are
    returned.
  - ``verify_hybrid`` (verify_hybrid_acasxu.py:321-527): the fan-out to
    ``init_leaves`` boxes, one freeze over them, then a LIFO worklist of
    boxes bounded by replay with the alphas of the box each descends from.

Every bound, gradient, Adam step and bookkeeping update is a launch of the
HIP library (the shared backward and gradient sweep with per-row alpha,
vc_bound_tighten, vc_best_sum, vc_best_rows_with_A, vc_adam_step); torch
holds the device memory.  Differences from the reference, by design:
  - the replay bounds every leaf of a batch in one call, each leaf with the
    alphas of its own group: the backward reads the frozen layer alphas
    through the leaf's group index, and the spec alphas (which Adam then
    moves per leaf) are gathered into per-leaf rows (the reference calls the
    replay once per group; the leaves' computations are independent, so the
    bounds are the same);
  - the replay's last iteration computes no gradient and takes no Adam
    step (neither reaches a returned value);
  - the early stop reads the sum of the running best accumulated in fp64
    and rounded once to fp32 (the reference sums in fp32 in torch's order,
    which lies within a few fp32 ulps of that value; both see the sum at
    fp32 resolution, so they stop alike unless an improvement is within
    those few ulps);
  - the sign-gradient PGD attacks (verify_hybrid_acasxu.py:39-161) are not
    part of this module: ``verify_hybrid`` runs as the reference does with
    ``disable_sat_finding``, so its verdicts are 'unsat' and 'unknown';
  - a box whose widest width is zero cannot be bisected: the driver
    answers 'unknown' there (the reference would bisect it into copies of
    itself until the timeout, also ending 'unknown').
The alpha gradient sweep covers fc/ReLU chains (the ACAS-Xu networks this
path is for); other graphs raise NotImplementedError.
"""
import time

import torch

from ._lib import call, f32, ptr, stream
from . import verify_zono_bnb as vz
from .verify_graph import DisjunctTable, _closure, _compact, _gather

_B1, _B2, _EPS = 0.9, 0.999, 1e-8


def _relu_feeds(gg):
    """{layer index L: the name of the op whose output feeds ReLU L}."""
    return {op['layer_idx']: op['inputs'][0] for op in gg['ops']
            if op['type'] == 'relu' and 'layer_idx' in op}


def _bound_rows(n, dev):
    """The seeded rows [+I; -I] (2n, n) and their zero offsets."""
    eye = torch.eye(n, device=dev)
    return torch.cat([eye, -eye], dim=0).contiguous(), torch.zeros(2 * n, device=dev)


def _per_leaf(a, B):
    """An alpha (1 or B, Q, n) as B per-leaf rows (B, Q, n), contiguous fp32."""
    a = f32(a)
    if a.shape[0] == B:
        return a.contiguous()
    if a.shape[0] != 1:
        raise ValueError(f'vibecheck_amd: alpha of {a.shape[0]} leaves for a batch of {B}')
    return a.expand(B, -1, -1).contiguous()


class _AlphaSet:
    """Per-row alphas {k: (B, Q, n_k)} in one flat buffer with their
    gradient and the Adam moments (torch.optim.Adam defaults: betas
    (0.9, 0.999), eps 1e-8, no weight decay), projected onto [0, 1] after
    every step."""

    def __init__(self, tight, keys, B, Q, dev, init_from=None):
        sizes = [B * Q * tight[k][0].shape[1] for k in keys]
        self.total = sum(sizes)
        self.flat = torch.empty(self.total, device=dev)
        self.grad = torch.zeros(self.total, device=dev)
        self.m1 = torch.zeros(self.total, device=dev)
        self.m2 = torch.zeros(self.total, device=dev)
        self.alpha, self.galpha = {}, {}
        self.step = 0
        st = stream()
        off = 0
        for k, sz in zip(keys, sizes):
            n = tight[k][0].shape[1]
            self.alpha[k] = self.flat[off:off + sz].view(B, Q, n)
            self.galpha[k] = self.grad[off:off + sz].view(B, Q, n)
            if init_from is None:
                # CROWN's lower slopes, (up_s > 0.5) on unstable neurons
                lo, hi = f32(tight[k][0]), f32(tight[k][1])
                a0 = torch.empty(B, n, device=dev)
                call('vc_alpha_init', ptr(lo), ptr(hi), B * n, ptr(a0), st)
                self.alpha[k].copy_(a0.unsqueeze(1).expand(B, Q, n))
            else:
                self.alpha[k].copy_(_per_leaf(init_from[k], B))
            off += sz

    def adam(self, lr):
        self.step += 1
        bc1 = 1 - _B1 ** self.step
        bc2 = 1 - _B2 ** self.step
        call('vc_adam_step', ptr(self.flat), ptr(self.grad), ptr(self.m1), ptr(self.m2),
             self.total, _B1, _B2, _EPS, lr / bc1, bc2 ** 0.5, 0.0, 1.0, stream())


def _optimise(ps, evaluate, best, n_iters, lr, lr_decay, early_stop_eps, deadline=None):
    """The freeze's Adam loop (verify_hybrid_acasxu.py:200-223, 234-252):
    evaluate, best = max(best, lb), Adam step, stop when the sum of the best
    improved by less than ``early_stop_eps`` (from the second iteration),
    decay lr.  ``deadline`` is checked before every iteration but the
    first.  Returns the number of evaluations."""
    total = torch.empty(1, dtype=torch.float64, device=best.device)
    prev = -float('inf')
    cur_lr = float(lr)
    n_eval = 0
    for it in range(n_iters):
        if deadline is not None and it > 0 and time.perf_counter() > deadline:
            break
        lb = evaluate()
        n_eval += 1
        call('vc_best_sum', ptr(best), ptr(lb.contiguous()), best.numel(),
             1 if it == 0 else 0, ptr(total), stream())
        cur = float(total.item())
        ps.adam(cur_lr)
        if it > 0 and cur - prev < early_stop_eps:
            break
        prev = cur
        cur_lr *= lr_decay
    return n_eval


def _tighten_layer(tight, L, sl):
    lo, hi = tight[L]
    call('vc_bound_tighten', ptr(lo), ptr(hi), ptr(sl.contiguous()), lo.shape[0],
         lo.shape[1], stream())


def _zono_tight(xl, xh, gg, device, dtype):
    """Zonotope pre-activation bounds, writable copies: only the bounds are
    needed, so narrow MLPs take the bounds-only whole-network kernel."""
    sb = vz._zono_sb(gg, xl, xh, device, dtype)
    return {L: (f32(lo).clone(), f32(hi).clone()) for L, (lo, hi) in sb.items()}


def _full_freeze(xl, xh, gg, spec_ew, device, dtype, n_iters_per_layer=100,
                 n_iters_spec=100, lr=0.25, deadline=None, lr_decay=0.98,
                 early_stop_eps=1e-6):
    """Per-query alpha-CROWN layer-wise tightening, then per-query spec
    alpha-CROWN, on a batch of B leaves (verify_hybrid_acasxu.py:164-257).

    Returns (tight {L: (lo, hi) (B, n_L)}, alpha_per_layer {L: {k: (B, 2 n_L,
    n_k)}}, alpha_spec {L: (B, Q, n_L)}, best_spec (B, Q)).  ``lr_decay`` and
    ``early_stop_eps`` are extensions (the reference fixes 0.98 and 1e-6).
    """
    vz._check_dtype(dtype)
    xl, xh = f32(xl).contiguous(), f32(xh).contiguous()
    B = xl.shape[0]
    dev = xl.device
    tight = _zono_tight(xl, xh, gg, device, dtype)
    order = sorted(tight)
    if not order:
        raise ValueError('vibecheck_amd: the hybrid freeze needs a ReLU layer')
    if n_iters_spec < 1:
        raise ValueError('vibecheck_amd: the spec loop needs at least one iteration')
    feeds = _relu_feeds(gg)
    alpha_per_layer = {}
    for L in order:
        if deadline is not None and time.perf_counter() > deadline:
            alpha_per_layer[L] = {}
            continue
        keys = [k for k in order if k < L]
        if keys:
            n = tight[L][0].shape[1]
            Wq, bq = _bound_rows(n, dev)
            ps = _AlphaSet(tight, keys, B, 2 * n, dev)
            best = torch.empty(B, 2 * n, device=dev)
            _optimise(ps, lambda: vz._alpha_backward_and_grad(
                tight, xl, xh, gg, Wq, bq, ps.alpha, True, ps.galpha, seed_name=feeds[L]),
                best, n_iters_per_layer, lr, lr_decay, early_stop_eps)
            if n_iters_per_layer > 0:
                _tighten_layer(tight, L, best)
            alpha_per_layer[L] = {k: ps.alpha[k].clone() for k in keys}
        else:
            alpha_per_layer[L] = {}
    Wq, bq = vz._spec_rows(spec_ew, dev)
    Q = Wq.shape[0]
    ps = _AlphaSet(tight, order, B, Q, dev)
    best_spec = torch.empty(B, Q, device=dev)
    _optimise(ps, lambda: vz._alpha_backward_and_grad(
        tight, xl, xh, gg, Wq, bq, ps.alpha, True, ps.galpha),
        best_spec, n_iters_spec, lr, lr_decay, early_stop_eps, deadline)
    alpha_spec = {k: ps.alpha[k].clone() for k in order}
    return tight, alpha_per_layer, alpha_spec, best_spec


def _replay_batched(xl_b, xh_b, gg, spec_ew, alpha_layer_b, alpha_spec_b,
                    device, dtype, spec_iters=10, spec_lr=0.1, return_tight=False,
                    group=None, check_groups=True):
    """Zonotope bounds, frozen-alpha layer tightening, per-leaf spec alpha
    Adam (verify_hybrid_acasxu.py:260-318).

    ``alpha_layer_b`` {L: {k: (1 or B, 2 n_L, n_k)}}, ``alpha_spec_b``
    {L: (1 or B, Q, n_L)}: one group's alphas (leading 1, expanded over the
    batch) or per-leaf alphas (leading B).  ``group`` (extension, (B,)
    int64): the alphas hold G groups (leading G) and leaf b takes those of
    group[b]; the layer alphas are then read in place by the backward
    (vc_backward_fc_grouped), without per-leaf copies.  Indices outside
    [0, G) raise ValueError (one host read; ``check_groups=False`` skips it
    for callers whose indices are valid by construction, and such an index
    then reads group 0, never memory past the alphas).  Returns (best (B, Q),
    best_A (B, Q, n_in)); ``return_tight`` (extension) also returns the
    tightened layer bounds.
    """
    vz._check_dtype(dtype)
    xl, xh = f32(xl_b).contiguous(), f32(xh_b).contiguous()
    B, n_in = xl.shape
    dev = xl.device
    if group is not None:
        group = group.to(device=dev, dtype=torch.int64).contiguous()
        G = next(iter(alpha_spec_b.values())).shape[0]
        if group.shape != (B,):
            raise ValueError('vibecheck_amd: group must hold one index per leaf')
        # every read below goes through the clamped indices; the flag says
        # whether any was out of range (one host read, skipped by the
        # driver, whose indices come from its own compaction)
        bad = torch.zeros(1, dtype=torch.int32, device=dev)
        safe = torch.empty_like(group)
        call('vc_group_clamp', ptr(group), B, G, ptr(safe), ptr(bad), stream())
        if check_groups and int(bad.item()):
            raise ValueError(f'vibecheck_amd: group index outside [0, {G})')
        group = safe
        alpha_spec_b = {k: _gather(f32(a).reshape(G, -1), group).view(B, *a.shape[1:])
                        for k, a in alpha_spec_b.items()}
    tight = _zono_tight(xl, xh, gg, device, dtype)
    feeds = _relu_feeds(gg)
    for L in sorted(tight):
        if not alpha_layer_b.get(L):
            continue
        n = tight[L][0].shape[1]
        Wq, bq = _bound_rows(n, dev)
        if group is not None:
            alpha = {k: (f32(a).contiguous(), group) for k, a in alpha_layer_b[L].items()}
        else:
            alpha = {k: _per_leaf(a, B) for k, a in alpha_layer_b[L].items()}
        sl = vz._alpha_backward_and_grad(tight, xl, xh, gg, Wq, bq, alpha, False, None,
                                         seed_name=feeds[L])
        _tighten_layer(tight, L, sl)
    Wq, bq = vz._spec_rows(spec_ew, dev)
    Q = Wq.shape[0]
    ps = _AlphaSet(tight, sorted(alpha_spec_b), B, Q, dev, init_from=alpha_spec_b)
    best = torch.empty(B, Q, device=dev)
    best_A = torch.empty(B, Q, n_in, device=dev)
    n_it = max(1, int(spec_iters))
    for it in range(n_it):
        last = it == n_it - 1
        lb, A = vz._alpha_backward_and_grad(tight, xl, xh, gg, Wq, bq, ps.alpha, not last,
                                            ps.galpha, want_A=True)
        call('vc_best_rows_with_A', ptr(best), ptr(lb.contiguous()), ptr(best_A), ptr(A),
             B, Q, n_in, 1 if it == 0 else 0, stream())
        if not last:
            ps.adam(spec_lr)
    if return_tight:
        return best, best_A, tight
    return best, best_A


def _bisect_widest(xl, xh):
    """Each box split at the middle of its widest dimension (lowest index on
    ties) into (low, high) children, adjacent and in box order
    (verify_hybrid_acasxu.py:378-389, 500-514).  Returns (children xl, xh,
    number of boxes of zero width, which have no children)."""
    B, n = xl.shape
    dev = xl.device
    st = stream()
    dims = torch.empty(B, 1, dtype=torch.int64, device=dev)
    usable = torch.empty(B, dtype=torch.bool, device=dev)
    call('vc_widest_axis', ptr(xl), ptr(xh), B, n, ptr(dims), ptr(usable), st)
    plan = torch.empty(B + 2, dtype=torch.int64, device=dev)
    call('vc_split_multi_plan', ptr(xl), ptr(xh), ptr(dims), B, n, 1, ptr(plan),
         ptr(plan[B + 1:]), st)
    total, n_deg = plan[B:].tolist()
    kl = torch.empty(total, n, device=dev)
    kh = torch.empty(total, n, device=dev)
    if total > 0:
        call('vc_split_multi', ptr(xl), ptr(xh), ptr(dims), ptr(plan), B, n, 1, ptr(kl),
             ptr(kh), st)
    return kl, kh, n_deg


def _setting(settings, name, default):
    if settings is None:
        return default
    if isinstance(settings, dict):
        return settings.get(name, default)
    return getattr(settings, name, default)


def _gather_alphas(alpha_layer, alpha_spec, gid):
    """Per-leaf alphas of the groups ``gid`` (B,) picks."""
    def g(a):
        return _gather(a.reshape(a.shape[0], -1), gid).view(gid.numel(), *a.shape[1:])
    return ({L: {k: g(a) for k, a in d.items()} for L, d in alpha_layer.items()},
            {L: g(a) for L, a in alpha_spec.items()})


def verify_hybrid(gg, spec, settings=None, timeout=120.0, init_leaves=32, batch=4096,
                  verbose=False, spec_iters=10, spec_lr=0.1):
    """The hybrid BaB driver (verify_hybrid_acasxu.py:321-527) without its
    PGD phases.  ``gg`` is the network's op graph (the reference builds it
    with ``graph.gpu_graph``).  Knob read from ``settings``:
    hybrid_freeze_iters (default 100).  Returns {'verdict': 'unsat' |
    'unknown', 'time', 'phase', ...}."""
    t_start = time.perf_counter()
    freeze_iters = int(_setting(settings, 'hybrid_freeze_iters', 100))
    dev = next(op['W'].device for op in gg['ops'] if op['type'] == 'fc')
    dtype = torch.float32
    n_output = next(int(op['W'].shape[0]) for op in reversed(gg['ops']) if op['type'] == 'fc')
    queries = spec.as_linear_queries(n_output)
    spec_ew = {qi: (torch.as_tensor(w, dtype=dtype, device=dev).flatten(), float(b))
               for qi, (di, w, b) in enumerate(queries)}
    disj_q_idx = {}
    for qi, (di, _, _) in enumerate(queries):
        disj_q_idx.setdefault(di, []).append(qi)
    table = DisjunctTable(disj_q_idx, dev)
    xl = torch.as_tensor(spec.x_lo, dtype=dtype, device=dev).flatten()[None, :].contiguous()
    xh = torch.as_tensor(spec.x_hi, dtype=dtype, device=dev).flatten()[None, :].contiguous()

    # fan-out: bisect every box on its widest dimension until there are
    # init_leaves of them (children adjacent, so the first init_leaves of a
    # full round are the reference's boxes)
    while xl.shape[0] < init_leaves:
        kl, kh, n_deg = _bisect_widest(xl, xh)
        if n_deg:
            break
        xl, xh = kl[:init_leaves].contiguous(), kh[:init_leaves].contiguous()
    n_init = xl.shape[0]
    try:
        _, alpha_layer, alpha_spec, best = _full_freeze(
            xl, xh, gg, spec_ew, dev, dtype, n_iters_per_layer=freeze_iters,
            n_iters_spec=freeze_iters, deadline=t_start + 0.8 * timeout)
    except torch.cuda.OutOfMemoryError:
        return {'verdict': 'unknown', 'time': time.perf_counter() - t_start,
                'phase': 'freeze_oom'}
    closed = _closure(best, table)
    open_idx = _compact(closed, select_zero=True)
    wl_xl, wl_xh, wl_gid = xl[open_idx], xh[open_idx], open_idx.clone()
    n_evaluated = n_init
    n_closed = n_init - open_idx.numel()
    if verbose:
        print(f'  freeze closure: {n_closed}/{n_init} open={open_idx.numel()}')
    cur_batch = batch
    iters = 0
    while wl_xl.shape[0] > 0:
        if time.perf_counter() - t_start > timeout - 0.5:
            return {'verdict': 'unknown', 'time': time.perf_counter() - t_start,
                    'phase': 'bab_timeout', 'residual': wl_xl.shape[0],
                    'evaluated': n_evaluated, 'closed': n_closed}
        N = wl_xl.shape[0]
        take = min(cur_batch, N)
        bxl, bxh, bgid = (t[N - take:].contiguous() for t in (wl_xl, wl_xh, wl_gid))
        try:
            # the group ids are freeze-leaf indices from this driver's own
            # compaction (and their children's copies): in range by
            # construction, so the replay's host check is skipped
            best, _ = _replay_batched(bxl, bxh, gg, spec_ew, alpha_layer, alpha_spec, dev,
                                      dtype, spec_iters=spec_iters, spec_lr=spec_lr,
                                      group=bgid, check_groups=False)
        except torch.cuda.OutOfMemoryError:
            if cur_batch <= 8:
                return {'verdict': 'unknown', 'time': time.perf_counter() - t_start,
                        'phase': 'bab_oom'}
            cur_batch = max(8, cur_batch // 2)
            continue
        wl_xl, wl_xh, wl_gid = wl_xl[:N - take], wl_xh[:N - take], wl_gid[:N - take]
        n_evaluated += take
        closed = _closure(best, table)
        open_idx = _compact(closed, select_zero=True)
        n_closed += take - open_idx.numel()
        if verbose and iters % 10 == 0:
            print(f'    iter {iters} t={time.perf_counter() - t_start:.1f} '
                  f'wl={wl_xl.shape[0]} eval={n_evaluated} closed={n_closed}')
        if open_idx.numel() > 0:
            kl, kh, n_deg = _bisect_widest(bxl[open_idx].contiguous(),
                                           bxh[open_idx].contiguous())
            if n_deg:
                return {'verdict': 'unknown', 'time': time.perf_counter() - t_start,
                        'phase': 'bab_point_box', 'evaluated': n_evaluated,
                        'closed': n_closed}
            wl_xl = torch.cat([wl_xl, kl])
            wl_xh = torch.cat([wl_xh, kh])
            wl_gid = torch.cat([wl_gid, bgid[open_idx].repeat_interleave(2)])
        iters += 1
    return {'verdict': 'unsat', 'time': time.perf_counter() - t_start,
            'phase': 'bab_complete', 'evaluated': n_evaluated, 'closed': n_closed,
            'bab_iters': iters}
