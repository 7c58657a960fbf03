"""Oracle: input-split branch-and-bound step restated in PyTorch (CPU).

Test infrastructure: see the package docstring.  Follows
``_input_split_batched_inner`` and ``_clip_box_by_halfspaces_batched`` of the
reference (verify_graph.py:12363-12426, 12511-13464) for the settings this
engine supports: CROWN or zonotope intermediate bounds, domain clipping,
batched alpha-CROWN on unclosed leaves, widest-dimension or SB (sum or
margin score) split dimensions, bisection or the 2^K-way split on the top K
dimensions.  Root PGD, leaf PGD, MILP/LP escalation are not part of it.
"""
import time

import torch

from .ref_bound import (alpha_crown_batched, crown_intermediate_batched,
                        spec_backward_batched, zono_forward_batched)


def closure(lb, disj_q_idx):
    """A domain is closed iff every disjunct has a query with lb > 0
    (verify_graph.py:12899-12908)."""
    B = lb.shape[0]
    if not disj_q_idx:
        return torch.ones(B, dtype=torch.bool)
    masks = [(lb[:, q] > 0).any(dim=1) for q in disj_q_idx.values()]
    return torch.stack(masks, dim=1).all(dim=1)


def clip_box_by_halfspaces_batched(xl, xh, A, b):
    """Bounding box of {x in [xl, xh] : A_q.x + b_q <= 0 for all q}
    (verify_graph.py:12363-12426).  Returns (xl', xh', feasible)."""
    B, Q, n = A.shape
    Ap = A.clamp(min=0)
    An = A.clamp(max=0)
    total = ((Ap * xl.unsqueeze(1)).sum(dim=-1)
             + (An * xh.unsqueeze(1)).sum(dim=-1))
    contrib = Ap * xl.unsqueeze(1) + An * xh.unsqueeze(1)
    other = total.unsqueeze(-1) - contrib
    nz = A.abs() > 1e-12
    safe = torch.where(nz, A, torch.ones_like(A))
    thr = (-b.unsqueeze(-1) - other) / safe
    pos = A > 1e-12
    neg = A < -1e-12
    xh_q = torch.where(pos, thr, xh.unsqueeze(1).expand(B, Q, n))
    xl_q = torch.where(neg, thr, xl.unsqueeze(1).expand(B, Q, n))
    xh_new = torch.minimum(xh_q.min(dim=1).values, xh)
    xl_new = torch.maximum(xl_q.max(dim=1).values, xl)
    empty_h = (total + b > 0).any(dim=1)
    empty_b = (xl_new > xh_new).any(dim=-1)
    return xl_new, xh_new, ~(empty_h | empty_b)


def clip_leaves(xl, xh, A, b, disj_q_idx):
    """One clip iteration over unclosed leaves; per-disjunct clip and the
    bounding box of the union for multi-disjunct specs
    (verify_graph.py:13036-13074)."""
    if len(disj_q_idx) <= 1:
        return clip_box_by_halfspaces_batched(xl, xh, A, b)
    pl, ph, pf = [], [], []
    for q in disj_q_idx.values():
        qt = torch.tensor(q, dtype=torch.long)
        l_d, h_d, f_d = clip_box_by_halfspaces_batched(
            xl, xh, A.index_select(1, qt), b.index_select(1, qt))
        pl.append(torch.where(f_d.unsqueeze(-1), l_d,
                              torch.full_like(l_d, float('inf'))))
        ph.append(torch.where(f_d.unsqueeze(-1), h_d,
                              torch.full_like(h_d, float('-inf'))))
        pf.append(f_d)
    xl_n = torch.stack(pl).min(dim=0).values
    xh_n = torch.stack(ph).max(dim=0).values
    feas = torch.stack(pf).any(dim=0)
    xl_n = torch.where(feas.unsqueeze(-1), xl_n, xl)
    xh_n = torch.where(feas.unsqueeze(-1), xh_n, xh)
    return xl_n, xh_n, feas


def clip_iterated(xl, xh, A, b, disj_q_idx, clip_iters=1):
    """The clip loop (verify_graph.py:13036-13081): clip_leaves with the same
    halfspaces until no box of the batch shrinks, at most clip_iters times;
    the feasibility is the last iteration's."""
    xl_c, xh_c, feas = xl, xh, None
    for _ in range(max(1, int(clip_iters))):
        xl_n, xh_n, feas = clip_leaves(xl_c, xh_c, A, b, disj_q_idx)
        shrunk = bool(((xl_n > xl_c) | (xh_n < xh_c)).any())
        xl_c, xh_c = xl_n, xh_n
        if not shrunk:
            break
    return xl_c, xh_c, feas


def widest_axis(xl, xh):
    """First index of the maximum width (verify_graph.py:13291)."""
    return (xh - xl).argmax(dim=1)


def bisect(xl, xh, ax):
    """Vectorized 2-way split (verify_graph.py:13366-13382).

    Returns (n_degenerate, low (xl, xh), high (xl, xh)); leaves whose split
    width is <= 1e-12 are dropped and counted.
    """
    lo_ax = xl.gather(1, ax.unsqueeze(1)).squeeze(1)
    hi_ax = xh.gather(1, ax.unsqueeze(1)).squeeze(1)
    usable = (hi_ax - lo_ax) > 1e-12
    n_deg = int((~usable).sum().item())
    u = usable.nonzero(as_tuple=True)[0]
    xl_u, xh_u = xl[u], xh[u]
    a = ax[u].unsqueeze(1)
    mid = ((lo_ax[u] + hi_ax[u]) * 0.5).unsqueeze(1)
    xh_low = xh_u.clone().scatter_(1, a, mid)
    xl_high = xl_u.clone().scatter_(1, a, mid)
    return n_deg, (xl_u, xh_low), (xl_high, xh_u)


def sb_scores(xl, xh, A, lb, margin=False, thr=0.01, mw=1.0):
    """Split-dimension scores of SB branching (verify_graph.py:13255-13285):
    widths * sum_q |A_q| (the default 'sum' form) or, with ``margin``,
    max_q (|A_q|.clamp(thr) * widths / 2 + lb_q * mw).  xl, xh (B, n);
    A (B, Q, n); lb (B, Q)."""
    widths = xh - xl
    if margin:
        base = A.abs().clamp(min=thr) * widths.unsqueeze(1) / 2
        base = base + lb.unsqueeze(-1) * mw
        return base.amax(dim=1)
    sens = A.abs().sum(dim=1)
    return widths * sens


def top_dims(scores, K):
    """The K best dimensions per row, best first (verify_graph.py:13291,
    13348-13351): argmax (first maximum) for K = 1; for K > 1 a stable
    descending sort, i.e. torch.topk's order with ties broken by the lower
    index."""
    if K == 1:
        return scores.argmax(dim=1, keepdim=True)
    return torch.sort(scores, dim=1, descending=True, stable=True).indices[:, :K]


def split_multi(xl, xh, dims):
    """2^K-way split of every leaf on its K dimensions dims (B, K)
    (verify_graph.py:13392-13420): the dimensions wider than 1e-12, in
    order, each halved at (lo + hi) / 2; child ``combo`` takes the high
    half of usable dimension k when bit k is set.  Leaves without a usable
    dimension are dropped and counted.  Returns (n_degenerate, (xl, xh) of
    the children, leaf-major)."""
    kids_l, kids_h = [], []
    n_deg = 0
    for i in range(xl.shape[0]):
        usable, mids = [], []
        for k in range(dims.shape[1]):
            d = int(dims[i, k])
            if float(xh[i, d] - xl[i, d]) > 1e-12:
                usable.append(d)
                mids.append(float((xl[i, d] + xh[i, d]) / 2))
        if not usable:
            n_deg += 1
            continue
        for combo in range(1 << len(usable)):
            cl, ch = xl[i].clone(), xh[i].clone()
            for k, d in enumerate(usable):
                if (combo >> k) & 1:
                    cl[d] = mids[k]
                else:
                    ch[d] = mids[k]
            kids_l.append(cl)
            kids_h.append(ch)
    n = xl.shape[1]
    if not kids_l:
        return n_deg, (xl.new_zeros(0, n), xh.new_zeros(0, n))
    return n_deg, (torch.stack(kids_l), torch.stack(kids_h))


class ChunkWorklist:
    """LIFO worklist of 2-D chunks (verify_graph.py:12695-12726)."""

    def __init__(self, xl0, xh0):
        self.xl = [xl0.reshape(1, -1)]
        self.xh = [xh0.reshape(1, -1)]

    def size(self):
        return sum(int(c.shape[0]) for c in self.xl)

    def push(self, xl, xh):
        self.xl.append(xl)
        self.xh.append(xh)

    def pop(self, n):
        """Pop exactly n rows from the end; parts are concatenated in pop
        order (last chunk first), a partial chunk gives its LAST rows."""
        got = 0
        pl, ph = [], []
        while got < n:
            cl, ch = self.xl[-1], self.xh[-1]
            m = int(cl.shape[0])
            if got + m <= n:
                pl.append(cl)
                ph.append(ch)
                self.xl.pop()
                self.xh.pop()
                got += m
            else:
                need = n - got
                pl.append(cl[-need:])
                ph.append(ch[-need:])
                self.xl[-1] = cl[:-need]
                self.xh[-1] = ch[:-need]
                got = n
        if len(pl) == 1:
            return pl[0], ph[0]
        return torch.cat(pl, 0), torch.cat(ph, 0)

    def __bool__(self):
        return bool(self.xl)


def bound_batch(xl, xh, gg, spec_ew, crown_intermediate=True,
                clip_enabled=True):
    """The 'bound' phase of one BaB iteration (verify_graph.py:12855-12871).
    Returns (lb, A, acc) (A, acc are None without clipping)."""
    if crown_intermediate:
        sb = crown_intermediate_batched(gg, xl, xh)
    else:
        sb, _ = zono_forward_batched(xl, xh, gg)
    if clip_enabled:
        return spec_backward_batched(sb, xl, xh, gg, spec_ew,
                                     return_input_linear=True)
    return spec_backward_batched(sb, xl, xh, gg, spec_ew), None, None


def band_select(lb, closed, disj_q_idx, eps, max_leaves):
    """Leaves of the alpha boundary band (verify_graph.py:12938-12950):
    unclosed with worst disjunct's best bound > -eps, in descending order of
    that bound, at most max_leaves.  Equal bounds keep their ascending leaf
    order (a stable sort: the reference's argsort leaves ties open)."""
    per_disj = [lb[:, q].max(dim=1).values for q in disj_q_idx.values()]
    worst = torch.stack(per_disj, dim=1).min(dim=1).values
    idx = ((~closed) & (worst > -eps)).nonzero(as_tuple=True)[0]
    order = worst[idx].argsort(descending=True, stable=True)
    return idx[order[:max_leaves]]


def alpha_on_leaves(lb, xl, xh, gg, spec_ew, disj_q_idx, closed,
                    alpha_iters, alpha_all, alpha_eps, alpha_max_leaves,
                    lr=0.25, lr_decay=0.98):
    """Batched alpha-CROWN on unclosed leaves, merged by max
    (verify_graph.py:12927-12975).  Returns (lb, closed, n_alpha_leaves,
    n_alpha_iters)."""
    if not (alpha_iters > 0 and (alpha_all or alpha_eps > 0)
            and not bool(closed.all())):
        return lb, closed, 0, 0
    idx = (~closed).nonzero(as_tuple=True)[0] if alpha_all else \
        band_select(lb, closed, disj_q_idx, alpha_eps, alpha_max_leaves)
    if idx.numel() == 0:
        return lb, closed, 0, 0
    new, n_it = alpha_crown_batched(xl[idx], xh[idx], gg, spec_ew,
                                    n_iters=alpha_iters, lr=lr,
                                    lr_decay=lr_decay, return_trace=True)
    lb = lb.clone()
    lb[idx] = torch.maximum(lb[idx], new)
    return lb, closure(lb, disj_q_idx), int(idx.numel()), n_it


def bab_step(xl, xh, gg, spec_ew, disj_q_idx, crown_intermediate=True,
             clip_enabled=True, alpha_iters=0, alpha_all=False, alpha_eps=0.0,
             alpha_max_leaves=200, alpha_lr=0.25, alpha_lr_decay=0.98,
             branch_sb=False, sb_margin=False, sb_thr=0.01, sb_mw=1.0, split_depth=1,
             clip_iters=1):
    """One BaB iteration on a popped batch: bound, closure, optional
    alpha-CROWN, the clip (repeated while a box shrinks, at most
    ``clip_iters`` times), split (verify_graph.py:12855-13423).

    The split dimension is the widest, or with ``branch_sb`` (and a clip,
    which gives the input linearization A) the best SB score of the
    feasible leaves' A rows and spec bounds.  ``split_depth`` K > 1 (SB
    only) splits every leaf on its top K dimensions at once.

    Returns a dict with lb, closed, unclosed (indices), feasible (after
    clip, over unclosed), xl_split/xh_split, ax, n_degenerate, crown_lb /
    crown_closed (the bound and closure before alpha-CROWN), the
    children as ``chunks`` (the worklist pushes, in order) and, for
    bisection, low/high.
    """
    lb, A, acc = bound_batch(xl, xh, gg, spec_ew, crown_intermediate,
                             clip_enabled)
    closed = closure(lb, disj_q_idx)
    crown_lb, crown_closed = lb, closed
    lb, closed, n_al, n_ait = alpha_on_leaves(
        lb, xl, xh, gg, spec_ew, disj_q_idx, closed, alpha_iters, alpha_all,
        alpha_eps, alpha_max_leaves, alpha_lr, alpha_lr_decay)
    unclosed = (~closed).nonzero(as_tuple=True)[0]
    out = {'lb': lb, 'A': A, 'acc': acc, 'closed': closed,
           'unclosed': unclosed, 'n_alpha_leaves': n_al,
           'n_alpha_iters': n_ait, 'crown_lb': crown_lb,
           'crown_closed': crown_closed}
    A_s = None
    if clip_enabled and unclosed.numel() > 0 and A is not None:
        xl_u, xh_u = xl[unclosed], xh[unclosed]
        xl_c, xh_c, feas = clip_iterated(xl_u, xh_u, A[unclosed], acc[unclosed],
                                         disj_q_idx, clip_iters)
        fidx = feas.nonzero(as_tuple=True)[0]
        out['feasible'] = feas
        xl_s, xh_s = xl_c[fidx], xh_c[fidx]
        A_s, lb_s = A[unclosed][fidx], lb[unclosed][fidx]
    else:
        out['feasible'] = None
        xl_s, xh_s = xl[unclosed], xh[unclosed]
    out['xl_split'], out['xh_split'] = xl_s, xh_s
    if xl_s.shape[0] > 0:
        if branch_sb and A_s is not None:
            scores = sb_scores(xl_s, xh_s, A_s, lb_s, sb_margin, sb_thr, sb_mw)
            K = min(split_depth, xl_s.shape[1])
            dims = top_dims(scores, K)
        else:
            dims = widest_axis(xl_s, xh_s).unsqueeze(1)
        ax = dims[:, 0]
        if dims.shape[1] > 1:
            n_deg, kids = split_multi(xl_s, xh_s, dims)
            out.update(ax=ax, dims=dims, n_degenerate=n_deg, chunks=[kids], low=None,
                       high=None)
            return out
        n_deg, low, high = bisect(xl_s, xh_s, ax)
    else:
        ax = torch.zeros(0, dtype=torch.long)
        n_deg, low, high = 0, (xl_s, xh_s), (xl_s, xh_s)
    out.update(ax=ax, n_degenerate=n_deg, low=low, high=high,
               chunks=[low, high] if low[0].shape[0] > 0 else [])
    return out


def input_split_batched(xl0, xh0, gg, spec_ew, disj_q_idx, batch_size=4096,
                        max_worklist=200_000, total_timeout=60.0,
                        max_iters=None, **step_kw):
    """Worklist-driven input-split BaB (verify_graph.py:12834-13464) with an
    optional cap on iterations.  A ``split_depth`` K > 1 applies only to a
    popped batch smaller than batch_size (verify_graph.py:13343-13344).
    Returns (verdict, details, trace) where trace lists per-iteration dicts
    (B, n_closed, n_children)."""
    t0 = time.perf_counter()
    wl = ChunkWorklist(xl0, xh0)
    n_leaves = n_iters = n_open = 0
    trace = []
    while wl:
        if max_iters is not None and n_iters >= max_iters:
            break
        wl_n = wl.size()
        if time.perf_counter() - t0 > total_timeout - 0.5:
            n_open = wl_n
            break
        B = min(batch_size, wl_n)
        xl, xh = wl.pop(B)
        kw = dict(step_kw)
        if B >= batch_size:
            kw['split_depth'] = 1
        st = bab_step(xl, xh, gg, spec_ew, disj_q_idx, **kw)
        n_leaves += B
        n_open += st['n_degenerate']
        for c in st['chunks']:
            wl.push(*c)
        trace.append({'B': B, 'n_closed': int(st['closed'].sum()),
                      'n_children': sum(int(c[0].shape[0]) for c in st['chunks'])})
        n_iters += 1
        if wl.size() > max_worklist:
            return 'unknown', {'phase': 'batched_worklist_overflow',
                               'batched_n_leaves': n_leaves,
                               'batched_n_iters': n_iters,
                               'worklist_size': wl.size()}, trace
    if not wl and n_open == 0:
        return 'verified', {'phase': 'batched_verified',
                            'batched_n_leaves': n_leaves,
                            'batched_n_iters': n_iters}, trace
    return 'unknown', {'phase': 'batched_timeout',
                       'batched_n_leaves': n_leaves,
                       'batched_n_iters': n_iters,
                       'batched_worklist_left': wl.size(),
                       'batched_open_degenerate': n_open}, trace
