"""Input-split branch-and-bound on the GPU, with the reference's function
names and signatures (verify_graph.py of the reference).

``_input_split_batched`` runs the reference's worklist loop
(verify_graph.py:12466-13464) for the bound engine's settings: CROWN or
zonotope intermediate bounds, domain clipping, batched alpha-CROWN on
unclosed leaves, widest-dimension bisection.  Closure, clipping,
compaction, branching and bisection run as HIP kernels; the worklist is a
LIFO list of device-resident 2-D chunks.  SB branching and 2^K-way splits
are supported; root/leaf PGD and LP/MILP escalation are not part of this
engine.
"""
import ctypes
import os
import time

import torch

from ._lib import call, f32, host_array, ptr, stream
from . import _lib
from .spec import dedup_queries
from .verify_zono_bnb import (_bound_crown_spec,
                              _forward_zonotope_graph_batched,
                              _run_alpha_crown_inputsplit_batched,
                              _spec_backward_graph_batched, _widths, _zono_sb)

__all__ = ['_clip_box_by_halfspaces_batched', '_input_split_batched',
           'DisjunctTable', 'bab_step', 'ChunkWorklist']


class DisjunctTable:
    """Device CSR of disjunct -> query positions (verify_graph.py:12658-12682)."""

    MAX_GROUP = 64  # per-disjunct query limit of the clip kernel

    def __init__(self, disj_q_idx, device):
        self.groups = [list(v) for v in disj_q_idx.values()]
        if any(len(g) > self.MAX_GROUP for g in self.groups):
            raise NotImplementedError(
                f'vibecheck_amd: a disjunct has more than {self.MAX_GROUP} queries')
        ptrs = [0]
        flat = []
        for g in self.groups:
            flat.extend(g)
            ptrs.append(len(flat))
        self.d_ptr = torch.tensor(ptrs, dtype=torch.int32, device=device)
        self.q_idx = torch.tensor(flat if flat else [0], dtype=torch.int32,
                                  device=device)
        self.n = len(self.groups)


def _compact_device(flags, select_zero=False, cnt=None):
    """Ascending positions of the set (or clear) flags and their count, both
    left on the device: idx (max(n, 1),) int64 valid up to cnt, cnt (1,)
    (or the given one-element int64 slot)."""
    n = flags.numel()
    dev = flags.device
    lib = _lib.load()
    ws_bytes = int(lib.vc_compact_workspace(n))
    ws = torch.empty(max(ws_bytes, 8), dtype=torch.uint8, device=dev)
    idx = torch.empty(max(n, 1), dtype=torch.int64, device=dev)
    if cnt is None:
        cnt = torch.empty(1, dtype=torch.int64, device=dev)
    call('vc_compact', ptr(flags), n, 1 if select_zero else 0, ptr(idx),
         ptr(cnt), ptr(ws), ws_bytes, stream())
    return idx, cnt


def _compact(flags, select_zero=False):
    """Ascending positions of the set (or, with select_zero, clear) flags."""
    idx, cnt = _compact_device(flags, select_zero)
    return idx[:int(cnt.item())]


def _gather(t, idx):
    """Rows t[idx] (any trailing shape), by the HIP row gather."""
    n = idx.numel()
    cols = 1
    for s in t.shape[1:]:
        cols *= s
    out = torch.empty((n,) + tuple(t.shape[1:]), dtype=t.dtype, device=t.device)
    if n > 0:
        call('vc_gather_rows', ptr(f32(t)), ptr(idx), n, cols, ptr(out),
             stream())
    return out


def _gather_many(ts, idx):
    """[t[idx] for t in ts] (fp32 tensors with the same rows), in one
    launch."""
    ins = [f32(t) for t in ts]
    outs = [torch.empty((idx.numel(),) + tuple(t.shape[1:]), device=t.device) for t in ins]
    if idx.numel() > 0:
        keep = [host_array(ctypes.c_void_p, [ptr(t) for t in ins]),
                host_array(ctypes.c_void_p, [ptr(t) for t in outs]),
                host_array(ctypes.c_int32, [t[0].numel() for t in ins])]
        call('vc_gather_rows_multi', keep[0][1], keep[1][1], keep[2][1], len(ins), ptr(idx),
             idx.numel(), stream())
    return outs


def _gather_layers(sb, idx):
    """{L: (lo[idx], hi[idx])} for every layer, in one launch."""
    Ls = sorted(sb)
    outs = _gather_many([t for L in Ls for t in sb[L]], idx)
    return {L: (outs[2 * k], outs[2 * k + 1]) for k, L in enumerate(Ls)}


def _closure(lb, table):
    B, Q = lb.shape
    closed = torch.empty(B, dtype=torch.bool, device=lb.device)
    if B > 0:
        call('vc_closure', ptr(lb.contiguous()), B, Q, ptr(table.d_ptr),
             ptr(table.q_idx), table.n, ptr(closed), stream())
    return closed


def _clip(xl, xh, A, b, table):
    B, Q, n = A.shape
    xl_o = torch.empty_like(xl)
    xh_o = torch.empty_like(xh)
    feas = torch.empty(B, dtype=torch.bool, device=xl.device)
    if B > 0:
        call('vc_clip_box', ptr(xl), ptr(xh), ptr(A.contiguous()),
             ptr(b.contiguous()), B, Q, n, ptr(table.d_ptr), ptr(table.q_idx),
             table.n, ptr(xl_o), ptr(xh_o), ptr(feas), stream())
    return xl_o, xh_o, feas


def _clip_iterated(xl, xh, A, b, table, clip_iters):
    """Clip until no box shrinks, at most clip_iters times, with the same
    halfspaces (verify_graph.py:13036-13081): the stop test is over the
    whole batch (one host read per iteration, as the reference's
    ``.any().item()``); feasibility is the last iteration's."""
    xl_c, xh_c = xl, xh
    feas = None
    flag = torch.empty(1, dtype=torch.int32, device=xl.device) if clip_iters > 1 else None
    for it in range(max(1, int(clip_iters))):
        xl_n, xh_n, feas = _clip(xl_c, xh_c, A, b, table)
        if it + 1 >= clip_iters:
            xl_c, xh_c = xl_n, xh_n
            break
        call('vc_box_shrunk', ptr(xl_c), ptr(xh_c), ptr(xl_n), ptr(xh_n), xl_c.numel(),
             ptr(flag), stream())
        xl_c, xh_c = xl_n, xh_n
        if int(flag.item()) == 0:
            break
    return xl_c, xh_c, feas


def _clip_box_by_halfspaces_batched(xl, xh, A, b):
    """Bounding box of {x in [xl, xh] : A_q.x + b_q <= 0 for all q}
    (verify_graph.py:12363-12426).  Returns (xl', xh', feasible)."""
    xl, xh, A, b = f32(xl), f32(xh), f32(A), f32(b)
    Q = A.shape[1]
    table = DisjunctTable({0: list(range(Q))}, xl.device)
    return _clip(xl, xh, A, b, table)


def _split_feasible(xl, xh, feas, branch=None, K=1):
    """The feasible rows (feas) of clipped boxes, their split dimensions and
    children, with one host read for the counts: the split dimension is
    taken on every row, so the feasible and the split lists are compacted
    together (verify_graph.py:13115-13121, 13244-13423).

    ``branch`` None: widest axis; else (A, lb, mode, thr, mw) for the SB
    score (mode 1 sum, 2 margin) over the rows' A (B, Q, n) and lb (B, Q).
    K > 1 (SB only): the 2^K-way split on each row's top K dimensions.
    Returns (xl_f, xh_f, n_degenerate, ax_f, chunks), chunks being the
    worklist pushes in order: [low, high] for a bisection, [children]."""
    B, n = xl.shape
    dev = xl.device
    K = max(1, min(int(K), n)) if branch is not None else 1
    dims = torch.empty(B, K, dtype=torch.int64, device=dev)
    usable = torch.empty(B, dtype=torch.bool, device=dev)
    if branch is None:
        call('vc_widest_axis', ptr(xl), ptr(xh), B, n, ptr(dims), ptr(usable), stream())
    else:
        A, lb, mode, thr, mw = branch
        call('vc_branch_topk', ptr(xl), ptr(xh), ptr(A), ptr(lb), B, A.shape[1], n, mode,
             float(thr), float(mw), K, ptr(dims), ptr(usable), stream())
    if K > 1:
        cnt = torch.empty(1, dtype=torch.int64, device=dev)
        fidx, _ = _compact_device(feas, cnt=cnt)
        nf = int(cnt.item())
        fidx = fidx[:nf]
        # the int64 dimensions travel as float pairs through the row gather
        xl_f, xh_f, d2 = _gather_many([xl, xh, dims.view(torch.float32).view(B, 2 * K)], fidx)
        dims_f = d2.contiguous().view(torch.int64).view(nf, K)
        plan = torch.empty(nf + 2, dtype=torch.int64, device=dev)
        call('vc_split_multi_plan', ptr(xl_f), ptr(xh_f), ptr(dims_f), nf, n, K, ptr(plan),
             ptr(plan[nf + 1:]), stream())
        total, n_deg = plan[nf:].tolist()
        kl = torch.empty(total, n, device=dev)
        kh = torch.empty(total, n, device=dev)
        call('vc_split_multi', ptr(xl_f), ptr(xh_f), ptr(dims_f), ptr(plan), nf, n, K, ptr(kl),
             ptr(kh), stream())
        return xl_f, xh_f, n_deg, dims_f[:, 0], ([(kl, kh)] if total > 0 else [])
    ax = dims.view(B)
    split = feas & usable
    cnts = torch.empty(2, dtype=torch.int64, device=dev)
    fidx, _ = _compact_device(feas, cnt=cnts[0:1])
    uidx, _ = _compact_device(split, cnt=cnts[1:2])
    nf, nu = cnts.tolist()
    fidx, uidx = fidx[:nf], uidx[:nu]
    # the int64 axes travel as float pairs through the row gather (bit copy)
    xl_f, xh_f, ax2 = _gather_many([xl, xh, ax.view(torch.float32).view(B, 2)], fidx)
    ax_f = ax2.view(torch.int64).view(nf)
    low_xl = torch.empty(nu, n, device=dev)
    low_xh = torch.empty_like(low_xl)
    high_xl = torch.empty_like(low_xl)
    high_xh = torch.empty_like(low_xl)
    if nu > 0:
        call('vc_bisect', ptr(xl), ptr(xh), ptr(ax), ptr(uidx), nu, n,
             ptr(low_xl), ptr(low_xh), ptr(high_xl), ptr(high_xh), stream())
    chunks = [(low_xl, low_xh), (high_xl, high_xh)] if nu > 0 else []
    return xl_f, xh_f, nf - nu, ax_f, chunks


def _widest_and_bisect(xl, xh):
    """Widest-axis split of every leaf: returns (n_degenerate, ax, low, high)
    (verify_graph.py:13291, 13366-13382)."""
    B, n = xl.shape
    dev = xl.device
    ax = torch.empty(B, dtype=torch.int64, device=dev)
    usable = torch.empty(B, dtype=torch.bool, device=dev)
    if B == 0:
        e = xl[:0]
        return 0, ax, (e, e), (e, e)
    call('vc_widest_axis', ptr(xl), ptr(xh), B, n, ptr(ax), ptr(usable),
         stream())
    u = _compact(usable)
    nu = u.numel()
    low_xl = torch.empty(nu, n, device=dev)
    low_xh = torch.empty_like(low_xl)
    high_xl = torch.empty_like(low_xl)
    high_xh = torch.empty_like(low_xl)
    if nu > 0:
        call('vc_bisect', ptr(xl), ptr(xh), ptr(ax), ptr(u), nu, n,
             ptr(low_xl), ptr(low_xh), ptr(high_xl), ptr(high_xh), stream())
    return B - nu, ax, (low_xl, low_xh), (high_xl, high_xh)


def _join_rows(parts):
    """torch.cat of 2-D row chunks, or a view when they lie back to back in
    one storage (the native round leaves a round's high and low children so,
    in the order they are popped)."""
    a = parts[0]
    if all(t.is_contiguous() for t in parts) and all(
            t.dtype == a.dtype and t.shape[1:] == a.shape[1:] for t in parts):
        base = a.untyped_storage().data_ptr()
        end = a.storage_offset() + a.numel()
        for t in parts[1:]:
            if t.untyped_storage().data_ptr() != base or t.storage_offset() != end:
                break
            end += t.numel()
        else:
            rows = sum(int(t.shape[0]) for t in parts)
            return torch.as_strided(a, (rows,) + tuple(a.shape[1:]), a.stride(),
                                    a.storage_offset())
    return torch.cat(parts, 0)


class ChunkWorklist:
    """LIFO worklist of device-resident 2-D chunks
    (verify_graph.py:12695-12726)."""

    def __init__(self, xl0, xh0):
        self.xl = [xl0.reshape(1, -1)]
        self.xh = [xh0.reshape(1, -1)]

    def size(self):
        return sum(int(c.shape[0]) for c in self.xl)

    def push(self, xl, xh):
        self.xl.append(xl)
        self.xh.append(xh)

    def pop(self, n):
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
            return pl[0].contiguous(), ph[0].contiguous()
        return _join_rows(pl), _join_rows(ph)

    def __bool__(self):
        return bool(self.xl)


# Run bab_step's round as one native call (vc_mlp_bab_round) where it
# applies; switching this off runs the same entry points from Python.
NATIVE_ROUND = True

# How the driver's native rounds hand the next batch's bound phase over
# (bab_step's ``lookahead``): 'tail' runs it at the end of each round's call
# on the same stream, so the GPU has work while the host returns from one
# call and makes the next; 'overlap' runs it while alpha runs on a second
# stream (on the ACAS-Xu rounds measured no faster than the rounds in
# order: alpha and the children's bound phase compete for the same compute
# units, each workgroup of either holding the net's weights in LDS); False:
# each round bounds its own batch.
LOOKAHEAD = 'tail'
# The most children a lookahead bounds (beyond that the round runs in order).
LOOKAHEAD_MAX_CHILDREN = 16384

_AUX_STREAMS = {}


def _aux_stream(dev):
    """A second stream of the device, at the default priority (the
    lookahead's alpha runs there)."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    s = _AUX_STREAMS.get(idx)
    if s is None:
        s = _AUX_STREAMS[idx] = torch.cuda.Stream(device=idx)
    return s.cuda_stream


class PhaseTimer:
    """The driver's per-phase profile (verify_graph.py:12814-12833,
    13430-13450): bound (alpha-CROWN included, as in the reference), clip
    and split time per BaB iteration, the closures by the bound (CROWN and
    alpha) and by the clip, and the clip's mean after/before ratio of the
    summed box widths.  Times come from HIP events recorded on the launch
    stream at the phase boundaries (five per round; the native round
    records them itself), read once by ``report``: no synchronisation per
    phase, so the profiled run keeps the native round and its timing.
    alpha's own share of the bound time is reported beside it."""

    def __init__(self, device, widths=True):
        self.device = torch.device(device)
        self.widths = widths    # the clip's width sums (one small device buffer per round)
        self.t0 = time.perf_counter()
        self.rounds = []        # (5 events, widths tensor or None)
        self.crown_closed = 0
        self.clip_closed = 0

    def begin(self, clip):
        """Events and clip-width accumulator of one round."""
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
        for e in ev:
            e.record()      # creates the HIP event; the round records it again
        w = torch.zeros(2, dtype=torch.float64, device=self.device) if clip else None
        self.rounds.append((ev, w))
        return ev, w

    def closures(self, B, n_unclosed, n_feasible):
        self.crown_closed += B - n_unclosed
        if n_feasible is not None:
            self.clip_closed += n_unclosed - n_feasible

    def totals(self):
        """{'bound', 'alpha', 'clip', 'split'} seconds, and the shrink
        ratio's sum and count (synchronises once)."""
        torch.cuda.synchronize(self.device)
        t = {'bound': 0.0, 'alpha': 0.0, 'clip': 0.0, 'split': 0.0,
             'clip_shrink_sum': 0.0, 'clip_shrink_n': 0}
        for ev, w in self.rounds:
            try:
                d = [ev[k].elapsed_time(ev[k + 1]) * 1e-3 for k in range(4)]
            except RuntimeError:
                continue        # a round that ended in an error
            t['bound'] += d[0] + d[1]
            t['alpha'] += d[1]
            t['clip'] += d[2]
            t['split'] += d[3]
            if w is not None:
                wb, wa = (float(v) for v in w.cpu())
                if wb > 0.0 or wa > 0.0:
                    t['clip_shrink_sum'] += wa / max(wb, 1e-12)
                    t['clip_shrink_n'] += 1
        return t

    def report(self, n_iters, n_leaves):
        """Prints the reference's two profile lines (verify_graph.py:
        13436-13450) and returns the totals."""
        t = self.totals()
        tot = max(time.perf_counter() - self.t0, 1e-12)
        acct = t['bound'] + t['clip'] + t['split']
        shrink = (t['clip_shrink_sum'] / t['clip_shrink_n'] if t['clip_shrink_n']
                  else float('nan'))
        print(f"[vc-phase] BAB total={tot:.2f}s | "
              f"bound={t['bound']:.2f}s ({100 * t['bound'] / tot:.0f}%) "
              f"clip={t['clip']:.2f}s ({100 * t['clip'] / tot:.0f}%) "
              f"split={t['split']:.2f}s ({100 * t['split'] / tot:.0f}%) "
              f"other={tot - acct:.2f}s ({100 * (tot - acct) / tot:.0f}%) | "
              f"iters={n_iters} leaves={n_leaves} | alpha={t['alpha']:.3f}s of bound",
              flush=True)
        print(f"[vc-phase] closures: crown={self.crown_closed} clip={self.clip_closed} | "
              f"clip avg post/pre box-width ratio={shrink:.4f} (1.0=no shrink) over "
              f"{t['clip_shrink_n']} clip-iters", flush=True)
        t.update(total=tot, crown_closed=self.crown_closed, clip_closed=self.clip_closed)
        return t


def _tag_phase(e, phase):
    """Marks an error raised after the bound phase, which the driver does not
    take for an OOM of the batch (the reference's try covers the bound
    phase only, verify_graph.py:12853-12897)."""
    if not hasattr(e, 'vc_phase'):
        try:
            e.vc_phase = phase
        except AttributeError:
            pass
    return e


def _bab_round_native(xl, xh, gg, spec_ew, table, alpha_iters, alpha_lr, alpha_lr_decay,
                      phase_timer=None, lookahead=False, pre=None, la_max=None):
    """bab_step's round (crown intermediate bounds, clip, alpha-CROWN on
    every open leaf) as one call of the native round orchestration, for
    nets with the shape-specialised kernels; None where it does not apply.
    Same entry points in the same order as the Python round, so the same
    results.  ``lookahead`` 'overlap' (or True): while alpha runs on a
    second stream, clip and split the leaves the CROWN bound leaves open and
    run the bound phase on all their children; 'tail': run the bound phase
    on the children after the split.  Either way the result's 'lookahead'
    then holds the bound phase of the round's children (high then low) for
    the next round's ``pre``, when there are at most ``la_max`` of them."""
    from . import mlp_fused
    from . import verify_zono_bnb as vz
    dev = xl.device
    plan = mlp_fused.plan_for(gg, dev) if vz.FUSED_MLP else None
    if plan is None or not mlp_fused._tiled(plan):
        return None
    if 1 + sum(plan.dims[:plan.n]) > _lib.VC_ZONO_WIDE_COLS or len(spec_ew) > 32:
        return None
    Wq, bq = vz._spec_rows(spec_ew, dev)
    Q = Wq.shape[0]
    if alpha_iters > 0 and not mlp_fused.alpha_supported(plan, Q):
        return None
    S, acc0 = mlp_fused.fold_spec(plan, Wq, bq)
    xl, xh = f32(xl), f32(xh)
    B, n_in = xl.shape
    # Between two rounds the GPU waits on this host code (each round ends
    # with the children's count read back), so the outputs are one
    # allocation addressed by offsets, and their views are made after the
    # call: floats (lb, acc, A, the feasible rows' xl and xh, the children's
    # xl and xh with 2 Bm rows each: high then low, so that the next batch
    # in pop order is one block), then int64 indices [2, Bm], then flags
    # [2, Bm], each 256-byte aligned.
    Bm = max(B, 1)
    nflt = Bm * (2 * Q + Q * n_in + 6 * n_in)
    o_idx = (4 * nflt + 255) & ~255
    o_flg = (o_idx + 16 * Bm + 255) & ~255
    buf = torch.empty(o_flg + 2 * Bm, dtype=torch.uint8, device=dev)
    p = buf.data_ptr()
    p_box = p + 4 * Bm * (2 * Q + Q * n_in)
    nb = 4 * Bm * n_in
    lib = _lib.load()
    nws = int(lib.vc_mlp_bab_round_workspace(plan.dims_p, plan.n, B, Q))
    ws = torch.empty(max(nws, 8), dtype=torch.uint8, device=dev)
    counts = (ctypes.c_int64 * 7)()
    if pre is not None and (pre.get('n') != B or pre.get('plan') is not plan
                            or pre.get('spec') is not spec_ew):
        pre = None
    # with a handed-over bound phase, the round reads and updates its spec
    # bound, A and acc where the previous call left them (no copies)
    p_lb, p_A, p_acc = p, p + 8 * Bm * Q, p + 4 * Bm * Q
    if pre is not None:
        hoff = (ctypes.c_int64 * 3)()
        call('vc_mlp_bab_round_handoff_offsets', plan.dims_p, plan.n, B, Q,
             ctypes.addressof(hoff))
        hp = pre['buf'].data_ptr()
        p_lb, p_A, p_acc = hp + hoff[0], hp + hoff[1], hp + hoff[2]
    la = aux = None
    la_bytes = la_cap = 0
    mode = 'overlap' if lookahead is True else lookahead
    if (mode in ('overlap', 'tail') and phase_timer is None and B > 0
            and (mode == 'tail' or alpha_iters > 0)):
        la_cap = min(2 * B, LOOKAHEAD_MAX_CHILDREN if la_max is None else int(la_max))
        la_bytes = int(lib.vc_mlp_bab_round_lookahead_workspace(plan.dims_p, plan.n, B, Q,
                                                                 la_cap))
        la = torch.empty(max(la_bytes, 8), dtype=torch.uint8, device=dev)
        aux = _aux_stream(dev) if mode == 'overlap' else None
    # work accounting and timing of the CROWN launch, as mlp_fused.crown does
    # (a handed-over bound phase ran inside the previous round's call)
    seeds = seed_row = ev = zev = None
    if pre is None:
        if mlp_fused.SEED_COUNTER is not None:
            seed_row = mlp_fused.SEED_ROW
            seeds = mlp_fused.SEED_COUNTER[seed_row]
            mlp_fused.SEED_ROW += 1
        ev = _lib.timing_events('vc_mlp_tiled_crown', B)
        # the zonotope passes' span: from an event recorded before the call
        # to the CROWN pass's start, which the round records right after them
        zev = _lib.timing_events('zonotope_pass', B) if ev else None
        if zev:
            zev[0].record()
    pev_arr = pev_p = widths = None
    if phase_timer is not None:
        pev, widths = phase_timer.begin(clip=phase_timer.widths)
        pev_arr, pev_p = host_array(ctypes.c_void_p, [e.cuda_event for e in pev])
    fail = ctypes.c_int32(-1)
    try:
        call('vc_mlp_bab_round', plan.dims_p, plan.n, plan.tfrag.data_ptr(),
             plan.bias_cat.data_ptr(), Q, S.data_ptr(), acc0.data_ptr(), ptr(table.d_ptr),
             ptr(table.q_idx), table.n, B, ptr(xl), ptr(xh), int(alpha_iters),
             float(alpha_lr), float(alpha_lr_decay), 1e-6, p_lb, p_A, p_acc,
             p + o_flg, p + o_idx, p + o_flg + Bm, p_box, p_box + nb, p + o_idx + 8 * Bm,
             None, None, p_box + 2 * nb, p_box + 4 * nb, ptr(seeds),
             ev[0].cuda_event if ev else None, ev[1].cuda_event if ev else None, pev_p,
             ptr(widths), ws.data_ptr(), nws,
             pre['buf'].data_ptr() if pre is not None else None,
             la.data_ptr() if la is not None else None, la_bytes, la_cap,
             aux, mlp_fused._stop_word().data_ptr(),
             mlp_fused._pinned_words().data_ptr(), ctypes.addressof(counts),
             ctypes.addressof(fail), stream())
    except RuntimeError as e:
        if phase_timer is not None:
            phase_timer.rounds.pop()
        if fail.value == 1:
            # alpha failed: the Python round redoes the step and keeps the
            # CROWN bound there (verify_graph.py:12962-12969)
            return None
        if fail.value >= 2:
            raise _tag_phase(e, 'clip' if fail.value == 2 else 'split')
        raise
    del pev_arr
    if ev:
        spec = _lib.mlp_crown_flops(plan.dims, plan.n, B, [0] * plan.n, 0, Q)
        _lib.timing_add('vc_mlp_tiled_crown', ev, spec, (None, None, None, None, B, seed_row))
        if zev:
            _lib.timing_add('zonotope_pass', (zev[0], ev[0]), 0.0, (B,), pool=zev)
    n_open, n_eval, n_unc, nf, nu, n_deg, n_next = (int(c) for c in counts)
    if phase_timer is not None:
        phase_timer.closures(B, n_unc, nf)
    # the views by absolute storage offsets (in elements of each dtype)
    fl = buf[:4 * nflt].view(torch.float32)
    i64 = buf[o_idx:o_idx + 16 * Bm].view(torch.int64)
    bl = buf[o_flg:].view(torch.bool)
    ast = torch.as_strided
    bo, nb, oi, r = Bm * (2 * Q + Q * n_in), Bm * n_in, o_idx // 8, (n_in, 1)
    if pre is None:
        lb_v = ast(fl, (B, Q), (Q, 1), 0)
        A_v = ast(fl, (B, Q, n_in), (Q * n_in, n_in, 1), 2 * Bm * Q)
        acc_v = ast(fl, (B, Q), (Q, 1), Bm * Q)
    else:
        hf = pre['buf'].view(torch.float32)
        lb_v = ast(hf, (B, Q), (Q, 1), hoff[0] // 4)
        A_v = ast(hf, (B, Q, n_in), (Q * n_in, n_in, 1), hoff[1] // 4)
        acc_v = ast(hf, (B, Q), (Q, 1), hoff[2] // 4)
    out = {'lb': lb_v, 'A': A_v, 'acc': acc_v,
           'closed': ast(bl, (B,), (1,), o_flg), 'unclosed': ast(i64, (n_unc,), (1,), oi),
           'n_alpha_leaves': n_open, 'n_alpha_iters': n_eval,
           'feasible': ast(bl, (n_unc,), (1,), o_flg + Bm) if n_unc > 0 else None,
           'xl_split': ast(fl, (nf, n_in), r, bo), 'xh_split': ast(fl, (nf, n_in), r, bo + nb),
           'ax': ast(i64, (nf,), (1,), oi + Bm), 'n_degenerate': n_deg,
           'low': (ast(fl, (nu, n_in), r, bo + 2 * nb + nu * n_in),
                   ast(fl, (nu, n_in), r, bo + 4 * nb + nu * n_in)),
           'high': (ast(fl, (nu, n_in), r, bo + 2 * nb), ast(fl, (nu, n_in), r, bo + 4 * nb)),
           # the next batch in pop order (high, then low), without a copy
           'next': (ast(fl, (2 * nu, n_in), r, bo + 2 * nb),
                    ast(fl, (2 * nu, n_in), r, bo + 4 * nb))}
    out['chunks'] = [out['low'], out['high']] if nu > 0 else []
    out['lookahead'] = ({'buf': la, 'n': n_next, 'plan': plan, 'spec': spec_ew}
                        if la is not None and n_next >= 0 else None)
    return out


def _alpha_band(lb, closed, table, eps, max_leaves):
    """The alpha-CROWN leaves of the boundary band (verify_graph.py:
    12938-12950): unclosed leaves whose worst disjunct's best bound is above
    -eps, best first, at most max_leaves; ties in leaf order."""
    B, Q = lb.shape
    dev = lb.device
    keys = torch.empty(B, device=dev)
    cand = torch.empty(B, dtype=torch.bool, device=dev)
    call('vc_alpha_band_keys', ptr(lb), B, Q, ptr(table.d_ptr), ptr(table.q_idx), table.n,
         ptr(closed), float(-eps), ptr(keys), ptr(cand), stream())
    cidx = _compact(cand)
    C = int(cidx.numel())
    k = min(C, int(max_leaves))
    sel = torch.empty(k, dtype=torch.int64, device=dev)
    if k > 0:
        call('vc_rank_select_desc', ptr(keys), ptr(cidx), C, k, ptr(sel), stream())
    return sel


def bab_step(xl, xh, gg, spec_ew, table, crown_intermediate=True,
             clip_enabled=True, alpha_iters=0, alpha_all=False, alpha_eps=0.0,
             alpha_max_leaves=200, alpha_lr=0.25, alpha_lr_decay=0.98,
             timers=None, branch_sb=False, sb_margin=False, sb_thr=0.01, sb_mw=1.0,
             split_depth=1, clip_iters=1, phase_timer=None, lookahead=False, pre=None,
             la_max=None):
    """One BaB iteration on a popped batch (verify_graph.py:12855-13423):
    bound, closure, optional alpha-CROWN on unclosed leaves (opportunistic:
    a RuntimeError or OOM inside it keeps the bound it had, as at
    verify_graph.py:12962-12969), the clip (repeated while any box shrinks,
    at most ``clip_iters`` times), split.  The split dimension is the widest, or with
    ``branch_sb`` (and a clip, which gives the input linearization) the best
    SB score (sum form, or ``sb_margin``); ``split_depth`` K > 1 (SB only)
    splits each leaf on its top K dimensions into 2^K children.  Returns a
    dict of device tensors (same keys as the oracle's bab_step; ``chunks``
    are the worklist pushes in order).  ``phase_timer`` (a PhaseTimer)
    records the round's phase events.  An error after the bound phase
    carries ``vc_phase`` ('clip' or 'split').

    ``lookahead`` (extension, native round only): 'tail' -- after the
    split, the round also runs the bound phase of its children; 'overlap'
    (or True) -- while alpha runs, the round bounds every child of the
    leaves the CROWN bound leaves open.  The result's 'lookahead' (None
    when it did not run, or with more than ``la_max`` children) is the
    bound phase of the round's children in the order cat(high, low), which
    the next call takes as ``pre`` when its batch is exactly that.  Each
    box's bounds depend on that box alone, so the results are the same as
    without it."""
    _widths(gg, xl.shape[1])
    if (NATIVE_ROUND and timers is None and crown_intermediate and clip_enabled
            and (alpha_iters == 0 or alpha_all) and not branch_sb and clip_iters == 1):
        out = _bab_round_native(xl, xh, gg, spec_ew, table, alpha_iters, alpha_lr,
                                alpha_lr_decay, phase_timer, lookahead=lookahead, pre=pre,
                                la_max=la_max)
        if out is not None:
            return out
    pev = pw = None
    if phase_timer is not None:
        pev, pw = phase_timer.begin(clip=False)
        pev[0].record()
    dev = xl.device
    dt = torch.float32
    sync_t = (lambda: (torch.cuda.synchronize(), time.perf_counter())[1]) \
        if timers is not None else None
    if timers is not None:
        t0 = sync_t()
    A = acc = None
    sb = None
    if crown_intermediate:
        out = _bound_crown_spec(gg, xl, xh, spec_ew, dev, dt,
                                return_input_linear=clip_enabled, return_zono_sb=True)
        if clip_enabled:
            _, lb, A, acc, sb = out
        else:
            _, lb, sb = out
    else:
        sb = _zono_sb(gg, xl, xh, dev, dt)
        if clip_enabled:
            lb, A, acc = _spec_backward_graph_batched(sb, xl, xh, gg, spec_ew, dev,
                                                      dt, return_input_linear=True)
        else:
            lb = _spec_backward_graph_batched(sb, xl, xh, gg, spec_ew, dev, dt)
    lb = lb.contiguous()
    closed = _closure(lb, table)
    if pev is not None:
        pev[1].record()
    n_al = n_ait = 0
    if timers is not None:
        t1 = sync_t()
        timers['bound'] = timers.get('bound', 0.0) + t1 - t0
        t0 = t1
    if alpha_iters > 0 and (alpha_all or alpha_eps > 0):
        if alpha_all:
            open_idx = _compact(closed, select_zero=True)
        else:
            open_idx = _alpha_band(lb, closed, table, alpha_eps, alpha_max_leaves)
        if open_idx.numel() > 0:
            # alpha starts from the zonotope bounds of the same boxes, which
            # the bound phase has already computed: gather their rows
            sb_open = None if sb is None else _gather_layers(sb, open_idx)
            xl_o, xh_o = _gather_many([xl, xh], open_idx)
            try:
                new, n_ait = _run_alpha_crown_inputsplit_batched(
                    xl_o, xh_o, gg, spec_ew,
                    dev, dt, n_iters=alpha_iters, lr=alpha_lr,
                    lr_decay=alpha_lr_decay, sb=sb_open, return_trace=True,
                    lazy_trace=True)
            except RuntimeError:
                # torch.cuda.OutOfMemoryError and NotImplementedError are
                # RuntimeErrors: alpha-CROWN only tightens, the step goes on
                # with the bound it has (verify_graph.py:12962-12969)
                new = None
                n_ait = 0
            n_al = int(open_idx.numel())
            if new is not None:
                call('vc_scatter_max_rows', ptr(lb), ptr(open_idx),
                     ptr(new.contiguous()), n_al, lb.shape[1], stream())
                closed = _closure(lb, table)
    if pev is not None:
        pev[2].record()
    if timers is not None:
        t1 = sync_t()
        timers['alpha'] = timers.get('alpha', 0.0) + t1 - t0
        t0 = t1
    try:
        return _round_tail(xl, xh, lb, A, acc, closed, n_al, n_ait, table, clip_enabled,
                           clip_iters, branch_sb, sb_margin, sb_thr, sb_mw, split_depth,
                           timers, sync_t, t0 if timers is not None else None, pev,
                           phase_timer)
    except RuntimeError as e:
        raise _tag_phase(e, 'clip')


def _round_tail(xl, xh, lb, A, acc, closed, n_al, n_ait, table, clip_enabled, clip_iters,
                branch_sb, sb_margin, sb_thr, sb_mw, split_depth, timers, sync_t, t0, pev,
                phase_timer):
    """bab_step after the bound and alpha phases: the unclosed leaves, the
    clip and the split."""
    unclosed = _compact(closed, select_zero=True)
    # the alpha loop's evaluation count was copied to the host in stream
    # order: the compaction's read above has waited for it
    n_ait = n_ait() if callable(n_ait) else n_ait
    out = {'lb': lb, 'A': A, 'acc': acc, 'closed': closed,
           'unclosed': unclosed, 'n_alpha_leaves': n_al,
           'n_alpha_iters': n_ait}
    if clip_enabled and unclosed.numel() > 0 and A is not None:
        xl_u, xh_u, A_u, acc_u, lb_u = _gather_many([xl, xh, A, acc, lb], unclosed)
        xl_c, xh_c, feas = _clip_iterated(xl_u, xh_u, A_u, acc_u, table, clip_iters)
        if pev is not None:
            pev[3].record()
        out['feasible'] = feas
        branch = ((A_u, lb_u, 2 if sb_margin else 1, sb_thr, sb_mw) if branch_sb
                  else None)
        xl_s, xh_s, n_deg, ax, chunks = _split_feasible(xl_c, xh_c, feas, branch,
                                                        split_depth)
        if timers is not None:
            timers['clip'] = timers.get('clip', 0.0) + sync_t() - t0
            t0 = sync_t()
    else:
        out['feasible'] = None
        xl_s, xh_s = _gather_many([xl, xh], unclosed)
        if pev is not None:
            pev[3].record()
        if timers is not None:
            t1 = sync_t()
            timers['clip'] = timers.get('clip', 0.0) + t1 - t0
            t0 = t1
        n_deg, ax, low, high = _widest_and_bisect(xl_s, xh_s)
        chunks = [low, high] if low[0].shape[0] > 0 else []
    out['xl_split'], out['xh_split'] = xl_s, xh_s
    if len(chunks) == 2:
        low, high = chunks
    elif chunks:             # the 2^K-way split: one chunk, no low/high halves
        low = high = None
    else:
        low = high = (xl_s[:0], xh_s[:0])
    out.update(ax=ax, n_degenerate=n_deg, chunks=chunks, low=low, high=high)
    if pev is not None:
        pev[4].record()
        phase_timer.closures(xl.shape[0], int(unclosed.numel()),
                             int(xl_s.shape[0]) if out['feasible'] is not None else None)
    if timers is not None:
        timers['split'] = timers.get('split', 0.0) + sync_t() - t0
    return out


def _setting(settings, name, default):
    if settings is None:
        return default
    if isinstance(settings, dict):
        return settings.get(name, default)
    return getattr(settings, name, default)


def _input_split_batched(graph, spec, settings, gg, device, dtype):
    """Worklist input-split BaB with batched leaf evaluation
    (verify_graph.py:12466-13464).

    Returns (verdict in {'verified', 'unknown'}, details).  Knobs read from
    ``settings`` (attribute or dict): total_timeout, input_split_batch_size,
    input_split_batched_max_worklist, input_split_batched_clip_enabled,
    input_split_crown_intermediate, input_split_batched_alpha_iters,
    input_split_batched_alpha_all_leaves, input_split_batched_alpha_boundary_eps,
    input_split_batched_alpha_max_leaves, input_split_batched_alpha_lr
    (extension; reference hard-codes 0.25), input_split_batched_max_iters
    (extension: stop after that many iterations), input_split_batched_branch_sb,
    input_split_sb_margin_score, input_split_sb_coeff_thresh,
    input_split_sb_margin_weight, bab_split_depth, input_split_batched_clip_iters,
    raise_on_oom.

    A RuntimeError in a step's bound phase (torch.cuda.OutOfMemoryError
    included) halves the batch size and pushes the popped batch back; at
    batch size 1 a real OOM is re-raised (unless raise_on_oom is off) and
    anything else ends the run 'unknown' / batched_oom
    (verify_graph.py:12872-12897).  Errors of the clip and split phases
    propagate, as the reference's try covers the bound phase only.

    With input_split_batched_phase_timing (or VC_PHASE_TIMING=1 in the
    environment) the run prints the reference's per-phase profile
    (verify_graph.py:12814-12833, 13436-13450) and returns it in the
    details under 'phase_timing'.
    """
    if dtype != torch.float32:
        raise NotImplementedError('vibecheck_amd computes in fp32 only')
    t_start = time.perf_counter()
    total_budget = float(_setting(settings, 'total_timeout', 60.0))
    batch_size = int(_setting(settings, 'input_split_batch_size', 4096))
    max_worklist = int(_setting(settings,
                                'input_split_batched_max_worklist', 200_000))
    clip_enabled = bool(_setting(settings,
                                 'input_split_batched_clip_enabled', True))
    crown_int = bool(_setting(settings, 'input_split_crown_intermediate',
                              False))
    alpha_iters = int(_setting(settings, 'input_split_batched_alpha_iters', 0))
    alpha_all = bool(_setting(settings,
                              'input_split_batched_alpha_all_leaves', False))
    alpha_eps = float(_setting(settings,
                               'input_split_batched_alpha_boundary_eps', 0.0))
    alpha_max_leaves = int(_setting(settings, 'input_split_batched_alpha_max_leaves', 200))
    alpha_lr = float(_setting(settings, 'input_split_batched_alpha_lr', 0.25))
    max_iters = _setting(settings, 'input_split_batched_max_iters', None)
    branch_sb = bool(_setting(settings, 'input_split_batched_branch_sb', False))
    sb_margin = bool(_setting(settings, 'input_split_sb_margin_score', False))
    sb_thr = float(_setting(settings, 'input_split_sb_coeff_thresh', 0.01))
    sb_mw = float(_setting(settings, 'input_split_sb_margin_weight', 1.0))
    split_depth = int(_setting(settings, 'bab_split_depth', 1))
    clip_iters = int(_setting(settings, 'input_split_batched_clip_iters', 1))
    dev = torch.device(device)

    xc = ((torch.as_tensor(spec.x_lo, dtype=dtype, device=dev)
           + torch.as_tensor(spec.x_hi, dtype=dtype, device=dev)) / 2
          ).reshape(1, -1)
    _, (c_probe, _) = _forward_zonotope_graph_batched(xc, xc, gg, dev, dtype)
    n_output = int(c_probe.shape[-1])
    queries = spec.as_linear_queries(n_output)
    if not queries:
        return 'verified', {'phase': 'batched_no_queries'}
    uniq, disj_q_idx = dedup_queries(queries)
    spec_ew = {pos: (torch.as_tensor(w, dtype=dtype, device=dev), b)
               for pos, (w, b) in enumerate(uniq)}
    table = DisjunctTable(disj_q_idx, dev)

    xl0 = torch.as_tensor(spec.x_lo, dtype=dtype, device=dev).flatten()
    xh0 = torch.as_tensor(spec.x_hi, dtype=dtype, device=dev).flatten()
    wl = ChunkWorklist(xl0, xh0)
    n_leaves = n_iters = n_open = 0
    pre = None
    pt = None
    if (bool(_setting(settings, 'input_split_batched_phase_timing', False))
            or os.environ.get('VC_PHASE_TIMING', '') == '1'):
        pt = PhaseTimer(dev)

    def done(verdict, details):
        if pt is not None:
            details['phase_timing'] = pt.report(n_iters, n_leaves)
        return verdict, details

    while wl:
        if max_iters is not None and n_iters >= int(max_iters):
            break
        wl_n = wl.size()
        if time.perf_counter() - t_start > total_budget - 0.5:
            n_open = wl_n
            break
        B = min(batch_size, wl_n)
        xl_b, xh_b = wl.pop(B)
        # a previous lookahead applies when this pop took exactly the two
        # chunks it pushed (high, then low); with the worklist now empty, the
        # next pop will be this round's children, so this round looks ahead
        use_pre = pre if (pre is not None and pre['n'] == B and not wl) else None
        pre = None
        try:
            # K > 1 only grows a queue that does not fill the batch
            # (verify_graph.py:13343-13344)
            st = bab_step(xl_b, xh_b, gg, spec_ew, table, crown_int,
                          clip_enabled, alpha_iters, alpha_all, alpha_eps,
                          alpha_max_leaves=alpha_max_leaves, alpha_lr=alpha_lr,
                          branch_sb=branch_sb, sb_margin=sb_margin,
                          sb_thr=sb_thr, sb_mw=sb_mw,
                          split_depth=split_depth if B < batch_size else 1,
                          clip_iters=clip_iters, phase_timer=pt,
                          lookahead=LOOKAHEAD if not wl else False, pre=use_pre,
                          la_max=min(batch_size, LOOKAHEAD_MAX_CHILDREN))
        except RuntimeError as e:
            # torch.cuda.OutOfMemoryError is a RuntimeError; only the bound
            # phase's errors halve the batch
            if getattr(e, 'vc_phase', 'bound') != 'bound':
                raise
            if torch.cuda.is_available():
                torch.cuda.empty_cache()
            new_bs = max(1, batch_size // 2)
            if new_bs == batch_size:
                if (isinstance(e, torch.cuda.OutOfMemoryError)
                        and bool(_setting(settings, 'raise_on_oom', True))):
                    raise
                return done('unknown', {'phase': 'batched_oom',
                                        'batch_size': batch_size})
            wl.push(xl_b, xh_b)
            batch_size = new_bs
            continue
        n_leaves += B
        n_open += st['n_degenerate']
        for c in st['chunks']:
            wl.push(*c)
        pre = st.get('lookahead')
        n_iters += 1
        if wl.size() > max_worklist:
            return done('unknown', {'phase': 'batched_worklist_overflow',
                                    'batched_n_leaves': n_leaves,
                                    'batched_n_iters': n_iters,
                                    'worklist_size': wl.size()})
    if not wl and n_open == 0:
        return done('verified', {'phase': 'batched_verified',
                                 'batched_n_leaves': n_leaves,
                                 'batched_n_iters': n_iters,
                                 'batched_batch_size': batch_size})
    return done('unknown', {'phase': 'batched_timeout',
                            'batched_n_leaves': n_leaves,
                            'batched_n_iters': n_iters,
                            'batched_worklist_left': wl.size(),
                            'batched_open_degenerate': n_open,
                            'batched_batch_size': batch_size})
