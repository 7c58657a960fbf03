"""Host side of the whole-network kernels for narrow fc/ReLU chains.

A network qualifies when its ops are fc, relu, fc, relu, ..., fc (every
relu fed by the preceding fc and carrying layer_idx 0, 1, ...), every width
is <= 64 and there are 1..16 ReLU layers -- the 5-50x6-5 ACAS-Xu shape.
For those nets the zonotope bounds, the CROWN intermediate bounds and the
spec backward run as one wavefront per domain (vc_mlp_* entry points);
other nets use the layer-wise kernels.
"""
import ctypes
import threading

import torch

from . import _lib
from ._lib import call, host_array, ptr, stream

MAX_W = 64
MAX_L = 16
PLAN_KEY = '_vc_amd_mlp_plan'

# Use the shape-specialised CROWN kernel (vc_mlp_tiled_crown) when the net
# has an instantiation; switching this off runs vc_mlp_crown.
TILED = True

# Batches above 4 x CUs run the layer-synchronous form (vc_mlp_crown_rows:
# rows of every domain packed into full tiles) instead of one wavefront per
# domain; both give the same results bit for bit.
ROWS = True

# The rows form builds the union of unstable neurons itself (in its seed-mask
# pass over the bounds); switching this off hands it the union lists of
# vc_unstable_union_layers + vc_union_compact instead (same results).
ROWS_OWN_UNION = True

# When set to a zeroed device int64 tensor (calls, MAX_L), the k-th call of
# the shape-specialised CROWN kernel adds its seeded neurons per layer to
# row k (work accounting; SEED_ROW is the next row).
SEED_COUNTER = None
SEED_ROW = 0


class MlpPlan:
    """Packed weights of a qualifying network on one device."""

    def __init__(self, gg, device):
        ops = gg['ops']
        fcs = [op for op in ops if op['type'] == 'fc']
        self.n = len(fcs) - 1
        Ws = [op['W'].detach().to(device=device, dtype=torch.float32).contiguous()
              for op in fcs]
        bs = []
        for op, W in zip(fcs, Ws):
            b = op.get('bias')
            bs.append(torch.zeros(W.shape[0], device=device) if b is None else
                      torch.as_tensor(b).detach().to(device=device, dtype=torch.float32)
                      .reshape(-1).contiguous())
        self.dims = [int(Ws[0].shape[1])] + [int(W.shape[0]) for W in Ws[:-1]]
        self.n_out = int(Ws[-1].shape[0])
        self.W_last, self.b_last = Ws[-1], bs[-1]
        self.Ws, self.bs = Ws[:-1], bs[:-1]
        self.bias_cat = torch.cat(self.bs).contiguous()
        self.device = device
        self._dims_arr, self.dims_p = host_array(ctypes.c_int32, self.dims)
        self._widths_arr, self.widths_p = host_array(ctypes.c_int32, self.dims[1:])
        wp_arr, wp = host_array(ctypes.c_void_p, [ptr(W) for W in self.Ws])
        lib = _lib.load()
        self.frag = {}
        for fwd in (0, 1):
            nf = int(lib.vc_mlp_frag_floats(self.dims_p, self.n, fwd))
            if nf <= 0:
                raise NotImplementedError('vibecheck_amd: network shape not fused')
            buf = torch.empty(nf, device=device)
            call('vc_mlp_pack', wp, self.dims_p, self.n, fwd, ptr(buf), stream())
            self.frag[fwd] = buf
        # fragments of the shape-specialised CROWN kernel (None: no instantiation)
        self.tfrag = None
        nt = int(lib.vc_mlp_tiled_floats(self.dims_p, self.n))
        if nt > 0:
            bp_arr, bp = host_array(ctypes.c_void_p, [ptr(b) for b in self.bs])
            self.tfrag = torch.empty(nt, device=device)
            call('vc_mlp_tiled_pack', wp, bp, self.dims_p, self.n, ptr(self.tfrag), stream())
            del bp_arr
        del wp_arr


def plan_for(gg, device):
    """The cached MlpPlan of gg on ``device``, or None if not eligible."""
    device = torch.device(device)
    cached = gg.get(PLAN_KEY)
    if cached is not None:
        if cached == 'no':
            return None
        if cached.device == device:
            return cached
    if not _eligible(gg):
        gg[PLAN_KEY] = 'no'
        return None
    plan = MlpPlan(gg, device)
    gg[PLAN_KEY] = plan
    return plan


def _eligible(gg):
    ops = gg['ops']
    if len(ops) < 3 or len(ops) % 2 == 0:
        return False
    # widths chained op by op (ValueError on a mismatch); the N-D MatMul
    # form of an fc is left to the layer-wise kernels
    from .verify_zono_bnb import _fc_form, validate_gg
    widths = validate_gg(gg)
    if any(op['type'] == 'fc' and _fc_form(op, widths[op['inputs'][0]])[0] > 1
           for op in ops):
        return False
    prev = gg['input_name']
    n_relu = 0
    for k, op in enumerate(ops):
        want = 'fc' if k % 2 == 0 else 'relu'
        if op['type'] != want or op['inputs'] != [prev]:
            return False
        if want == 'relu':
            if op.get('layer_idx') != n_relu:
                return False
            n_relu += 1
        else:
            W = op['W']
            if W.dim() != 2:
                return False
            if k < len(ops) - 1 and (W.shape[0] > MAX_W or W.shape[1] > MAX_W):
                return False
            if k == len(ops) - 1 and W.shape[1] > MAX_W:
                return False
        prev = op['name']
    return 1 <= n_relu <= MAX_L


def zono_bounds(plan, xl, xh, fallback):
    """Zonotope pre-activation bounds {L: (lo, hi)} for every ReLU layer.
    ``fallback(xl_sub, xh_sub)`` computes the layer-wise bounds for the
    domains whose generator matrix exceeds the register capacity."""
    B = xl.shape[0]
    dev = xl.device
    lo = [torch.empty(B, plan.dims[l + 1], device=dev) for l in range(plan.n)]
    hi = [torch.empty_like(t) for t in lo]
    # every relu but the last can append one generator per neuron
    max_cols = 1 + sum(plan.dims[:plan.n])
    lo_a, lo_p = host_array(ctypes.c_void_p, [ptr(t) for t in lo])
    hi_a, hi_p = host_array(ctypes.c_void_p, [ptr(t) for t in hi])
    from .verify_graph import _compact, _compact_device, _gather
    if _tiled(plan):
        # one wavefront per domain (128 generator columns), then the 4-wave
        # pass (512 columns) over the list of domains that did not fit,
        # compacted on the device
        ovf = torch.empty(B, dtype=torch.uint8, device=dev)
        args = (B, ptr(xl), ptr(xh), lo_p, hi_p, ptr(ovf))
        # the domain queue's counter, per call (the library resets it on the
        # stream), so calls from several host threads never share one
        queue = torch.empty(1, dtype=torch.int32, device=dev)
        call('vc_mlp_tiled_zono_bounds', plan.dims_p, plan.n, ptr(plan.tfrag),
             ptr(plan.bias_cat), *args, ptr(queue), stream())
        lst, cnt = _compact_device(ovf)
        call('vc_mlp_tiled_zono_wide', plan.dims_p, plan.n, ptr(plan.tfrag),
             ptr(plan.bias_cat), *args, ptr(lst), ptr(cnt), stream())
        if max_cols <= _lib.VC_ZONO_WIDE_COLS:
            # the wide pass holds every generator this net can have: no
            # domain is left over (and no host round trip to find out)
            del lo_a, hi_a
            return {L: (lo[L], hi[L]) for L in range(plan.n)}, 0
    else:
        ovf = torch.empty(B, dtype=torch.int32, device=dev)
        call('vc_mlp_zono_bounds', plan.dims_p, plan.n, ptr(plan.frag[1]),
             ptr(plan.bias_cat), B, ptr(xl), ptr(xh), lo_p, hi_p, ptr(ovf), stream())
        ovf = ovf.to(torch.uint8)
    del lo_a, hi_a
    bad = _compact(ovf)
    if bad.numel() > 0:
        sub = fallback(_gather(xl, bad), _gather(xh, bad))
        for L in range(plan.n):
            # the sources are held in locals until both launches are queued
            s_lo, s_hi = sub[L][0].contiguous(), sub[L][1].contiguous()
            call('vc_scatter_rows', ptr(s_lo), ptr(bad), bad.numel(), plan.dims[L + 1],
                 ptr(lo[L]), stream())
            call('vc_scatter_rows', ptr(s_hi), ptr(bad), bad.numel(), plan.dims[L + 1],
                 ptr(hi[L]), stream())
    return {L: (lo[L], hi[L]) for L in range(plan.n)}, int(bad.numel())


def union_idx(plan, sb):
    """Per layer, the neurons unstable in any domain (one host sync)."""
    dev = plan.device
    flags = torch.empty(sum(plan.dims[1:]), dtype=torch.uint8, device=dev)
    off = 0
    for L in range(plan.n):
        n = plan.dims[L + 1]
        lo, hi = sb[L]
        call('vc_unstable_union', ptr(lo), ptr(hi), lo.shape[0], n,
             ptr(flags[off:off + n]), stream())
        off += n
    f = flags.cpu()
    idx, cnt = [], []
    off = 0
    for L in range(plan.n):
        n = plan.dims[L + 1]
        sel = f[off:off + n].nonzero(as_tuple=True)[0].tolist()
        idx.extend(sel)
        cnt.append(len(sel))
        off += n
    idx_t = torch.tensor(idx if idx else [0], dtype=torch.int32).to(dev)
    return idx_t, cnt


def fold_spec(plan, Wq, bq):
    """Spec rows through the final fc: S = Wq W_last (Q, d_n), acc0 = bq +
    Wq b_last, by the backward fc kernel on the shared rows.  The last fold
    is kept on the plan (keyed on the rows' identity and in-place version);
    callers only read it."""
    key = (id(Wq), Wq._version, id(bq), bq._version)
    hit = getattr(plan, '_fold', None)
    if hit is not None and hit[0] == key:
        return hit[3], hit[4]
    Q = Wq.shape[0]
    S = torch.empty(Q, plan.dims[plan.n], device=plan.device)
    acc = bq.clone()
    call('vc_backward_fc', ptr(Wq), Q, Q, plan.n_out, None, None, None, 0, None,
         ptr(plan.W_last), ptr(plan.b_last), plan.dims[plan.n], ptr(S), ptr(acc),
         None, 0, stream())
    plan._fold = (key, Wq, bq, S, acc)
    return S, acc


ALPHA_MAX_L = 7
ALPHA_MAX_Q = 16


def _tiled(plan):
    return TILED and plan.tfrag is not None


def alpha_supported(plan, Q):
    if not 1 <= Q <= ALPHA_MAX_Q:
        return False
    return _tiled(plan) or plan.n <= ALPHA_MAX_L


# Pinned host words the library's kernels store into and the host polls:
# one set per host thread, so rounds and alpha loops run from different
# threads (on their own streams) never read each other's words.
_HOST_WORDS = threading.local()


def _stop_word():
    """Two pinned host int32 words the alpha loop's control kernel stores
    into (stopped; iterations taken), so that the host stops enqueueing
    iterations (one pair per host thread; each alpha loop ends with a host
    read, so it is free again)."""
    w = getattr(_HOST_WORDS, 'stop', None)
    if w is None:
        w = _HOST_WORDS.stop = torch.zeros(2, dtype=torch.int32, pin_memory=True)
    return w


def _pinned_words():
    """Pinned host int64 words the native BaB round's counts are stored in
    (one set per host thread; each round ends with them read)."""
    w = getattr(_HOST_WORDS, 'counts', None)
    if w is None:
        w = _HOST_WORDS.counts = torch.zeros(4, dtype=torch.int64, pin_memory=True)
    return w


def alpha_crown(plan, xl, xh, sb, Wq, bq, n_iters, lr, lr_decay, early_stop_eps, lazy=False):
    """Batched alpha-CROWN with the reference's schedule
    (verify_zono_bnb.py:5137-5288), one fused kernel launch per Adam
    iteration.  Returns (best (B, Q), evaluated iterations)."""
    B = xl.shape[0]
    dev = xl.device
    st = stream()
    S, acc0 = fold_spec(plan, Wq, bq)
    Q = S.shape[0]
    lo = [sb[L][0].contiguous() for L in range(plan.n)]
    hi = [sb[L][1].contiguous() for L in range(plan.n)]
    tiled = _tiled(plan)
    # one allocation for alpha and the Adam state of every layer: per layer
    # pointers into it (alpha block, then m, then v)
    sizes = [t.numel() for t in lo]
    tot = sum(sizes)
    flat = torch.empty(3 * tot, device=dev)
    offs = [0]
    for sz in sizes[:-1]:
        offs.append(offs[-1] + sz)
    base = flat.data_ptr()
    state = [[base + 4 * (k * tot + o) for o in offs] for k in range(3)]
    if not tiled:
        # the tiled kernel initialises alpha and the Adam state itself
        flat[tot:].zero_()
        for L in range(plan.n):
            call('vc_alpha_init', ptr(lo[L]), ptr(hi[L]), sizes[L], state[0][L], st)
    keep = []
    ptrs = []
    for lst in ([ptr(t) for t in lo], [ptr(t) for t in hi], *state):
        a, p = host_array(ctypes.c_void_p, lst)
        keep.append(a)
        ptrs.append(p)
    # per-iteration bounds: up to VC_ALPHA_CHUNK iterations per launch
    lb = torch.empty(_lib.VC_ALPHA_CHUNK if tiled else 1, B, Q, device=dev)
    best = torch.empty(B, Q, device=dev)
    red = torch.empty(2, device=dev)
    b1, b2, eps = 0.9, 0.999, 1e-8
    prev_max = -float('inf')
    cur_lr = float(lr)
    n_eval = 0
    if tiled:
        # the whole loop in one call, its control on the device: every
        # iteration is launched, the ones after the stop do nothing; one
        # host read at the end
        if n_iters < 1:
            raise ValueError('alpha_crown: n_iters must be >= 1')
        ctl = torch.empty(4, device=dev)
        stop = _stop_word()
        stop.zero_()
        call('vc_mlp_tiled_alpha_run', plan.dims_p, plan.n, ptr(plan.tfrag),
             ptr(plan.bias_cat), B, ptr(xl), ptr(xh), *ptrs, Q, ptr(S), ptr(acc0), ptr(lb),
             ptr(best), b1, b2, eps, cur_lr, float(lr_decay), int(n_iters),
             float(early_stop_eps), ptr(ctl), stop.data_ptr(), st)
        if lazy:
            # the count travels to pinned memory in stream order; reading it
            # after any later host synchronisation costs nothing
            host = torch.empty(1, dtype=torch.float32, pin_memory=True)
            host.copy_(ctl[2:3], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()

            def n_eval():
                ev.synchronize()
                return int(host[0])
            return best, n_eval
        return best, int(ctl[2].item())
    name, frag = 'vc_mlp_alpha_iter', plan.frag[0]
    for it in range(n_iters):
        step = it + 1
        call(name, plan.dims_p, plan.n, ptr(frag), ptr(plan.bias_cat),
             B, ptr(xl), ptr(xh), *ptrs, Q, ptr(S), ptr(acc0), ptr(lb), b1, b2, eps,
             cur_lr / (1 - b1 ** step), (1 - b2 ** step) ** 0.5, st)
        n_eval += 1
        call('vc_best_update', ptr(best), ptr(lb), B * Q, 1 if it == 0 else 0, ptr(red), st)
        curr_max, all_pos = red.tolist()
        if all_pos > 0.5:
            break
        if it > 0 and curr_max - prev_max < early_stop_eps:
            break
        prev_max = curr_max
        cur_lr *= lr_decay
    return best, n_eval


def crown(plan, xl, xh, sb, do_crown, spec=None, want_linear=False, per_domain=False):
    """CROWN intermediate bounds (do_crown) and/or the spec backward.

    ``per_domain``: seed, in each domain, only the union neurons whose
    slopes depend on their bounds there (see vc_mlp_tiled_crown): identical
    spec bound, A and acc; the returned bounds of the other neurons stay
    the starting ones.  Ignored without the shape-specialised kernel.
    Returns (tight {L: (lo, hi)} or None, lb (B, Q) or None, A, acc)."""
    B = xl.shape[0]
    dev = xl.device
    lo_in = [sb[L][0].contiguous() for L in range(plan.n)]
    hi_in = [sb[L][1].contiguous() for L in range(plan.n)]
    keep = []                       # host arrays alive until the call
    a, lin_p = host_array(ctypes.c_void_p, [ptr(t) for t in lo_in])
    keep.append(a)
    a, hin_p = host_array(ctypes.c_void_p, [ptr(t) for t in hi_in])
    keep.append(a)
    lo_out = hi_out = None
    lout_p = hout_p = None
    idx_t = None
    cnt_p = None
    tiled = _tiled(plan)
    lib = _lib.load()
    rows = tiled and ROWS and lib.vc_mlp_tiled_crown_mode(B) == 0
    # the rows form's workspace size is negative past its batch limit
    nws = int(lib.vc_mlp_crown_rows_workspace(plan.dims_p, plan.n, B)) if rows else 0
    rows = rows and nws >= 0
    if do_crown:
        if rows and ROWS_OWN_UNION:
            pass  # the rows form builds the union in its own pass over the bounds
        elif tiled:
            # union of the unstable sets and its index lists, on the device
            nw = sum(plan.dims[1:])
            flags = torch.empty(nw, dtype=torch.uint8, device=dev)
            call('vc_unstable_union_layers', lin_p, hin_p, plan.widths_p, plan.n, B,
                 ptr(flags), stream())
            idx_t = torch.empty(nw, dtype=torch.int32, device=dev)
            meta = torch.empty(2 * plan.n, dtype=torch.int32, device=dev)
            call('vc_union_compact', ptr(flags), plan.widths_p, plan.n, ptr(idx_t), ptr(meta),
                 stream())
            cnt_p = ptr(meta)
        else:
            idx_t, cnt = union_idx(plan, sb)
            a, cnt_p = host_array(ctypes.c_int32, cnt)
            keep.append(a)
        lo_out = [torch.empty_like(t) for t in lo_in]
        hi_out = [torch.empty_like(t) for t in hi_in]
        a, lout_p = host_array(ctypes.c_void_p, [ptr(t) for t in lo_out])
        keep.append(a)
        a, hout_p = host_array(ctypes.c_void_p, [ptr(t) for t in hi_out])
        keep.append(a)
    Q = 0
    S = acc0 = lb = A = acc = None
    if spec is not None:
        S, acc0 = fold_spec(plan, *spec)
        Q = S.shape[0]
        lb = torch.empty(B, Q, device=dev)
        if want_linear:
            A = torch.empty(B, Q, plan.dims[0], device=dev)
            acc = torch.empty(B, Q, device=dev)
    if tiled:
        seeds = None
        if SEED_COUNTER is not None:
            global SEED_ROW
            seeds = SEED_COUNTER[SEED_ROW]
            SEED_ROW += 1
        if rows:
            ws = torch.empty(max(nws, 8), dtype=torch.uint8, device=dev)
            call('vc_mlp_crown_rows', plan.dims_p, plan.n, ptr(plan.tfrag), ptr(plan.bias_cat),
                 B, ptr(xl), ptr(xh), lin_p, hin_p, lout_p, hout_p, ptr(idx_t), cnt_p,
                 1 if do_crown else 0, 1 if per_domain else 0, Q, ptr(S), ptr(acc0), ptr(lb),
                 ptr(A), ptr(acc), ptr(seeds), ptr(ws), nws, stream())
        else:
            call('vc_mlp_tiled_crown', plan.dims_p, plan.n, ptr(plan.tfrag), ptr(plan.bias_cat),
                 B, ptr(xl), ptr(xh), lin_p, hin_p, lout_p, hout_p, ptr(idx_t), cnt_p,
                 1 if do_crown else 0, 1 if per_domain else 0, Q, ptr(S), ptr(acc0), ptr(lb),
                 ptr(A), ptr(acc), ptr(seeds),
                 ptr(torch.empty(2, dtype=torch.int32, device=dev)), stream())
    else:
        call('vc_mlp_crown', plan.dims_p, plan.n, ptr(plan.frag[0]), ptr(plan.bias_cat), B,
             ptr(xl), ptr(xh), lin_p, hin_p, lout_p, hout_p, ptr(idx_t), cnt_p,
             1 if do_crown else 0, Q, ptr(S), ptr(acc0), ptr(lb), ptr(A), ptr(acc), stream())
    tight = None
    if do_crown:
        tight = {L: (lo_out[L], hi_out[L]) for L in range(plan.n)}
    return tight, lb, A, acc
