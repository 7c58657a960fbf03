"""ReLU-split branch-and-bound bound on the GPU: the per-batch body of the
reference's ``_ibp_crown_bab`` (verify_milp.py:2698-2807).

A batch of subdomains of ONE input box, each fixing the sign of a few ReLU
neurons (split clamps), is bounded by per-domain alpha/beta-CROWN: the
pre-relu bounds are refreshed under the clamps (IBP forward with the root
bounds intersected, or the root bounds broadcast when ``no_reforward``),
then Adam optimises alpha (lower relu slopes, in [0, 1]) and beta (the
Lagrange multipliers of the split half-spaces, >= 0) jointly on -sum(lb).

Everything runs in the HIP library: the clamps come from per-domain split
lists (vc_split_clamps), the backward with the signed beta
(vc_backward_fc / vc_backward_relu), the analytic gradient sweep
(vc_alpha_grad_step / _reduce / _input), and the two Adam updates
(vc_adam_step for alpha, vc_beta_adam_step for beta).
"""
import torch

from ._lib import call, f32, ptr, stream
from .verify_zono_bnb import (_alpha_backward_and_grad, _check_dtype,
                              _ibp_forward_graph_batched, _spec_rows)

__all__ = ['_split_clamps_batched', '_sb_for_domains', '_ibp_crown_bab_bound']


def _split_clamps_batched(layer, neuron, side, widths, device):
    """Dense ``relu_clamps`` and beta signs from per-domain split lists.

    layer/neuron/side: (D, S) int64 GPU tensors; slot (d, s) splits neuron
    ``neuron`` of relu layer ``layer`` OFF (side 0, z <= 0) or ON (side 1,
    z >= 0); layer -1 marks an unused slot.  ``widths[L]`` = n_L.
    Returns (relu_clamps {L: (cl, ch)}, beta_sign {L: sign}) for the layers
    that hold at least one split -- the tensors the reference builds in its
    per-domain loop (verify_milp.py:2738-2752) and sign loop (:2777-2784).
    """
    if layer.dim() != 2 or layer.shape != neuron.shape or layer.shape != side.shape:
        raise ValueError('split lists must be (D, S) tensors of one shape')
    layer = layer.to(device=device, dtype=torch.int64).contiguous()
    neuron = neuron.to(device=device, dtype=torch.int64).contiguous()
    side = side.to(device=device, dtype=torch.int64).contiguous()
    D, S = layer.shape
    present = sorted(int(v) for v in torch.unique(layer).tolist() if v >= 0)
    st = stream()
    clamps, signs = {}, {}
    for L in present:
        n = int(widths[L])
        cl = torch.empty(D, n, device=device)
        ch = torch.empty_like(cl)
        sg = torch.empty_like(cl)
        call('vc_split_clamps', ptr(layer), ptr(neuron), ptr(side), D, S, L, n,
             ptr(cl), ptr(ch), ptr(sg), st)
        clamps[L] = (cl, ch)
        signs[L] = sg
    return clamps, signs


def _sb_for_domains(xl, xh, gg, sb_root, relu_clamps, B, device, dtype,
                    no_reforward=False):
    """Per-domain pre-relu bounds (the inner ``_sb_for_domains`` of
    verify_milp.py:2698-2721).

    ``no_reforward``: the root bounds broadcast to the B domains, with the
    clamps intersected (and crossings repaired) on the layers that have
    clamps.  Otherwise the batched IBP forward of the B copies of the box
    under the clamps, with the root bounds intersected at every relu.
    xl/xh: the box, (n_in,) or (B, n_in).  sb_root: {L: (lo, hi)} of (n_L,).
    """
    _check_dtype(dtype)
    st = stream()
    if no_reforward:
        sb = {}
        for L, (lo_r, hi_r) in sb_root.items():
            lo_r = f32(lo_r).reshape(-1)
            hi_r = f32(hi_r).reshape(-1)
            n = lo_r.shape[0]
            if relu_clamps and L in relu_clamps:
                cl, ch = relu_clamps[L]
                lo = torch.empty(B, n, device=lo_r.device)
                hi = torch.empty_like(lo)
                call('vc_ibp_relu', None, None, B, n, ptr(lo_r), ptr(hi_r),
                     ptr(f32(cl)), ptr(f32(ch)), ptr(lo), ptr(hi), None, None, st)
            else:
                lo = lo_r.unsqueeze(0).expand(B, n).contiguous()
                hi = hi_r.unsqueeze(0).expand(B, n).contiguous()
            sb[L] = (lo, hi)
        return sb
    xl_b, xh_b = _expand_box(xl, xh, B)
    root = {L: (f32(lo).reshape(-1), f32(hi).reshape(-1))
            for L, (lo, hi) in sb_root.items()}
    return _ibp_forward_graph_batched(xl_b, xh_b, gg, device, dtype,
                                      relu_clamps=relu_clamps or None,
                                      root_sb=root)


def _expand_box(xl, xh, B):
    xl, xh = f32(xl), f32(xh)
    if xl.dim() == 1:
        xl = xl.unsqueeze(0).expand(B, -1).contiguous()
        xh = xh.unsqueeze(0).expand(B, -1).contiguous()
    if xl.shape[0] != B:
        raise ValueError(f'box batch {xl.shape[0]} != {B} domains')
    return xl, xh


def _ibp_crown_bab_bound(gg, xl, xh, sb_root, relu_clamps, spec_ew, device,
                         dtype, *, alpha_iters=8, lr=0.25, alpha_init=None,
                         no_reforward=False, time_left=None, beta_sign=None,
                         sb=None, return_trace=False):
    """Best per-domain alpha/beta-CROWN lower bound of a batch of ReLU-split
    domains (verify_milp.py:2738-2807, the bound of each ``_ibp_crown_bab``
    step).

    gg: the network; xl/xh: the box, (n_in,) or (B, n_in); sb_root: root
    pre-relu bounds {L: (n_L,)}; relu_clamps: {L: (cl, ch)} (B, n_L) with 0
    at split neurons and -inf/+inf elsewhere (``_split_clamps_batched``
    builds them from split lists); spec_ew: {q: (w, b)}, the reference
    passes one query.  alpha starts at the root ``alpha_init[L]`` (n_L,)
    broadcast, else at (up_s > 0.5) * unstable of the domain bounds; beta at
    0.  Each of at most ``alpha_iters`` (>= 1) iterations: evaluate the
    backward with alpha and the signed beta, keep the best lb, stop when
    every best lb is > 0 or ``time_left()`` <= 3 s, else one Adam step
    (lr, torch defaults) on -sum(lb) for alpha and beta, clamp alpha to
    [0, 1] and beta to >= 0.  ``beta_sign`` (extension) supplies the signs
    when the caller has them already; ``sb`` (extension) supplies the domain
    bounds.  Returns best (B, Q); ``return_trace`` adds the number of
    evaluations.
    """
    _check_dtype(dtype)
    if not relu_clamps:
        relu_clamps = {}
    B = None
    for cl, _ in relu_clamps.values():
        B = cl.shape[0]
        break
    if B is None:
        B = xl.shape[0] if xl.dim() == 2 else 1
    xl_b, xh_b = _expand_box(xl, xh, B)
    dev = xl_b.device
    st = stream()
    if sb is None:
        sb = _sb_for_domains(xl_b, xh_b, gg, sb_root, relu_clamps, B, device,
                             dtype, no_reforward=no_reforward)
    sb = {L: (f32(lo), f32(hi)) for L, (lo, hi) in sb.items()}
    Wq, bq = _spec_rows(spec_ew, dev)
    Q = Wq.shape[0]

    # alpha: one flat buffer over all relu layers
    Ls = sorted(sb)
    sizes = [sb[L][0].numel() for L in Ls]
    na = sum(sizes)
    a_flat = torch.empty(na, device=dev)
    ga_flat = torch.zeros(na, device=dev)
    am = torch.zeros(na, device=dev)
    av = torch.zeros(na, device=dev)
    alpha, galpha = {}, {}
    off = 0
    for L, sz in zip(Ls, sizes):
        shape = sb[L][0].shape
        alpha[L] = a_flat[off:off + sz].view(shape)
        galpha[L] = ga_flat[off:off + sz].view(shape)
        if alpha_init is not None and L in alpha_init:
            a0 = f32(alpha_init[L]).reshape(1, -1)
            alpha[L].copy_(a0.expand(shape))
        else:
            call('vc_alpha_init', ptr(sb[L][0]), ptr(sb[L][1]), sz,
                 ptr(alpha[L]), st)
        off += sz

    # beta: one flat buffer over the layers with clamps
    Lb = sorted(L for L in relu_clamps if L in sb)
    bsz = [sb[L][0].numel() for L in Lb]
    nb = sum(bsz)
    b_flat = torch.zeros(nb, device=dev)
    bs_flat = torch.zeros(nb, device=dev)        # signed beta, seen by the backward
    gb_flat = torch.zeros(nb, device=dev)
    sg_flat = torch.empty(nb, device=dev)
    bm = torch.zeros(nb, device=dev)
    bv = torch.zeros(nb, device=dev)
    beta_s, gbeta = {}, {}
    off = 0
    for L, sz in zip(Lb, bsz):
        shape = sb[L][0].shape
        beta_s[L] = bs_flat[off:off + sz].view(shape)
        gbeta[L] = gb_flat[off:off + sz].view(shape)
        sg = sg_flat[off:off + sz]
        if beta_sign is not None and L in beta_sign:
            sg.copy_(f32(beta_sign[L]).reshape(-1))
        else:
            cl, ch = relu_clamps[L]
            call('vc_split_beta_sign', ptr(f32(cl)), ptr(f32(ch)), sz, ptr(sg), st)
        off += sz

    best = torch.empty(B, Q, device=dev)
    red = torch.empty(2, device=dev)
    b1, b2, eps = 0.9, 0.999, 1e-8
    n_eval = 0
    step = 0
    n_it = max(1, int(alpha_iters))
    for it in range(n_it):
        # the Adam step after the last evaluation is never used: skip its gradient
        last = it == n_it - 1
        lb = _alpha_backward_and_grad(sb, xl_b, xh_b, gg, Wq, bq, alpha, not last,
                                      galpha, beta=beta_s or None,
                                      gbeta=gbeta or None)
        n_eval += 1
        call('vc_best_update', ptr(best), ptr(lb.contiguous()), B * Q,
             1 if it == 0 else 0, ptr(red), st)
        all_pos = float(red[1].item()) > 0.5
        if all_pos or last or (time_left is not None and time_left() <= 3.0):
            break
        step += 1
        bc1 = 1 - b1 ** step
        bc2 = (1 - b2 ** step) ** 0.5
        if na:
            call('vc_adam_step', ptr(a_flat), ptr(ga_flat), ptr(am), ptr(av), na,
                 b1, b2, eps, lr / bc1, bc2, 0.0, 1.0, st)
        if nb:
            call('vc_beta_adam_step', ptr(b_flat), ptr(sg_flat), ptr(gb_flat),
                 ptr(bm), ptr(bv), nb, b1, b2, eps, lr / bc1, bc2, ptr(bs_flat), st)
    if return_trace:
        return best, n_eval
    return best
