"""Oracle: bound primitives restated in PyTorch (CPU).

Test infrastructure: see the package docstring.  Each function follows the
reference function named in its docstring (paths relative to
src/vibecheck/ of the reference).  Supported ops: fc, relu, conv, reshape,
and add (a constant, or the residual merge of two live inputs), sub and mul
by constants -- the op set of the Linear/Conv/ReLU networks this engine
targets, with the affine ops the reference's ONNX reader emits around them.
Anything else raises NotImplementedError, as the reference does for
unsupported ops.
"""
import numpy as np
import torch
import torch.nn.functional as F


def make_slopes(lo, hi):
    """CROWN adaptive ReLU relaxation (verify_zono_bnb.py:503-522).

    Returns (lo_s, up_s, up_t, active, dead, unstable).
    """
    dt = lo.dtype
    lb_r = torch.clamp(lo, max=0)
    ub_r = torch.maximum(torch.clamp(hi, min=0), lb_r + 1e-8)
    up_s = ub_r / (ub_r - lb_r)
    up_t = -lb_r * up_s
    active = lo >= 0
    dead = hi <= 0
    unstable = ~active & ~dead
    a = active.to(dt)
    d = dead.to(dt)
    lo_s = (up_s > 0.5).to(dt) * (1 - a) * (1 - d) + a
    return lo_s, up_s, up_t, active, dead, unstable


def _unsupported(fn, op):
    raise NotImplementedError(
        f'{fn}: unsupported op {op["type"]!r} at {op["name"]!r}')


def _const(op, key, n, dt):
    """An add/sub 'bias' or a mul 'scale' as a flat tensor broadcastable
    against n values: the float64 constant rounded to dt, one value or n;
    otherwise a per-channel scale (in_shapes_nd (C, H, W),
    verify_zono_bnb.py:3523-3534) or a trailing-dimension vector
    (out_shape_nd, :3240-3251, :4490-4503) spelled out to n values."""
    v = op.get(key)
    if v is None:
        return None
    t = torch.as_tensor(v, dtype=dt).reshape(-1)
    if t.numel() in (1, n):
        return t
    shp_in = (op.get('in_shapes_nd') or [None])[0]
    shp_out = op.get('out_shape_nd')
    if key == 'scale' and shp_in is not None and len(shp_in) == 3 and shp_in[0] == t.numel():
        C, H, W = shp_in
        return t.view(C, 1, 1).expand(C, H, W).reshape(-1)
    if shp_out is not None and shp_out[-1] == t.numel():
        return t.reshape(*([1] * (len(shp_out) - 1)), -1).expand(*shp_out).reshape(-1)
    raise ValueError(f'{op["name"]}: {key} does not broadcast to {n} values')


def fork_points(gg):
    """Names consumed by more than one op (network.py:1713's 'fork_points'),
    from the gg when present."""
    if gg.get('fork_points') is not None:
        return gg['fork_points']
    cnt = {}
    for op in gg['ops']:
        for i in op['inputs']:
            cnt[i] = cnt.get(i, 0) + 1
    return {k for k, c in cnt.items() if c > 1}


def shared_gens_count(name_a, name_b, gg, gen_count):
    """_find_shared_gens_count (verify_zono_bnb.py:2387-2428): walk name_a's
    ancestors depth-first (a stack, each node's inputs pushed in order); the
    first one that is an ancestor of name_b and a fork point gives its
    generator count; none: the input's."""
    forks = fork_points(gg)
    pred = {op['name']: op['inputs'] for op in gg['ops']}

    def walk(name):
        out, stack, seen = [], [name], set()
        while stack:
            x = stack.pop()
            if x in seen:
                continue
            seen.add(x)
            out.append(x)
            for i in pred.get(x, []):
                stack.append(i)
        return out

    in_b = set(walk(name_b))
    for x in walk(name_a):
        if x in in_b and x in forks:
            return gen_count.get(x, 0)
    return gen_count.get(gg['input_name'], 0)


def _fc_nd(op, width):
    """The prefix of an fc in the N-D batched MatMul form, or None: an
    in_shapes_nd of two or more dims whose last is W.shape[1] and whose
    product is the input width (verify_zono_bnb.py:3145-3152)."""
    shp = (op.get('in_shapes_nd') or [None])[0]
    if (shp is not None and len(shp) >= 2 and op['W'].shape[1] == shp[-1]
            and width == int(np.prod(shp))):
        return tuple(int(s) for s in shp[:-1])
    return None


def point_forward(x, gg):
    """Concrete forward of a batch of points x (P, n_in).

    Returns (output (P, n_out), {layer_idx: pre-activation (P, n_L)}).
    Ground truth for sampling checks.
    """
    P = x.shape[0]
    act = {gg['input_name']: x}
    pre = {}
    for op in gg['ops']:
        a = act[op['inputs'][0]]
        t = op['type']
        if t == 'fc':
            pre_nd = _fc_nd(op, a.shape[-1])
            if pre_nd is not None:
                y = a.reshape(*a.shape[:-1], *pre_nd, op['W'].shape[1]) @ op['W'].T + op['bias']
                act[op['name']] = y.reshape(*a.shape[:-1], -1)
            else:
                act[op['name']] = a @ op['W'].T + op['bias']
        elif t == 'conv':
            y = F.conv2d(a.reshape(P, *op['in_shape']), op['kernel'],
                         op['bias'], stride=op['stride'],
                         padding=op['padding'])
            act[op['name']] = y.reshape(P, -1)
        elif t == 'relu':
            if 'layer_idx' in op:
                pre[op['layer_idx']] = a.clone()
            act[op['name']] = a.clamp(min=0)
        elif t == 'reshape':
            act[op['name']] = a
        elif t == 'add' and op.get('is_merge'):
            act[op['name']] = a + act[op['inputs'][1]]
        elif t == 'add':
            act[op['name']] = a + _const(op, 'bias', a.shape[1], a.dtype)
        elif t == 'sub':
            act[op['name']] = a - _const(op, 'bias', a.shape[1], a.dtype)
        elif t == 'mul':
            act[op['name']] = a * _const(op, 'scale', a.shape[1], a.dtype)
        else:
            _unsupported('point_forward', op)
    return act[gg['ops'][-1]['name']], pre


def ibp_forward_batched(xl, xh, gg, relu_clamps=None, root_sb=None):
    """Batched interval forward (verify_zono_bnb.py:1066-1153).

    fc/conv via mid/rad with |W|; relu intersects root bounds, then split
    clamps, repairs crossings with hi = max(hi, lo), records sb[L], and
    passes clamp(min=0) on.  Returns {layer_idx: (lo, hi)} of (B, n_L).
    """
    B = xl.shape[0]
    lo = {gg['input_name']: xl}
    hi = {gg['input_name']: xh}
    sb = {}
    for op in gg['ops']:
        t = op['type']
        name = op['name']
        l, h = lo[op['inputs'][0]], hi[op['inputs'][0]]
        if t == 'fc':
            mid, rad = (l + h) / 2, (h - l) / 2
            W, b = op['W'], op['bias']
            mc = mid @ W.T + b
            rc = rad @ W.T.abs()
            lo[name], hi[name] = mc - rc, mc + rc
        elif t == 'conv':
            mid, rad = (l + h) / 2, (h - l) / 2
            mc = F.conv2d(mid.reshape(B, *op['in_shape']), op['kernel'],
                          op['bias'], stride=op['stride'],
                          padding=op['padding'])
            rc = F.conv2d(rad.reshape(B, *op['in_shape']), op['kernel'].abs(),
                          None, stride=op['stride'], padding=op['padding'])
            lo[name] = (mc - rc).reshape(B, -1)
            hi[name] = (mc + rc).reshape(B, -1)
        elif t == 'relu':
            L = op.get('layer_idx')
            if L is not None:
                if root_sb is not None and L in root_sb:
                    l = torch.maximum(l, root_sb[L][0].unsqueeze(0))
                    h = torch.minimum(h, root_sb[L][1].unsqueeze(0))
                if relu_clamps is not None and L in relu_clamps:
                    cl, ch = relu_clamps[L]
                    l = torch.maximum(l, cl)
                    h = torch.minimum(h, ch)
                h = torch.maximum(h, l)
                sb[L] = (l.clone(), h.clone())
            lo[name], hi[name] = l.clamp(min=0), h.clamp(min=0)
        elif t == 'reshape':
            lo[name], hi[name] = l, h
        elif t == 'add' and op.get('is_merge'):
            # verify_zono_bnb.py:1133-1135
            lo[name] = l + lo[op['inputs'][1]]
            hi[name] = h + hi[op['inputs'][1]]
        elif t in ('add', 'sub'):
            # verify_zono_bnb.py:1136-1143
            b = _const(op, 'bias', l.shape[1], l.dtype)
            lo[name], hi[name] = (l + b, h + b) if t == 'add' else (l - b, h - b)
        elif t == 'mul':
            # verify_zono_bnb.py:1144-1148
            sc = _const(op, 'scale', l.shape[1], l.dtype)
            p, q = sc * l, sc * h
            lo[name], hi[name] = torch.minimum(p, q), torch.maximum(p, q)
        else:
            _unsupported('ibp_forward_batched', op)
    return sb


def zono_forward_batched(xl, xh, gg):
    """Batched zonotope forward (verify_zono_bnb.py:3079-3211, conv 3400-3425).

    State per domain: centre c (B, n) and generators G (B, n, K).  Input
    generators are the diagonal of the radii over dims with non-zero radius
    in any domain.  ReLU: lo/hi = c -/+ sum_k |G|, lambda = hi/(hi-lo) and
    mu = -hi*lo/(2(hi-lo)) on unstable neurons (0/1 on dead/active), one new
    generator column per unstable neuron, ranked by a cumulative count,
    padded to the batch maximum.  Returns (sb, (c, G)).
    """
    B, n_in = xl.shape
    dt = xl.dtype
    c = (xl + xh) / 2
    radii = (xh - xl) / 2
    varying = radii.abs().max(dim=0).values > 0
    K = int(varying.sum())
    if K == n_in:
        G = torch.diag_embed(radii)
    else:
        vidx = varying.nonzero(as_tuple=True)[0]
        G = torch.zeros(B, n_in, K, dtype=dt)
        G[:, vidx, torch.arange(K)] = radii[:, vidx]
    state = {gg['input_name']: (c, G)}
    gen_count = {gg['input_name']: K}
    sb = {}
    for op in gg['ops']:
        t = op['type']
        name = op['name']
        c_in, G_in = state[op['inputs'][0]]
        if t == 'add' and op.get('is_merge'):
            # verify_zono_bnb.py:3213-3234: shared columns summed, then a's
            # own columns, then b's
            c_b, G_b = state[op['inputs'][1]]
            sh = shared_gens_count(op['inputs'][0], op['inputs'][1], gg, gen_count)
            Ka, Kb = G_in.shape[2], G_b.shape[2]
            assert 0 <= sh <= Ka and 0 <= sh <= Kb
            G_out = torch.cat([G_in[:, :, :sh] + G_b[:, :, :sh], G_in[:, :, sh:],
                               G_b[:, :, sh:]], dim=2)
            state[name] = (c_in + c_b, G_out)
        elif t in ('add', 'sub'):
            # verify_zono_bnb.py:3235-3265: the centre moves
            b = _const(op, 'bias', c_in.shape[1], dt)
            if b is not None:
                c_in = c_in + b if t == 'add' else c_in - b
            state[name] = (c_in, G_in)
        elif t == 'mul':
            # verify_zono_bnb.py:3501-3536
            sc = _const(op, 'scale', c_in.shape[1], dt)
            state[name] = (c_in * sc, G_in * sc.reshape(1, -1, 1)
                           if sc.numel() > 1 else G_in * sc)
        elif t == 'fc':
            W = op['W']
            pre_nd = _fc_nd(op, c_in.shape[1])
            if pre_nd is not None:
                # N-D batched MatMul (verify_zono_bnb.py:3145-3168)
                Kc = G_in.shape[2]
                c_o = F.linear(c_in.reshape(B, *pre_nd, W.shape[1]), W,
                               op['bias']).reshape(B, -1)
                G_o = torch.einsum('...ik,oi->...ok',
                                   G_in.reshape(B, *pre_nd, W.shape[1], Kc),
                                   W).reshape(B, -1, Kc)
                state[name] = (c_o, G_o)
            else:
                state[name] = (c_in @ W.T + op['bias'],
                               torch.einsum('oi,bik->bok', W, G_in))
        elif t == 'conv':
            shp = op['in_shape']
            c_out = F.conv2d(c_in.reshape(B, *shp), op['kernel'],
                             bias=op['bias'], stride=op['stride'],
                             padding=op['padding']).reshape(B, -1)
            Kc = G_in.shape[2]
            if Kc == 0:
                G_out = torch.zeros(B, c_out.shape[1], 0, dtype=dt)
            else:
                g = G_in.permute(0, 2, 1).reshape(B * Kc, *shp)
                g = F.conv2d(g, op['kernel'], bias=None, stride=op['stride'],
                             padding=op['padding'])
                G_out = g.reshape(B, Kc, -1).permute(0, 2, 1).contiguous()
            state[name] = (c_out, G_out)
        elif t == 'relu':
            s = G_in.abs().sum(dim=2)
            lo = c_in - s
            hi = c_in + s
            ust = (lo < 0) & (hi > 0)
            dead = hi <= 0
            lam = torch.where(ust, hi / (hi - lo),
                              torch.where(dead, torch.zeros_like(hi),
                                          torch.ones_like(hi)))
            mu = torch.where(ust, -hi * lo / (2 * (hi - lo)),
                             torch.zeros_like(hi))
            c_out = lam * c_in + mu
            G_sc = G_in * lam.unsqueeze(-1)
            cnt = ust.sum(dim=1)
            max_k = int(cnt.max().item()) if B > 0 else 0
            if max_k == 0:
                G_out = G_sc
            else:
                n = c_in.shape[1]
                new = torch.zeros(B, n, max_k, dtype=dt)
                rank = ust.long().cumsum(dim=1) - 1
                bi = torch.arange(B).unsqueeze(1).expand(B, n)
                ri = torch.arange(n).unsqueeze(0).expand(B, n)
                new[bi[ust], ri[ust], rank[ust]] = mu[ust]
                G_out = torch.cat([G_sc, new], dim=2)
            state[name] = (c_out, G_out)
            if 'layer_idx' in op:
                sb[op['layer_idx']] = (lo.clone(), hi.clone())
        elif t == 'reshape':
            state[name] = (c_in, G_in)
        else:
            _unsupported('zono_forward_batched', op)
        gen_count[name] = state[name][1].shape[2]
    return sb, state[gg['ops'][-1]['name']]


def spec_backward_batched(tight, xl, xh, gg, spec_ew=None,
                          return_input_linear=False, alpha_at_layer=None,
                          relu_split_beta=None, seed_ew_at=None,
                          seed_acc=None):
    """Batched CROWN backward + concretization
    (verify_zono_bnb.py:4270-4453 fc/relu, 4568-4593 conv, 5117-5134).

    Seeds ew (B, Q, n_out) with the spec rows (or ``seed_ew_at``), walks the
    ops in reverse: fc adds ew.b to acc and maps ew <- ew @ W; relu splits
    ew into positive/negative parts, adds en.up_t to acc and maps
    ew <- ep*lo_s + en*up_s (lo_s = active + unstable*alpha when alpha is
    given; + beta when given); conv adds the per-channel bias term and maps
    ew through conv_transpose2d.  Concretizes
    lb = acc + pos(A).xl + neg(A).xh.
    """
    ops = gg['ops']
    B, n_in = xl.shape
    dt = xl.dtype
    if seed_ew_at is not None:
        ew_at = {k: v.clone() for k, v in seed_ew_at.items()}
        Q = next(iter(seed_ew_at.values())).shape[1]
        acc = (torch.zeros(B, Q, dtype=dt) if seed_acc is None
               else seed_acc.clone())
    else:
        qids = sorted(spec_ew.keys())
        Q = len(qids)
        Wq = torch.stack([torch.as_tensor(spec_ew[q][0], dtype=dt).reshape(-1)
                          for q in qids])
        bq = torch.tensor([float(spec_ew[q][1]) for q in qids], dtype=dt)
        ew_at = {ops[-1]['name']: Wq.unsqueeze(0).expand(B, -1, -1).clone()}
        acc = bq.unsqueeze(0).expand(B, -1).clone()

    def _put(inp, v):
        prev = ew_at.get(inp)
        ew_at[inp] = v if prev is None else prev + v

    for op in reversed(ops):
        name = op['name']
        if name not in ew_at:
            continue
        ew = ew_at[name]
        t = op['type']
        if t == 'fc':
            shp_in = (op.get('in_shapes_nd') or [None])[0]
            shp_out = op.get('out_shape_nd')
            if (shp_in is not None and len(shp_in) >= 2
                    and op['W'].shape[1] == shp_in[-1]
                    and shp_out is not None and len(shp_out) >= 2):
                # N-D batched MatMul (verify_zono_bnb.py:4382-4401)
                n_p = int(np.prod(shp_out[:-1]))
                ew_nd = ew.reshape(*ew.shape[:-1], n_p, int(shp_out[-1]))
                acc = acc + (ew_nd * op['bias']).sum(dim=(-2, -1))
                back = ew_nd @ op['W']
                _put(op['inputs'][0], back.reshape(*back.shape[:-2], -1))
            else:
                acc = acc + ew @ op['bias']
                _put(op['inputs'][0], ew @ op['W'])
        elif t == 'relu':
            if 'layer_idx' in op:
                L = op['layer_idx']
                lo, hi = tight[L]
                lo_s, up_s, up_t, active, dead, unstable = make_slopes(lo, hi)
                ep = ew.clamp(min=0)
                en = ew.clamp(max=0)
                acc = acc + (en * up_t.unsqueeze(1)).sum(dim=-1)
                if alpha_at_layer is not None and L in alpha_at_layer:
                    a = alpha_at_layer[L]
                    if a.dim() == 2:
                        ls = (active.to(dt) + unstable.to(dt) * a).unsqueeze(1)
                    else:
                        ls = (active.to(dt).unsqueeze(1)
                              + unstable.to(dt).unsqueeze(1) * a)
                    back = ep * ls + en * up_s.unsqueeze(1)
                else:
                    back = ep * lo_s.unsqueeze(1) + en * up_s.unsqueeze(1)
                if relu_split_beta is not None and L in relu_split_beta:
                    back = back + relu_split_beta[L].unsqueeze(1)
            else:
                back = ew
            _put(op['inputs'][0], back)
        elif t == 'conv':
            C_out, H_o, W_o = op['out_shape']
            bias_flat = op['bias'].repeat_interleave(H_o * W_o)
            acc = acc + (ew * bias_flat).sum(dim=-1)
            back = F.conv_transpose2d(
                ew.reshape(B * Q, *op['out_shape']), op['kernel'], bias=None,
                stride=op['stride'], padding=op['padding'],
                output_padding=op['output_padding'])
            _put(op['inputs'][0], back.reshape(B, Q, -1))
        elif t == 'reshape':
            prev = ew_at.get(op['inputs'][0])
            ew_at[op['inputs'][0]] = ew.clone() if prev is None else prev + ew
        elif t == 'add' and op.get('is_merge'):
            # verify_zono_bnb.py:4462-4469: to both inputs, no constant
            for i in op['inputs']:
                _put(i, ew.clone())
        elif t in ('add', 'sub'):
            # verify_zono_bnb.py:4470-4518: acc +/-= (ew * bias).sum
            b = _const(op, 'bias', ew.shape[-1], dt)
            if b is not None:
                term = (ew * b).sum(dim=-1)
                acc = acc + term if t == 'add' else acc - term
            _put(op['inputs'][0], ew.clone())
        elif t == 'mul':
            # verify_zono_bnb.py:4686-4712
            _put(op['inputs'][0], ew * _const(op, 'scale', ew.shape[-1], dt))
        else:
            _unsupported('spec_backward_batched', op)

    A = ew_at.get(gg['input_name'])
    if A is None:
        if return_input_linear:
            return acc, torch.zeros(B, Q, n_in, dtype=dt), acc
        return acc
    lb = (acc + (A.clamp(min=0) * xl.unsqueeze(1)).sum(dim=-1)
          + (A.clamp(max=0) * xh.unsqueeze(1)).sum(dim=-1))
    if return_input_linear:
        return lb, A, acc
    return lb


def crown_intermediate_batched(gg, xl, xh, chunk=2048, sb=None):
    """Backward-CROWN intermediate pre-ReLU bounds
    (verify_zono_bnb.py:4077-4147).

    Starts from the zonotope bounds (or ``sb`` when given).  For each ReLU
    layer L in ascending order: seed [+I; -I] rows at L's input for the
    neurons unstable in ANY domain of the batch, in chunks of ``chunk``,
    run the backward through the already-tightened earlier layers, and
    intersect: lo = max(lo, lb+), hi = max(min(hi, -lb-), lo).
    """
    if sb is None:
        sb, _ = zono_forward_batched(xl, xh, gg)
    tight = {L: (lo.clone(), hi.clone()) for L, (lo, hi) in sb.items()}
    relu_by_L = {op['layer_idx']: op for op in gg['ops']
                 if op['type'] == 'relu' and 'layer_idx' in op}
    B = xl.shape[0]
    dt = xl.dtype
    for L in sorted(tight):
        if L not in relu_by_L:
            continue
        feed = relu_by_L[L]['inputs'][0]
        lo_L, hi_L = tight[L]
        n = lo_L.shape[1]
        idx = (((lo_L < 0) & (hi_L > 0)).any(dim=0)).nonzero(as_tuple=True)[0]
        m = int(idx.numel())
        if m == 0:
            continue
        new_lo = lo_L.clone()
        new_hi = hi_L.clone()
        for c0 in range(0, m, max(1, int(chunk))):
            cidx = idx[c0:c0 + max(1, int(chunk))]
            k = int(cidx.numel())
            eye = torch.zeros(k, n, dtype=dt)
            eye[torch.arange(k), cidx] = 1.0
            seed = {feed: torch.cat([eye, -eye], 0).unsqueeze(0)
                    .expand(B, -1, -1)}
            sl = spec_backward_batched(tight, xl, xh, gg, None,
                                       seed_ew_at=seed,
                                       seed_acc=torch.zeros(B, 2 * k, dtype=dt))
            lo_c = torch.maximum(lo_L[:, cidx], sl[:, :k])
            hi_c = torch.maximum(torch.minimum(hi_L[:, cidx], -sl[:, k:]), lo_c)
            new_lo[:, cidx] = lo_c
            new_hi[:, cidx] = hi_c
        tight[L] = (new_lo, new_hi)
    return tight


def alpha_crown_batched(xl, xh, gg, spec_ew, n_iters=10, lr=0.25,
                        lr_decay=0.98, early_stop_eps=1e-6, sb=None,
                        return_trace=False):
    """Batched alpha-CROWN with Adam (verify_zono_bnb.py:5137-5288).

    alpha_L (B, n_L) starts at (up_s > 0.5) * unstable on the zonotope
    bounds (or ``sb``); each iteration evaluates the backward with alpha,
    keeps the running best lb, stops when every best lb is > 0, otherwise
    steps Adam on -sum(lb), clamps alpha to [0, 1], stops when the global
    max of the best lb improved by less than ``early_stop_eps`` (from the
    second iteration on), and decays lr.  Returns best (B, Q); with
    ``return_trace`` also the number of evaluated iterations.
    """
    if sb is None:
        with torch.no_grad():
            sb, _ = zono_forward_batched(xl, xh, gg)
    dt = xl.dtype
    alpha = {}
    for L, (lo, hi) in sb.items():
        _, up_s, _, _, _, unstable = make_slopes(lo, hi)
        alpha[L] = ((up_s > 0.5).to(dt) * unstable.to(dt)).detach().clone() \
            .requires_grad_(True)
    if not alpha:
        with torch.no_grad():
            lb = spec_backward_batched(sb, xl, xh, gg, spec_ew)
        return (lb, 1) if return_trace else lb
    opt = torch.optim.Adam([alpha[L] for L in alpha], lr=lr)
    best = None
    prev_max = -float('inf')
    n_eval = 0
    for it in range(n_iters):
        opt.zero_grad()
        lb = spec_backward_batched(sb, xl, xh, gg, spec_ew,
                                   alpha_at_layer=alpha)
        n_eval += 1
        with torch.no_grad():
            best = (lb.detach().clone() if best is None
                    else torch.maximum(best, lb.detach()))
            curr_max = float(best.max().item())
        if bool((best > 0).all().item()):
            break
        (-lb.sum()).backward()
        opt.step()
        with torch.no_grad():
            for L in alpha:
                alpha[L].clamp_(0.0, 1.0)
        if it > 0 and curr_max - prev_max < early_stop_eps:
            break
        prev_max = curr_max
        for g in opt.param_groups:
            g['lr'] *= lr_decay
    if return_trace:
        return best, n_eval
    return best


def split_domain_bounds(xl, xh, gg, sb_root, relu_clamps, no_reforward=False):
    """Pre-relu bounds of a batch of ReLU-split domains (the inner
    ``_sb_for_domains`` of verify_milp.py:2698-2721).

    ``no_reforward``: the root bounds broadcast to every domain, intersected
    with the split clamps where a layer has any (then crossing repair).
    Otherwise an IBP forward of the (B, n_in) boxes with the clamps and the
    root bounds intersected at every relu."""
    if no_reforward:
        B = xl.shape[0]
        sb = {}
        for L, (lo_r, hi_r) in sb_root.items():
            lo = lo_r.reshape(1, -1).expand(B, -1).clone()
            hi = hi_r.reshape(1, -1).expand(B, -1).clone()
            if relu_clamps and L in relu_clamps:
                cl, ch = relu_clamps[L]
                lo = torch.maximum(lo, cl)
                hi = torch.minimum(hi, ch)
                hi = torch.maximum(hi, lo)
            sb[L] = (lo, hi)
        return sb
    root = {L: (lo.reshape(-1), hi.reshape(-1)) for L, (lo, hi) in sb_root.items()}
    return ibp_forward_batched(xl, xh, gg, relu_clamps=relu_clamps or None,
                               root_sb=root)


def beta_crown_bound(sb, xl, xh, gg, spec_ew, beta_sign, n_iters=10, lr=0.25,
                     return_trace=False, alpha_init=None):
    """Per-domain joint alpha/beta bound of one batch of ReLU-split domains
    (verify_milp.py:2762-2807).

    alpha starts at the root alpha ``alpha_init[L]`` (n_L,) broadcast to
    every domain where given, else at (up_s > 0.5) * unstable on ``sb``;
    beta starts at 0 and enters the backward as beta * sign at each split
    neuron (sign +1 for an OFF split, -1 for ON).  Adam on -sum(lb); alpha
    clamped to [0, 1], beta to >= 0; stops when every best lb is > 0.
    Returns best (B, Q); with ``return_trace`` also the number of
    evaluated iterations.
    """
    dt = xl.dtype
    alpha = {}
    for L, (lo, hi) in sb.items():
        if alpha_init is not None and L in alpha_init:
            a0 = alpha_init[L].to(dt).reshape(1, -1).expand(lo.shape[0], -1)
            alpha[L] = a0.detach().clone().requires_grad_(True)
            continue
        _, up_s, _, _, _, unstable = make_slopes(lo, hi)
        alpha[L] = ((up_s > 0.5).to(dt) * unstable.to(dt)).detach().clone() \
            .requires_grad_(True)
    beta = {L: torch.zeros_like(s).requires_grad_(True)
            for L, s in beta_sign.items()}
    opt = torch.optim.Adam(list(alpha.values()) + list(beta.values()), lr=lr)
    best = None
    n_eval = 0
    for _ in range(max(1, n_iters)):
        opt.zero_grad()
        rsb = {L: beta[L] * beta_sign[L] for L in beta} or None
        lb = spec_backward_batched(sb, xl, xh, gg, spec_ew,
                                   alpha_at_layer=alpha, relu_split_beta=rsb)
        n_eval += 1
        with torch.no_grad():
            best = (lb.detach().clone() if best is None
                    else torch.maximum(best, lb.detach()))
        if bool((best > 0).all()):
            break
        (-lb.sum()).backward()
        opt.step()
        with torch.no_grad():
            for L in alpha:
                alpha[L].clamp_(0.0, 1.0)
            for L in beta:
                beta[L].clamp_(min=0.0)
    if return_trace:
        return best, n_eval
    return best


def beta_signs_from_clamps(relu_clamps):
    """sign +1 where ch == 0 (OFF), -1 where cl == 0 (ON), else 0
    (verify_milp.py:2777-2784)."""
    out = {}
    for L, (cl, ch) in relu_clamps.items():
        s = torch.zeros_like(cl)
        s[ch == 0] = 1.0
        s[cl == 0] = -1.0
        out[L] = s
    return out
