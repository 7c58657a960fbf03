"""Batched bound primitives on the GPU (HIP library), with the reference's
function names and signatures (verify_zono_bnb.py of the reference).

Every function takes the reference's ``gg`` dict (fc / relu / conv /
reshape ops, and the constant add / sub / mul and residual-merge add ops)
and fp32 GPU tensors, computes with the kernels of
libvibecheck_amd.so, and returns new tensors.  Unsupported ops raise
NotImplementedError, fp64 raises NotImplementedError, CPU tensors raise
RuntimeError: there is no other compute path.
"""
import torch

from . import _lib, mlp_fused
from ._lib import call, f32, ptr, stream

__all__ = ['_make_slopes', '_ibp_forward_graph_batched',
           '_forward_zonotope_graph_batched', '_crown_intermediate_batched',
           '_spec_backward_graph_batched',
           '_run_alpha_crown_inputsplit_batched']

# Use the whole-network kernels for narrow fc/ReLU chains (<= 64 wide).
# Switching this off routes those nets through the layer-wise kernels.
FUSED_MLP = True
# Fuse a relu relaxation into the conv backward after it where the conv
# qualifies (vc_backward_relu_conv); off: the relu is applied on its own.
FUSED_RELU_CONV = True


def _plan(gg, dev):
    return mlp_fused.plan_for(gg, dev) if FUSED_MLP else None


def _zono_sb(gg, xl, xh, device, dtype):
    """Zonotope pre-activation bounds only (the fused kernel when the net
    qualifies, else the layer-wise forward)."""
    plan = _plan(gg, xl.device)
    if plan is not None:
        sb, _ = mlp_fused.zono_bounds(
            plan, xl, xh,
            lambda a, b: _forward_zonotope_graph_batched(a, b, gg, device, dtype)[0])
        return sb
    return _forward_zonotope_graph_batched(xl, xh, gg, device, dtype)[0]


def _check_dtype(dtype):
    if dtype is not None and dtype != torch.float32:
        raise NotImplementedError(
            f'vibecheck_amd computes in fp32 only, got {dtype}')


# --------------------------------------------------------------------------
# Device copies of the network parameters, cached on the gg dict
# --------------------------------------------------------------------------

def _op_params(op, device):
    """fp32 contiguous device copies of an op's tensors (cached on the op,
    like the reference caches converted biases on op dicts,
    verify_zono_bnb.py:4482-4486)."""
    key = '_vc_amd_params'
    cached = op.get(key)
    if cached is not None and cached['device'] == device:
        return cached
    p = {'device': device}
    if op['type'] == 'fc':
        p['W'] = op['W'].detach().to(device=device, dtype=torch.float32).contiguous()
        b = op.get('bias')
        p['b'] = (None if b is None else
                  torch.as_tensor(b).detach().to(device=device, dtype=torch.float32)
                  .reshape(-1).contiguous())
        p['n_out'], p['n_in'] = p['W'].shape
    elif op['type'] == 'conv':
        k = op['kernel'].detach().to(device=device, dtype=torch.float32).contiguous()
        if k.dim() != 4:
            raise NotImplementedError('vibecheck_amd: conv kernels must be 4-D')
        p['K'] = k
        b = op.get('bias')
        p['b'] = (None if b is None else
                  torch.as_tensor(b).detach().to(device=device, dtype=torch.float32)
                  .reshape(-1).contiguous())
        C_in, H, W = op['in_shape']
        C_out, Ho, Wo = op['out_shape']
        kh, kw = k.shape[2], k.shape[3]
        sh, sw = _pair(op['stride'])
        ph, pw = _pair(op['padding'])
        p['geom'] = (C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, Ho, Wo)
        p['n_in'] = C_in * H * W
        p['n_out'] = C_out * Ho * Wo
    op[key] = p
    return p


def _prod(shape):
    n = 1
    for s in shape:
        n *= int(s)
    return n


def _fc_form(op, width):
    """How an fc reads a node of ``width`` values per domain: (P, nd_out).

    P = 1 is the plain form, width == W.shape[1].  The N-D batched MatMul
    form (an ONNX MatMul on a (prefix..., n_in) input,
    verify_zono_bnb.py:3145-3168 and 4382-4401) has in_shapes_nd[0] with
    two or more dims, W.shape[1] equal to its last and width equal to its
    product: W applies to each of the P = prod(prefix) slices of n_in
    values, and the output holds P slices of W.shape[0].  nd_out tells
    whether the op also carries the out_shape_nd the reference's backward
    needs for that form (two or more dims).  Any other width raises
    ValueError: the kernels would read a wider tensor as rows of
    W.shape[1]."""
    n_out, n_in = (int(s) for s in op['W'].shape)
    shp = (op.get('in_shapes_nd') or [None])[0]
    if shp is not None and len(shp) >= 2 and int(shp[-1]) == n_in \
            and width == _prod(shp):
        P = _prod(shp[:-1])
        shp_o = op.get('out_shape_nd')
        nd_out = shp_o is not None and len(shp_o) >= 2 and _prod(shp_o) == P * n_out
        return P, nd_out
    if width == n_in:
        return 1, True
    raise ValueError(f'fc {op["name"]!r}: input of {width} values per domain, but W is '
                     f'{n_out}x{n_in} and in_shapes_nd is {shp}')


def validate_gg(gg, n_in=None):
    """The width of every node of ``gg``, checked op by op from the input's
    (``n_in``, else gg['input_n'], else the product of gg['input_shape']
    past the batch dim) before any launch, with the ops' shapes only (no
    device tensors): an fc reads W.shape[1] values or the N-D MatMul form
    (_fc_form); a conv reads prod(in_shape) and writes prod(out_shape); a
    residual merge adds two nodes of one width; relu, reshape and the
    constant add / sub / mul keep the width.  Raises ValueError on the
    first mismatch, NotImplementedError on an op type outside
    fc / conv / relu / reshape / add / sub / mul.  Returns {name: width}."""
    if n_in is None:
        n_in = gg.get('input_n')
        if n_in is None:
            shp = gg.get('input_shape')
            if shp is None:
                raise ValueError('gg has neither input_n nor input_shape')
            n_in = _prod(shp[1:]) if len(shp) > 1 else _prod(shp)
    width = {gg['input_name']: int(n_in)}
    for op in gg['ops']:
        t, name = op['type'], op['name']
        for i in op['inputs']:
            if i not in width:
                raise ValueError(f'{t} {name!r}: input {i!r} is not computed before it')
        w = width[op['inputs'][0]]
        if t == 'fc':
            P, _ = _fc_form(op, w)
            width[name] = P * int(op['W'].shape[0])
        elif t == 'conv':
            want = _prod(op['in_shape'])
            if w != want:
                raise ValueError(f'conv {name!r}: input of {w} values per domain, '
                                 f'in_shape {tuple(op["in_shape"])} holds {want}')
            width[name] = _prod(op['out_shape'])
        elif t == 'add' and op.get('is_merge'):
            w2 = width[op['inputs'][1]]
            if w2 != w:
                raise ValueError(f'add {name!r}: merges widths {w} and {w2}')
            width[name] = w
        elif t in ('relu', 'reshape', 'add', 'sub', 'mul'):
            width[name] = w
        else:
            _unsupported('validate_gg', op)
    return width


def _widths(gg, n_in):
    """validate_gg for a call on inputs of n_in values per domain, cached on
    the gg for its op list and input width."""
    key = (id(gg['ops']), len(gg['ops']), int(n_in))
    hit = gg.get('_vc_amd_widths')
    if hit is not None and hit[0] == key:
        return hit[1]
    w = validate_gg(gg, n_in)
    gg['_vc_amd_widths'] = (key, w)
    return w


def _conv_t_taps(p, st):
    """The conv kernel's transposed taps packed per output-parity class
    (vc_conv_t_pack), made on first use by a backward pass and cached with
    the op's other device tensors."""
    packed = p.get('KT')
    if packed is None:
        C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, Ho, Wo = p['geom']
        n = _lib.load().vc_conv_t_pack_floats(C_out, C_in, kh, kw, sh, sw)
        if n < 0:
            raise RuntimeError(f'vc_conv_t_pack_floats: bad geometry {p["geom"]}')
        packed = torch.empty(n, device=p['K'].device)
        call('vc_conv_t_pack', ptr(p['K']), C_out, C_in, kh, kw, sh, sw, ph, pw,
             ptr(packed), st)
        p['KT'] = packed
    return packed


def _pair(v):
    if isinstance(v, int):
        return v, v
    v = tuple(int(x) for x in v)
    return (v[0], v[0]) if len(v) == 1 else (v[0], v[1])


def _unsupported(fn, op):
    raise NotImplementedError(
        f'{fn}: unsupported op {op["type"]!r} at {op["name"]!r} -- silently '
        f'skipping would certify unsound bounds')


# --------------------------------------------------------------------------
# add / sub / mul: their constants, and residual merges
# --------------------------------------------------------------------------

def _op_const(op, key, device, n):
    """An add/sub op's 'bias' or a mul op's 'scale' as an fp32 device
    vector of n values, or of one value for a scalar (None when the op has
    none).  The reference converts the float64 constant with
    torch.as_tensor(..., dtype=float32) and broadcasts it against the n
    values: a vector of the trailing N-D dimension repeats along the
    leading ones (out_shape_nd, verify_zono_bnb.py:3240-3251, 4490-4503);
    a mul's per-channel vector repeats over each channel's H x W
    (in_shapes_nd, :3523-3534, :4702-4708).  Cached on the op."""
    cached = op.get('_vc_amd_' + key)
    if cached is not None and cached[0] == (str(device), n):
        return cached[1]
    v = op.get(key)
    if v is None:
        return None
    t = torch.as_tensor(v, dtype=torch.float32).reshape(-1).cpu()
    k = t.numel()
    if k not in (1, n):
        shp_in = (op.get('in_shapes_nd') or [None])[0]
        shp_out = op.get('out_shape_nd')
        if (key == 'scale' and shp_in is not None and len(shp_in) == 3
                and int(shp_in[0]) == k and k * int(shp_in[1]) * int(shp_in[2]) == n):
            t = t.repeat_interleave(int(shp_in[1]) * int(shp_in[2]))
        elif shp_out is not None and len(shp_out) >= 1 and int(shp_out[-1]) == k and n % k == 0:
            t = t.repeat(n // k)
        else:
            raise ValueError(f'{op["type"]} {op["name"]!r}: {key} of {k} values does not '
                             f'broadcast to {n}')
    t = t.to(device).contiguous()
    op['_vc_amd_' + key] = ((str(device), n), t)
    return t


def _fork_points(gg):
    """The names consumed by more than one op (the gg's 'fork_points',
    network.py:1713; derived from the ops when the dict has none)."""
    fp = gg.get('fork_points')
    if fp is not None:
        return fp
    uses = {}
    for op in gg['ops']:
        for i in op['inputs']:
            uses[i] = uses.get(i, 0) + 1
    return {k for k, v in uses.items() if v > 1}


def _shared_gens(name_a, name_b, gg, gen_count):
    """Generator columns two merging branches share: the count at the first
    fork point among name_a's ancestors (depth-first from name_a, inputs
    pushed in order) that is also an ancestor of name_b, else at the input.
    The reference's _find_shared_gens_count (verify_zono_bnb.py:2387-2428);
    column k of every descendant of a fork is that fork's k-th noise."""
    forks = _fork_points(gg)
    pred = {op['name']: op['inputs'] for op in gg['ops']}

    def ancestors(name):
        order, stack, seen = [], [name], set()
        while stack:
            x = stack.pop()
            if x in seen:
                continue
            seen.add(x)
            order.append(x)
            stack.extend(pred.get(x, ()))
        return order

    anc_b = set(ancestors(name_b))
    for a in ancestors(name_a):
        if a in anc_b and a in forks:
            return gen_count.get(a, 0)
    return gen_count.get(gg['input_name'], 0)


# --------------------------------------------------------------------------
# a1: ReLU relaxation
# --------------------------------------------------------------------------

def _make_slopes(lo, hi):
    """CROWN adaptive slopes (verify_zono_bnb.py:503-522).

    Returns (lo_s, up_s, up_t, active, dead, unstable) like the reference.
    """
    lo, hi = f32(lo), f32(hi)
    if lo.shape != hi.shape:
        raise ValueError('lo/hi shape mismatch')
    outs = [torch.empty_like(lo) for _ in range(3)]
    masks = [torch.empty(lo.shape, dtype=torch.bool, device=lo.device)
             for _ in range(3)]
    call('vc_make_slopes', ptr(lo), ptr(hi), lo.numel(),
         *[ptr(t) for t in outs], *[ptr(t) for t in masks], stream())
    return (*outs, *masks)


# --------------------------------------------------------------------------
# a2: IBP forward
# --------------------------------------------------------------------------

def _ibp_forward_graph_batched(xl, xh, gg, device, dtype, relu_clamps=None,
                               root_sb=None):
    """Batched interval forward (verify_zono_bnb.py:1066-1153).

    Returns {layer_idx: (lo, hi)} of (B, n_L) pre-activation bounds after
    root intersection, split clamps and crossing repair.
    """
    _check_dtype(dtype)
    xl, xh = f32(xl), f32(xh)
    B = xl.shape[0]
    dev = xl.device
    widths = _widths(gg, xl.shape[1])
    lo = {gg['input_name']: xl}
    hi = {gg['input_name']: xh}
    sb = {}
    st = stream()
    for op in gg['ops']:
        t = op['type']
        name = op['name']
        l, h = lo[op['inputs'][0]], hi[op['inputs'][0]]
        if t == 'fc':
            if _fc_form(op, widths[op['inputs'][0]])[0] > 1:
                # the reference's interval fc is mid @ W.T (verify_zono_bnb.py:
                # 1108-1113), which has no N-D MatMul form
                raise NotImplementedError(
                    f'_ibp_forward_graph_batched: fc {name!r} is an N-D batched MatMul, '
                    f'which the interval forward does not take')
            p = _op_params(op, dev)
            lo_o = torch.empty(B, p['n_out'], device=dev)
            hi_o = torch.empty_like(lo_o)
            call('vc_ibp_fc', ptr(l), ptr(h), B, p['n_in'], ptr(p['W']),
                 ptr(p['b']), p['n_out'], ptr(lo_o), ptr(hi_o), st)
            lo[name], hi[name] = lo_o, hi_o
        elif t == 'conv':
            p = _op_params(op, dev)
            C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, Ho, Wo = p['geom']
            lo_o = torch.empty(B, p['n_out'], device=dev)
            hi_o = torch.empty_like(lo_o)
            call('vc_ibp_conv', ptr(l), ptr(h), B, C_in, H, W, ptr(p['K']),
                 ptr(p['b']), C_out, kh, kw, sh, sw, ph, pw, Ho, Wo,
                 ptr(lo_o), ptr(hi_o), st)
            lo[name], hi[name] = lo_o, hi_o
        elif t == 'relu':
            L = op.get('layer_idx')
            n = l.shape[1]
            rlo = rhi = cl = ch = None
            if L is not None and root_sb is not None and L in root_sb:
                rlo = f32(root_sb[L][0]).reshape(-1)
                rhi = f32(root_sb[L][1]).reshape(-1)
            if L is not None and relu_clamps is not None and L in relu_clamps:
                cl = f32(relu_clamps[L][0])
                ch = f32(relu_clamps[L][1])
            sl = torch.empty_like(l)
            sh_ = torch.empty_like(l)
            pl = torch.empty_like(l)
            ph_ = torch.empty_like(l)
            call('vc_ibp_relu', ptr(l), ptr(h), B, n, ptr(rlo), ptr(rhi),
                 ptr(cl), ptr(ch), ptr(sl), ptr(sh_), ptr(pl), ptr(ph_), st)
            if L is not None:
                sb[L] = (sl, sh_)
            lo[name], hi[name] = pl, ph_
        elif t == 'reshape':
            lo[name], hi[name] = l, h
        elif t == 'add' and op.get('is_merge'):
            # residual merge (verify_zono_bnb.py:1133-1135)
            l2, h2 = lo[op['inputs'][1]], hi[op['inputs'][1]]
            lo_o, hi_o = torch.empty_like(l), torch.empty_like(h)
            call('vc_add_ew', ptr(l), ptr(l2), l.numel(), ptr(lo_o), st)
            call('vc_add_ew', ptr(h), ptr(h2), h.numel(), ptr(hi_o), st)
            lo[name], hi[name] = lo_o, hi_o
        elif t in ('add', 'sub'):
            # constant shift (verify_zono_bnb.py:1136-1143)
            n = l.shape[1]
            b = _op_const(op, 'bias', dev, n)
            if b is None:
                raise ValueError(f'{t} {name!r}: no constant')
            mode = 0 if t == 'add' else 1
            lo_o, hi_o = torch.empty_like(l), torch.empty_like(h)
            call('vc_affine_ew', ptr(l), B, n, 1, ptr(b), b.numel(), mode, ptr(lo_o), st)
            call('vc_affine_ew', ptr(h), B, n, 1, ptr(b), b.numel(), mode, ptr(hi_o), st)
            lo[name], hi[name] = lo_o, hi_o
        elif t == 'mul':
            # constant scale (verify_zono_bnb.py:1144-1148)
            n = l.shape[1]
            s = _op_const(op, 'scale', dev, n)
            if s is None:
                raise ValueError(f'mul {name!r}: no scale')
            lo_o, hi_o = torch.empty_like(l), torch.empty_like(h)
            call('vc_interval_mul', ptr(l), ptr(h), B, n, ptr(s), s.numel(), ptr(lo_o),
                 ptr(hi_o), st)
            lo[name], hi[name] = lo_o, hi_o
        else:
            raise NotImplementedError(
                f'_ibp_forward_graph_batched: unsupported op {t!r} at '
                f'{name!r} -- silently skipping would certify unsound bounds')
    return sb


# --------------------------------------------------------------------------
# a3: zonotope forward
# --------------------------------------------------------------------------

def _forward_zonotope_graph_batched(xl, xh, gg, device, dtype):
    """Batched zonotope forward (verify_zono_bnb.py:3079-4075, fc/relu/conv/
    reshape/add/sub/mul).  Returns (sb, (c, G)); G is (B, n, K) with the new
    generator columns of each ReLU padded to the batch maximum, as in the
    reference; a residual merge sums the generator columns the two branches
    share from their fork point and appends each branch's own.
    (The (c, G) output needs the layer-wise kernels; bound-only callers use
    the fused kernel through _zono_sb.)
    """
    _check_dtype(dtype)
    xl, xh = f32(xl), f32(xh)
    B, n_in = xl.shape
    dev = xl.device
    st = stream()
    widths = _widths(gg, n_in)
    varying = ((xh - xl) / 2).abs().amax(dim=0) > 0 if B > 0 else \
        torch.zeros(n_in, dtype=torch.bool, device=dev)
    vidx = varying.nonzero(as_tuple=True)[0].to(torch.int32).contiguous()
    K = int(vidx.numel())
    c = torch.empty(B, n_in, device=dev)
    G = torch.empty(B, n_in, K, device=dev)
    call('vc_zono_input', ptr(xl), ptr(xh), B, n_in, ptr(vidx), K, ptr(c),
         ptr(G), st)
    state = {gg['input_name']: (c, G)}
    gen_count = {gg['input_name']: K}
    sb = {}
    for op in gg['ops']:
        t = op['type']
        name = op['name']
        c_in, G_in = state[op['inputs'][0]]
        Kc = G_in.shape[2]
        n = c_in.shape[1]
        if t == 'add' and op.get('is_merge'):
            # residual merge: the fork point's generators are shared
            # (verify_zono_bnb.py:3213-3234)
            c_b, G_b = state[op['inputs'][1]]
            Kb = G_b.shape[2]
            shared = _shared_gens(op['inputs'][0], op['inputs'][1], gg, gen_count)
            if not (0 <= shared <= Kc and shared <= Kb):
                raise ValueError(f'add {name!r}: {shared} shared generators of {Kc} and {Kb}')
            c_o = torch.empty_like(c_in)
            call('vc_add_ew', ptr(c_in), ptr(c_b), c_in.numel(), ptr(c_o), st)
            G_o = torch.empty(B, n, Kc + Kb - shared, device=dev)
            call('vc_zono_merge', ptr(G_in), Kc, ptr(G_b), Kb, shared, B * n, ptr(G_o), st)
            state[name] = (c_o, G_o)
        elif t in ('add', 'sub'):
            # constant shift of the centre (verify_zono_bnb.py:3235-3265)
            b = _op_const(op, 'bias', dev, n)
            c_o = c_in
            if b is not None:
                c_o = torch.empty_like(c_in)
                call('vc_affine_ew', ptr(c_in), B, n, 1, ptr(b), b.numel(),
                     0 if t == 'add' else 1, ptr(c_o), st)
            state[name] = (c_o, G_in)
        elif t == 'mul':
            # constant scale of centre and generators (verify_zono_bnb.py:3501-3536)
            s = _op_const(op, 'scale', dev, n)
            if s is None:
                raise ValueError(f'mul {name!r}: no scale')
            c_o = torch.empty_like(c_in)
            call('vc_affine_ew', ptr(c_in), B, n, 1, ptr(s), s.numel(), 2, ptr(c_o), st)
            G_o = torch.empty_like(G_in)
            if Kc > 0:
                call('vc_affine_ew', ptr(G_in), B, n, Kc, ptr(s), s.numel(), 2, ptr(G_o), st)
            state[name] = (c_o, G_o)
        elif t == 'fc':
            p = _op_params(op, dev)
            # the N-D MatMul form (verify_zono_bnb.py:3145-3168) applies W to
            # each of P slices: (B, P * n_in) centres and (B, P * n_in, K)
            # generators are (B * P, n_in) and (B * P, n_in, K) as they lie
            P, _ = _fc_form(op, widths[op['inputs'][0]])
            c_o = torch.empty(B, P * p['n_out'], device=dev)
            G_o = torch.empty(B, P * p['n_out'], Kc, device=dev)
            call('vc_zono_fc', ptr(c_in), ptr(G_in), B * P, p['n_in'], Kc,
                 ptr(p['W']), ptr(p['b']), p['n_out'], ptr(c_o), ptr(G_o), st)
            state[name] = (c_o, G_o)
        elif t == 'conv':
            p = _op_params(op, dev)
            C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, Ho, Wo = p['geom']
            c_o = torch.empty(B, p['n_out'], device=dev)
            G_o = torch.empty(B, p['n_out'], Kc, device=dev)
            call('vc_zono_conv', ptr(c_in), ptr(G_in), B, Kc, C_in, H, W,
                 ptr(p['K']), ptr(p['b']), C_out, kh, kw, sh, sw, ph, pw, Ho,
                 Wo, ptr(c_o), ptr(G_o), st)
            state[name] = (c_o, G_o)
        elif t == 'relu':
            n = c_in.shape[1]
            lo = torch.empty(B, n, device=dev)
            hi = torch.empty_like(lo)
            rank = torch.empty(B, n, dtype=torch.int32, device=dev)
            cnt = torch.empty(B, dtype=torch.int32, device=dev)
            call('vc_zono_relu_bounds', ptr(c_in), ptr(G_in), B, n, Kc,
                 ptr(lo), ptr(hi), ptr(rank), ptr(cnt), st)
            k_new = int(cnt.max().item()) if B > 0 else 0
            c_o = torch.empty(B, n, device=dev)
            G_o = torch.empty(B, n, Kc + k_new, device=dev)
            call('vc_zono_relu_apply', ptr(c_in), ptr(G_in), ptr(lo), ptr(hi),
                 ptr(rank), B, n, Kc, k_new, ptr(c_o), ptr(G_o), st)
            state[name] = (c_o, G_o)
            if 'layer_idx' in op:
                sb[op['layer_idx']] = (lo, hi)
        elif t == 'reshape':
            state[name] = (c_in, G_in)
        else:
            raise ValueError(f'batched zono forward: unknown op type {t!r}')
        gen_count[name] = state[name][1].shape[2]
    _forward_zonotope_graph_batched.last_bilinear_op_bounds = {}
    return sb, state[gg['ops'][-1]['name']]


# --------------------------------------------------------------------------
# a5-a8: CROWN backward + concretization
# --------------------------------------------------------------------------

class _Rows:
    """Backward coefficient rows at one graph node.

    ``ew`` is (R, n) when ``shared`` (identical for every domain, before the
    first per-domain relaxation) else (B*R, n).  ``relu`` names a relu layer
    whose relaxation is still to be applied (it is fused into the next fc).
    ``alpha``/``beta`` belong to that pending relu; ``alpha_group`` (B,)
    int64 makes ``alpha`` (G*R, n) the rows of each domain's group.
    """
    __slots__ = ('ew', 'shared', 'relu', 'alpha', 'alpha_row', 'beta', 'alpha_group',
                 'n_groups')

    def __init__(self, ew, shared):
        self.ew = ew
        self.shared = shared
        self.relu = None
        self.alpha = None
        self.alpha_row = 0
        self.beta = None
        self.alpha_group = None
        self.n_groups = 0


class BackwardTrace:
    """Per-relu stored pre-relaxation rows of one backward, for the alpha
    gradient sweep: entries (L, P, p_shared) in backward order.  ``other``
    names an op the sweep does not replay (add, sub, mul, a fan-in)."""

    def __init__(self):
        self.relus = []
        self.fcs = []
        self.other = None


# vc_backward_fc runs as relaxation pass + plain MFMA GEMM from this row
# width up when given a relaxed-rows buffer (measured 2x faster on 1024-wide
# layers than relaxing inside the GEMM's loads).
_TWO_PHASE_MIN_WIDTH = 64


def _expand_rows(t, B):
    """(R, n) shared rows -> (B*R, n) per-domain rows."""
    R, n = t.shape
    return t.unsqueeze(0).expand(B, R, n).reshape(B * R, n).contiguous()


def _backward(tight, xl, xh, gg, seed_name, seed, seed_shared, acc0,
              alpha_at_layer=None, relu_split_beta=None, trace=None):
    """Walk the ops backward from ``seed_name`` and concretize.

    seed: (R, n) rows when ``seed_shared`` else (B*R, n); acc0: (R,) when
    shared else (B*R,).  Returns (lb (B, R), A, a_shared, acc (B*R,)).
    """
    B, n_in = xl.shape
    dev = xl.device
    st = stream()
    widths = _widths(gg, n_in)
    R = seed.shape[0] if seed_shared else seed.shape[0] // max(B, 1)
    acc = acc0.clone()
    acc_shared = seed_shared
    ew_at = {seed_name: _Rows(seed, seed_shared)}
    ops = gg['ops']

    def per_domain_acc():
        nonlocal acc, acc_shared
        if acc_shared:
            acc = acc.unsqueeze(0).expand(B, R).reshape(B * R).contiguous()
            acc_shared = False

    def combine(a, b):
        """Rows reaching one node from two consumers, summed (ew_at[inp] +
        ew, verify_zono_bnb.py:4462-4469)."""
        a, b = materialize(a), materialize(b)
        if a.shared and b.shared:
            out = torch.empty_like(a.ew)
            call('vc_add_ew', ptr(a.ew), ptr(b.ew), a.ew.numel(), ptr(out), st)
            return _Rows(out, True)
        per_domain_acc()
        ea = _expand_rows(a.ew, B) if a.shared else a.ew
        eb = _expand_rows(b.ew, B) if b.shared else b.ew
        out = torch.empty_like(ea)
        call('vc_add_ew', ptr(ea), ptr(eb), ea.numel(), ptr(out), st)
        return _Rows(out, False)

    def put(inp, rows):
        prev = ew_at.get(inp)
        if prev is not None and trace is not None:
            trace.other = trace.other or 'fan-in'
        ew_at[inp] = rows if prev is None else combine(prev, rows)

    def bias_dot(rows, v, sign):
        """acc += sign * rows . v (the constant of an add or sub)."""
        n = rows.ew.shape[1]
        if rows.shared and acc_shared:
            call('vc_rows_bias_dot', ptr(rows.ew), R, R, n, 1, ptr(v), v.numel(), sign,
                 ptr(acc), st)
        else:
            per_domain_acc()
            call('vc_rows_bias_dot', ptr(rows.ew), B * R, R, n, 1 if rows.shared else 0,
                 ptr(v), v.numel(), sign, ptr(acc), st)

    def materialize(rows):
        """Apply a pending relu relaxation with the standalone kernel."""
        if rows.relu is None:
            return rows
        if rows.alpha_group is not None:
            raise NotImplementedError(
                'vibecheck_amd: group-indexed alpha is supported before an fc only')
        L = rows.relu
        lo, hi = tight[L]
        lo, hi = f32(lo), f32(hi)
        n = lo.shape[1]
        ew = _expand_rows(rows.ew, B) if rows.shared else rows.ew
        per_domain_acc()
        if trace is not None:
            trace.relus.append((L, rows.ew, rows.shared))
        out = torch.empty(B * R, n, device=dev)
        call('vc_backward_relu', ptr(ew), B * R, R, n, ptr(lo), ptr(hi),
             ptr(rows.alpha), rows.alpha_row, ptr(rows.beta), ptr(out),
             ptr(acc), st)
        return _Rows(out, False)

    def relu_conv(rows, op, p):
        """The pending relu relaxation fused into the conv backward that
        follows it (vc_backward_relu_conv), or None when the geometry or
        the relaxation's form is outside the fused kernel."""
        if rows.alpha_group is not None or (rows.alpha is not None and rows.alpha_row):
            return None
        ok = p.get('relu_conv_ok')
        if ok is None:
            C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, Ho, Wo = p['geom']
            ok = bool(_lib.load().vc_backward_relu_conv_ok(C_out, Ho, Wo, C_in, H, W, kh, kw,
                                                           sh, sw, ph, pw))
            p['relu_conv_ok'] = ok
        if not ok:
            return None
        L = rows.relu
        lo, hi = f32(tight[L][0]), f32(tight[L][1])
        n = lo.shape[1]
        per_domain_acc()
        if trace is not None:
            trace.relus.append((L, rows.ew, rows.shared))
        ls, us, ut = (torch.empty(B, n, device=dev) for _ in range(3))
        call('vc_relax_slopes', ptr(lo), ptr(hi), ptr(rows.alpha), B * n, ptr(ls), ptr(us),
             ptr(ut), st)
        C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, Ho, Wo = p['geom']
        out = torch.empty(B * R, p['n_in'], device=dev)
        call('vc_backward_relu_conv', ptr(rows.ew), B * R, R, 1 if rows.shared else 0, ptr(ls),
             ptr(us), ptr(ut), ptr(rows.beta), ptr(p['K']), ptr(p['b']), C_out, Ho, Wo, C_in,
             H, W, kh, kw, sh, sw, ph, pw, ptr(out), ptr(acc), st)
        return out

    for op in reversed(ops):
        name = op['name']
        if name not in ew_at:
            continue
        rows = ew_at.pop(name)
        t = op['type']
        inp = op['inputs'][0]
        if t in ('add', 'sub', 'mul') and trace is not None:
            trace.other = trace.other or t
        if t == 'add' and op.get('is_merge'):
            # the rows flow to both branches unchanged (verify_zono_bnb.py:4462-4469)
            rows = materialize(rows)
            for i in op['inputs']:
                put(i, _Rows(rows.ew, rows.shared))
        elif t in ('add', 'sub'):
            # constant shift: acc +/-= rows . bias, rows unchanged
            # (verify_zono_bnb.py:4470-4518)
            rows = materialize(rows)
            b = _op_const(op, 'bias', dev, rows.ew.shape[1])
            if b is not None:
                bias_dot(rows, b, 1.0 if t == 'add' else -1.0)
            put(inp, rows)
        elif t == 'mul':
            # constant scale: rows * scale (verify_zono_bnb.py:4686-4712)
            rows = materialize(rows)
            s = _op_const(op, 'scale', dev, rows.ew.shape[1])
            if s is None:
                raise ValueError(f'mul {name!r}: no scale')
            out = torch.empty_like(rows.ew)
            call('vc_affine_ew', ptr(rows.ew), rows.ew.shape[0], rows.ew.shape[1], 1, ptr(s),
                 s.numel(), 2, ptr(out), st)
            put(inp, _Rows(out, rows.shared))
        elif t == 'fc' and _fc_form(op, widths[inp])[0] > 1:
            # N-D batched MatMul (verify_zono_bnb.py:4382-4401): acc += the
            # rows . bias repeated over the P slices, then each row's P
            # slices of n_out times W, as (M * P, n_out) rows
            P, nd_out = _fc_form(op, widths[inp])
            if not nd_out:
                raise NotImplementedError(
                    f'batched spec backward: fc {name!r} is an N-D batched MatMul '
                    f'without out_shape_nd')
            if trace is not None:
                trace.other = trace.other or 'N-D fc'
            p = _op_params(op, dev)
            rows = materialize(rows)
            if p['b'] is not None:
                key = ('b_rep', P)
                if key not in p:
                    p[key] = p['b'].repeat(P).contiguous()
                bias_dot(rows, p[key], 1.0)
            M = rows.ew.shape[0]
            out = torch.empty(M, P * p['n_in'], device=dev)
            call('vc_backward_fc', ptr(rows.ew), M * P, R * P, p['n_out'], None,
                 None, None, 0, None, ptr(p['W']), None, p['n_in'], ptr(out), None,
                 None, 0, st)
            put(inp, _Rows(out, rows.shared))
        elif t == 'fc':
            p = _op_params(op, dev)
            if rows.relu is not None:
                L = rows.relu
                lo, hi = f32(tight[L][0]), f32(tight[L][1])
                per_domain_acc()
                M = B * R
                out = torch.empty(M, p['n_in'], device=dev)
                if trace is not None:
                    trace.relus.append((L, rows.ew, rows.shared))
                    trace.fcs.append(op)
                # the relaxed rows buffer selects the library's two-phase
                # step (relaxation streamed through HBM, then a plain GEMM)
                rel = (torch.empty(M, p['n_out'], device=dev)
                       if p['n_out'] >= _TWO_PHASE_MIN_WIDTH else None)
                if rows.alpha_group is not None:
                    if rows.beta is not None:
                        raise NotImplementedError(
                            'vibecheck_amd: group-indexed alpha takes no beta')
                    call('vc_backward_fc_grouped', ptr(rows.ew), M, R, p['n_out'],
                         ptr(lo), ptr(hi), ptr(rows.alpha), ptr(rows.alpha_group),
                         rows.n_groups, ptr(p['W']), ptr(p['b']), p['n_in'], ptr(out), ptr(acc),
                         ptr(rel), 1 if rows.shared else 0, st)
                else:
                    call('vc_backward_fc', ptr(rows.ew), M, R, p['n_out'],
                         ptr(lo), ptr(hi), ptr(rows.alpha), rows.alpha_row,
                         ptr(rows.beta), ptr(p['W']), ptr(p['b']), p['n_in'],
                         ptr(out), ptr(acc), ptr(rel), 1 if rows.shared else 0, st)
                del rel
                put(inp, _Rows(out, False))
            else:
                if not rows.shared:
                    per_domain_acc()
                M = R if rows.shared else B * R
                out = torch.empty(M, p['n_in'], device=dev)
                if trace is not None:
                    trace.fcs.append(op)
                call('vc_backward_fc', ptr(rows.ew), M, R, p['n_out'], None,
                     None, None, 0, None, ptr(p['W']), ptr(p['b']),
                     p['n_in'], ptr(out), ptr(acc), None, 0, st)
                put(inp, _Rows(out, rows.shared))
        elif t == 'relu':
            if 'layer_idx' in op:
                rows = materialize(rows)
                L = op['layer_idx']
                rows.relu = L
                if alpha_at_layer is not None and L in alpha_at_layer:
                    a = alpha_at_layer[L]
                    if isinstance(a, tuple):
                        # (alpha of each group (G, R, n), group of each domain (B,))
                        rows.alpha = f32(a[0]).reshape(-1, a[0].shape[-1])
                        rows.alpha_row = 0
                        rows.alpha_group = a[1]
                        rows.n_groups = int(a[0].shape[0])
                        a = None
                    else:
                        a = f32(a)
                    if a is None:
                        pass
                    elif a.dim() == 3:
                        rows.alpha = a.reshape(B * R, -1)
                        rows.alpha_row = 1
                    else:
                        rows.alpha = a
                        rows.alpha_row = 0
                if relu_split_beta is not None and L in relu_split_beta:
                    rows.beta = f32(relu_split_beta[L])
            put(inp, rows)
        elif t == 'conv':
            p = _op_params(op, dev)
            if rows.relu is not None and FUSED_RELU_CONV:
                out = relu_conv(rows, op, p)
                if out is not None:
                    put(inp, _Rows(out, False))
                    continue
            rows = materialize(rows)
            C_in, H, W, C_out, kh, kw, sh, sw, ph, pw, Ho, Wo = p['geom']
            if not rows.shared:
                per_domain_acc()
            M = R if rows.shared else B * R
            out = torch.empty(M, p['n_in'], device=dev)
            call('vc_backward_conv_packed', ptr(rows.ew), M, ptr(p['K']),
                 ptr(_conv_t_taps(p, st)), ptr(p['b']), C_out, Ho, Wo, C_in, H, W,
                 kh, kw, sh, sw, ph, pw, ptr(out), ptr(acc), st)
            put(inp, _Rows(out, rows.shared))
        elif t == 'reshape':
            put(inp, rows)
        else:
            raise ValueError(f'batched spec backward: unknown op {t!r}')

    rows = ew_at.get(gg['input_name'])
    if rows is None:
        per_domain_acc()
        return acc.reshape(B, R).clone(), None, False, acc
    rows = materialize(rows)
    A = rows.ew
    per_domain_acc()
    lb = torch.empty(B * R, device=dev)
    call('vc_concretize', ptr(A), ptr(acc), ptr(xl), ptr(xh), B * R, R, n_in,
         1 if rows.shared else 0, ptr(lb), st)
    return lb.reshape(B, R), A, rows.shared, acc


_SPEC_CACHE = {}


def _spec_rows(spec_ew, dev):
    """The spec rows stacked (Q, n_out) and their offsets (Q,) on ``dev``.
    Cached for tensor rows (keyed on each tensor's identity and in-place
    version): building them copies the offsets from the host, which would
    stall the stream once per bound call.  Callers only read the result."""
    qids = sorted(spec_ew.keys())
    key = None
    if all(torch.is_tensor(spec_ew[q][0]) and not torch.is_tensor(spec_ew[q][1])
           for q in qids):
        key = (str(dev), tuple((q, id(spec_ew[q][0]), spec_ew[q][0]._version,
                                float(spec_ew[q][1])) for q in qids))
        hit = _SPEC_CACHE.get(key)
        if hit is not None:
            return hit[1], hit[2]
    Wq = torch.stack([torch.as_tensor(spec_ew[q][0]).reshape(-1)
                      .to(device=dev, dtype=torch.float32) for q in qids]).contiguous()
    bq = torch.tensor([float(spec_ew[q][1]) for q in qids],
                      dtype=torch.float32, device=dev)
    if key is not None:
        if len(_SPEC_CACHE) >= 32:
            _SPEC_CACHE.pop(next(iter(_SPEC_CACHE)))
        # the rows are held so that their identities stay unique
        _SPEC_CACHE[key] = ([spec_ew[q][0] for q in qids], Wq, bq)
    return Wq, bq


def _spec_backward_graph_batched(tight, xl, xh, gg, spec_ew, device, dtype,
                                 return_input_linear=False,
                                 alpha_at_layer=None, relu_split_beta=None,
                                 alpha_mccormick=None, alpha_recip=None,
                                 bilinear_op_bounds=None, seed_ew_at=None,
                                 seed_acc=None):
    """Batched CROWN spec backward + concretization
    (verify_zono_bnb.py:4270-5134; fc/relu/conv/reshape ops).

    Returns lb (B, Q), or (lb, A (B, Q, n_in), acc (B, Q)) with
    ``return_input_linear``.
    """
    _check_dtype(dtype)
    if alpha_mccormick or alpha_recip or bilinear_op_bounds:
        raise NotImplementedError(
            'vibecheck_amd: bilinear / reciprocal relaxations are not '
            'supported (Linear/Conv/ReLU networks only)')
    xl, xh = f32(xl), f32(xh)
    _widths(gg, xl.shape[1])
    B, n_in = xl.shape
    dev = xl.device
    plan = _plan(gg, dev)
    if (plan is not None and seed_ew_at is None and alpha_at_layer is None
            and relu_split_beta is None and len(spec_ew) <= 32):
        Wq, bq = _spec_rows(spec_ew, dev)
        sb = {L: (f32(tight[L][0]), f32(tight[L][1])) for L in range(plan.n)}
        _, lb, A, acc = mlp_fused.crown(plan, xl, xh, sb, False, spec=(Wq, bq),
                                        want_linear=return_input_linear)
        return (lb, A, acc) if return_input_linear else lb
    if seed_ew_at is not None:
        if len(seed_ew_at) != 1:
            raise NotImplementedError('vibecheck_amd: one seed node only')
        seed_name, seed = next(iter(seed_ew_at.items()))
        Q = seed.shape[1]
        if seed.dim() == 3 and seed.stride(0) == 0:
            rows, shared = f32(seed[0]).contiguous(), True
        else:
            rows, shared = f32(seed).reshape(B * Q, -1).contiguous(), False
        if seed_acc is None:
            acc0 = torch.zeros(Q if shared else B * Q, device=dev)
        else:
            sa = f32(seed_acc)
            if shared and sa.stride(0) == 0:
                acc0 = sa[0].contiguous().clone()
            else:
                if shared:
                    rows, shared = _expand_rows(rows, B), False
                acc0 = sa.reshape(B * Q).contiguous().clone()
    else:
        rows, acc0 = _spec_rows(spec_ew, dev)
        seed_name, shared = gg['ops'][-1]['name'], True
        Q = rows.shape[0]
    lb, A, a_shared, acc = _backward(tight, xl, xh, gg, seed_name, rows,
                                     shared, acc0, alpha_at_layer,
                                     relu_split_beta)
    if not return_input_linear:
        return lb
    if A is None:
        return lb, torch.zeros(B, Q, n_in, device=dev), acc.reshape(B, Q)
    if a_shared:
        A = A.unsqueeze(0).expand(B, Q, n_in).contiguous()
    else:
        A = A.reshape(B, Q, n_in)
    return lb, A, acc.reshape(B, Q)


# --------------------------------------------------------------------------
# a4: CROWN intermediate bounds
# --------------------------------------------------------------------------

def _crown_intermediate_batched(gg, xl, xh, device, dtype, chunk=2048,
                                sb=None):
    """Backward-CROWN intermediate pre-ReLU bounds
    (verify_zono_bnb.py:4077-4147).

    For each ReLU layer L in ascending order: seed [+I; -I] at L's input for
    the neurons unstable in ANY domain of the batch, in chunks of ``chunk``,
    propagate through the already-tightened earlier layers and intersect.
    The seeded rows are identical for every domain until the first ReLU, so
    that prefix is computed once (R rows) and broadcast.  ``sb`` (extension)
    replaces the zonotope starting bounds, e.g. by IBP bounds.
    """
    _check_dtype(dtype)
    xl, xh = f32(xl), f32(xh)
    _widths(gg, xl.shape[1])
    dev = xl.device
    if sb is None:
        sb = _zono_sb(gg, xl, xh, device, dtype)
    plan = _plan(gg, dev)
    if plan is not None:
        tight, _, _, _ = mlp_fused.crown(
            plan, xl, xh, {L: (f32(sb[L][0]), f32(sb[L][1])) for L in range(plan.n)}, True)
        return tight
    tight = {L: (f32(lo).clone(), f32(hi).clone()) for L, (lo, hi) in sb.items()}
    relu_by_L = {op['layer_idx']: op for op in gg['ops']
                 if op['type'] == 'relu' and 'layer_idx' in op}
    B = xl.shape[0]
    st = stream()
    ch = max(1, int(chunk))
    for L in sorted(tight):
        if L not in relu_by_L:
            continue
        feed = relu_by_L[L]['inputs'][0]
        lo_L, hi_L = tight[L]
        n = lo_L.shape[1]
        flag = torch.empty(n, dtype=torch.uint8, device=dev)
        call('vc_unstable_union', ptr(lo_L), ptr(hi_L), B, n, ptr(flag), st)
        idx = flag.nonzero(as_tuple=True)[0].to(torch.int32)
        m = int(idx.numel())
        if m == 0:
            continue
        new_lo, new_hi = lo_L.clone(), hi_L.clone()
        for c0 in range(0, m, ch):
            cidx = idx[c0:c0 + ch].contiguous()
            k = int(cidx.numel())
            seed = torch.zeros(2 * k, n, device=dev)
            ar = torch.arange(k, device=dev)
            seed[ar, cidx.long()] = 1.0
            seed[ar + k, cidx.long()] = -1.0
            acc0 = torch.zeros(2 * k, device=dev)
            sl, _, _, _ = _backward(tight, xl, xh, gg, feed, seed, True, acc0)
            sl = sl.contiguous()
            call('vc_crown_intersect', ptr(sl), ptr(cidx), k, B, n,
                 ptr(new_lo), ptr(new_hi), st)
        tight[L] = (new_lo, new_hi)
    return tight


# --------------------------------------------------------------------------
# a9: alpha-CROWN
# --------------------------------------------------------------------------

def _alpha_backward_and_grad(sb, xl, xh, gg, Wq, bq, alpha, want_grad, galpha,
                             beta=None, gbeta=None, seed_name=None, want_A=False):
    """One alpha-CROWN evaluation: lb (B, Q); when ``want_grad`` also fills
    ``galpha[L]`` with d(sum lb)/d alpha_L (the autograd of the reference's
    backward, torch clamp subgradients included).  ``beta`` is the signed
    ReLU-split beta {L: (B, n_L)} added at each relu's input
    (``relu_split_beta``); ``gbeta[L]`` receives d(sum lb)/d beta_L.
    ``seed_name`` (default: the output op) is the op whose output the Q
    shared rows Wq (Q, n) seed, as ``seed_ew_at`` does; an alpha_L of shape
    (B, Q, n_L) is one alpha per row (per-query alpha), and galpha_L then
    has that shape too.  ``want_A``: returns (lb, A) with A (B*Q, n_in) the
    input linearization of the rows."""
    B, n_in = xl.shape
    Q = Wq.shape[0]
    dev = xl.device
    st = stream()
    trace = BackwardTrace() if want_grad else None
    seed = gg['ops'][-1]['name'] if seed_name is None else seed_name
    lb, A, a_shared, _ = _backward(sb, xl, xh, gg, seed, Wq,
                                   True, bq, alpha, beta, trace)
    if want_A and (A is None or a_shared):
        raise NotImplementedError('vibecheck_amd: per-row linearization needs a relu')
    if not want_grad:
        return (lb, A) if want_A else lb
    if A is None or a_shared:
        raise NotImplementedError('vibecheck_amd: alpha gradient needs a relu')
    if trace.other is not None:
        raise NotImplementedError(
            f'vibecheck_amd: alpha-CROWN gradient supports fc/relu chains (found {trace.other})')
    # trace.relus: (L, P, shared) in backward order (top relu first);
    # trace.fcs: fc ops in backward order.  Sequential fc/relu nets only:
    # fcs[i] sits below relus[i-1] ... check the chain shape.
    relus = trace.relus
    fcs = trace.fcs
    if len(fcs) != len(relus) + 1:
        raise NotImplementedError(
            'vibecheck_amd: alpha-CROWN gradient supports fc/relu chains')
    M = B * Q
    # input side: gE_0 = gA W_0^T + b_0, W_0 = fcs[-1]
    f0 = _op_params(fcs[-1], dev)
    g = torch.empty(M, f0['n_out'], device=dev)
    call('vc_alpha_grad_input', ptr(A), ptr(xl), ptr(xh), M, Q, n_in,
         ptr(f0['W']), ptr(f0['b']), f0['n_out'], ptr(g), st)
    for i in range(len(relus) - 1, -1, -1):
        L, P, p_shared = relus[i]
        lo, hi = f32(sb[L][0]), f32(sb[L][1])
        n = lo.shape[1]
        a = f32(alpha[L]) if (alpha is not None and L in alpha) else None
        per_row = a is not None and a.dim() == 3
        ga = galpha.get(L) if galpha is not None else None
        gb = gbeta.get(L) if gbeta is not None else None
        if per_row and ga is not None:
            if i == 0:  # above the input: no gradient step to fuse it into
                call('vc_alpha_grad_rows', ptr(g), ptr(P), 1 if p_shared else 0, M, Q, n,
                     ptr(lo), ptr(hi), ptr(ga), st)
            ga_rows = ga
            ga = None
        else:
            ga_rows = None
        if ga is not None or gb is not None:
            call('vc_alpha_grad_reduce', ptr(g), ptr(P), 1 if p_shared else 0,
                 B, Q, n, ptr(lo), ptr(hi), ptr(ga), ptr(gb), st)
        if i > 0 and per_row:
            fn = _op_params(fcs[i], dev)
            g2 = torch.empty(M, fn['n_out'], device=dev)
            call('vc_alpha_grad_step_rows', ptr(g), ptr(P), M, Q, n, ptr(lo), ptr(hi),
                 ptr(a.reshape(M, n)), 1 if p_shared else 0, ptr(fn['W']), ptr(fn['b']),
                 fn['n_out'], ptr(g2), ptr(ga_rows), st)
            g = g2
        elif i > 0:
            fn = _op_params(fcs[i], dev)
            g2 = torch.empty(M, fn['n_out'], device=dev)
            # slopes once per (domain, neuron), then the sweep step without
            # a per-element division
            ls, us, ut = (torch.empty(B, n, device=dev) for _ in range(3))
            call('vc_relax_slopes', ptr(lo), ptr(hi), ptr(a), B * n, ptr(ls),
                 ptr(us), ptr(ut), st)
            call('vc_alpha_grad_step_slopes', ptr(g), ptr(P), M, Q, n,
                 ptr(ls), ptr(us), ptr(ut), 1 if p_shared else 0,
                 ptr(fn['W']), ptr(fn['b']), fn['n_out'], ptr(g2), st)
            g = g2
    return (lb, A) if want_A else lb


def _run_alpha_crown_inputsplit_batched(xl, xh, gg, spec_ew, device, dtype,
                                        n_iters=10, lr=0.25, lr_decay=0.98,
                                        early_stop_eps=1e-6, sb=None,
                                        return_trace=False, lazy_trace=False):
    """Batched alpha-CROWN with Adam (verify_zono_bnb.py:5137-5288).

    Same schedule as the reference: alpha starts at (up_s > 0.5)*unstable on
    the zonotope bounds; per iteration: evaluate, keep the best lb, stop if
    every best lb > 0, Adam step (torch.optim.Adam defaults) on -sum(lb),
    clamp alpha to [0, 1], stop if the global max of the best lb improved by
    less than ``early_stop_eps`` (from the second iteration), decay lr.
    The gradient is computed analytically by the HIP gradient sweep.
    ``sb`` (extension) replaces the zonotope bounds; ``return_trace`` also
    returns the number of evaluated iterations; with ``lazy_trace`` that
    number may come as a callable, to be called after a later host
    synchronisation (it then costs no round trip of its own).
    """
    _check_dtype(dtype)
    xl, xh = f32(xl), f32(xh)
    _widths(gg, xl.shape[1])
    B = xl.shape[0]
    dev = xl.device
    st = stream()
    if sb is None:
        sb = _zono_sb(gg, xl, xh, device, dtype)
    sb = {L: (f32(lo), f32(hi)) for L, (lo, hi) in sb.items()}
    if n_iters < 1 and sb:
        # every ReLU layer is an Adam parameter, the loop body never runs:
        # no best bound (verify_zono_bnb.py:5169-5173, 5247-5288)
        return (None, 0) if return_trace else None
    Wq, bq = _spec_rows(spec_ew, dev)
    Q = Wq.shape[0]
    plan = _plan(gg, dev)
    if plan is not None and mlp_fused.alpha_supported(plan, Q):
        best, n_eval = mlp_fused.alpha_crown(plan, xl, xh, sb, Wq, bq, n_iters, lr,
                                             lr_decay, early_stop_eps, lazy=lazy_trace)
        return (best, n_eval) if return_trace else best
    Ls = sorted(sb)
    sizes = [sb[L][0].numel() for L in Ls]
    total = sum(sizes)
    if total == 0:
        lb = _alpha_backward_and_grad(sb, xl, xh, gg, Wq, bq, None, False,
                                      None)
        return (lb, 1) if return_trace else lb
    flat = torch.empty(total, device=dev)
    gflat = torch.zeros(total, device=dev)
    m1 = torch.zeros(total, device=dev)
    m2 = torch.zeros(total, device=dev)
    alpha, galpha = {}, {}
    off = 0
    for L, sz in zip(Ls, sizes):
        alpha[L] = flat[off:off + sz].view(sb[L][0].shape)
        galpha[L] = gflat[off:off + sz].view(sb[L][0].shape)
        call('vc_alpha_init', ptr(sb[L][0]), ptr(sb[L][1]), sz,
             ptr(alpha[L]), st)
        off += sz
    best = torch.empty(B, Q, device=dev)
    red = torch.empty(2, device=dev)
    b1, b2, eps = 0.9, 0.999, 1e-8
    prev_max = -float('inf')
    n_eval = 0
    step = 0
    cur_lr = float(lr)
    for it in range(n_iters):
        lb = _alpha_backward_and_grad(sb, xl, xh, gg, Wq, bq, alpha, True,
                                      galpha)
        n_eval += 1
        call('vc_best_update', ptr(best), ptr(lb.contiguous()), B * Q,
             1 if it == 0 else 0, ptr(red), st)
        r = red.tolist()
        curr_max, all_pos = r[0], r[1] > 0.5
        if all_pos:
            break
        step += 1
        bc1 = 1 - b1 ** step
        bc2 = 1 - b2 ** step
        call('vc_adam_step', ptr(flat), ptr(gflat), ptr(m1), ptr(m2), total,
             b1, b2, eps, cur_lr / bc1, bc2 ** 0.5, 0.0, 1.0, st)
        if it > 0 and curr_max - prev_max < early_stop_eps:
            break
        prev_max = curr_max
        cur_lr *= lr_decay
    if return_trace:
        return best, n_eval
    return best


def _bound_crown_spec(gg, xl, xh, spec_ew, device, dtype,
                      return_input_linear=False, return_zono_sb=False, union_seeds=False):
    """CROWN intermediate bounds followed by the spec bound -- the 'bound'
    phase of an input-split BaB iteration (verify_graph.py:12855-12871).
    For narrow fc/ReLU chains both run in one whole-network kernel launch,
    which by default seeds in each domain only the union neurons whose
    slopes depend on their bounds there: the spec bound, A and acc are
    those of the reference's union seeding, and so are the bounds of every
    neuron unstable in the domain; the bounds of the domain's stable
    neurons stay the zonotope ones (``union_seeds=True`` tightens them
    too, as _crown_intermediate_batched does).
    Returns (tight, lb) or (tight, lb, A, acc); ``return_zono_sb``
    (extension) appends the zonotope bounds the CROWN pass started from,
    which the alpha-CROWN of the same boxes starts from as well."""
    _check_dtype(dtype)
    xl, xh = f32(xl), f32(xh)
    plan = _plan(gg, xl.device)
    sb = _zono_sb(gg, xl, xh, device, dtype)
    if plan is not None and len(spec_ew) <= 32:
        Wq, bq = _spec_rows(spec_ew, xl.device)
        tight, lb, A, acc = mlp_fused.crown(plan, xl, xh, sb, True, spec=(Wq, bq),
                                            want_linear=return_input_linear,
                                            per_domain=not union_seeds)
        out = (tight, lb, A, acc) if return_input_linear else (tight, lb)
    else:
        tight = _crown_intermediate_batched(gg, xl, xh, device, dtype, sb=sb)
        res = _spec_backward_graph_batched(tight, xl, xh, gg, spec_ew, device, dtype,
                                           return_input_linear=return_input_linear)
        out = (tight,) + tuple(res) if return_input_linear else (tight, res)
    return out + (sb,) if return_zono_sb else out
