"""Benchmark: CROWN-bounded domains/s on the 5-50x6-5 ReLU MLP.

One step = three input-split BaB rounds starting from 65,536 seeded boxes
(centres U[-1,1]^5, half-widths U[0.005,0.05]): per round CROWN
intermediate bounds, CROWN spec bounds with input linearization, closure,
alpha-CROWN (20 Adam iterations, lr 0.1, decay 0.98) on every unclosed
leaf, one halfspace clip, widest-dimension bisection; the children are the
next round's batch.  value = domains bounded / wall time of the step.

Prints one JSON line.  Extra keys:
  roofline     the dominant kernel work, the CROWN pass of the 65,536-box
               round (vc_mlp_crown_rows: per ReLU layer one k_crown_rows
               launch over the packed rows plus its k_rows_cut, then
               k_spec_rows), timed with HIP events on its launch stream
               inside the timed region; traffic from the committed
               rocprofv3 counter summary of the same source;
  secondary    the step's other kernels on the step's own batches, each
               launch timed alone (zonotope bounds, small-batch CROWN, one
               alpha iteration at the open leaves and at 65,536 domains);
  alpha        alpha-CROWN's own iterations/s and domain-iterations/s;
  rounds       per round: batch, closed, alpha leaves and iterations, and the
               domains whose spec bound lies within the bound tolerance of 0;
  cpu_baseline the oracle on the same 3-round step (all host threads,
               median of 3), and round 1 of it on all 65,536 boxes at one
               thread;
  configs      the other configurations' lines (C0: 4,096 ACAS boxes, one
               BaB step; C2: 784-1024x4-10 MLP, 512 boxes, CROWN + alpha 10
               it; C3: CIFAR CNN, 64 boxes; C4: 784-256x6-10 MLP, 8,192
               ReLU-split subdomains, alpha/beta 10 it), each with its
               roofline and CPU line (--no-configs skips them).
--config c0|c2|c3|c4 prints the line of another configuration instead.
"""
import argparse
import gc
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, 'vibecheck-nn_amd')):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

N_DOMAINS = 65536
N_ROUNDS = 3
ALPHA_ITERS = 20
ALPHA_LR = 0.1
HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK = 157.3

# The CROWN pass's entry points as timed: vc_mlp_tiled_crown (also the name
# the native round files its CROWN pass under, whichever form runs) and the
# layer-synchronous form called directly.
CROWN_ENTRIES = ['vc_mlp_tiled_crown', 'vc_mlp_crown_rows']


def _seed_row(k, args):
    """The seed-counter row of the k-th timed CROWN launch: the native round
    files its row with the launch (rounds it does not time still take one);
    launches timed through the entry point take one row each, in order."""
    return args[5] if len(args) > 5 and args[5] is not None else k


def _crown_launches(kt):
    """The timed CROWN passes, in call order within each entry point (a
    workload calls one of them)."""
    return [x for n in CROWN_ENTRIES for x in kt.get(n, {}).get('per_launch', [])]


def crown_kernel_name(B):
    """The kernels that run the CROWN pass of a B-box batch."""
    from vibecheck_amd import _lib
    if _lib.load().vc_mlp_tiled_crown_mode(B) == 1:
        return 'k_crown_dom (vc_mlp_tiled_crown)'
    return ('CROWN rows pass (vc_mlp_crown_rows: k_rows_scan1/2, k_rows_write, per ReLU '
            'layer k_crown_rows + k_rows_cut, k_spec_rows; in the native round the seed '
            'masks come from the zonotope passes)')


def vz_sb(gg, xl, xh, dev):
    """The zonotope bounds of a batch (the fused kernel)."""
    from vibecheck_amd import verify_zono_bnb as vz
    return vz._zono_sb(gg, xl, xh, dev, torch.float32)


# --lookahead: how each round but the last hands the next batch's bound
# phase over (None: the driver's own setting, verify_graph.LOOKAHEAD)
LOOKAHEAD = None


def _lookahead_mode():
    from vibecheck_amd import verify_graph as vg
    m = LOOKAHEAD if LOOKAHEAD is not None else vg.LOOKAHEAD
    return {True: 'overlap', False: 'off'}.get(m, m)


def run_rounds(gg, xl, xh, spec_ew, table, timers=None, keep=None, lookahead=None):
    """Three BaB rounds; returns per-round stats.  ``keep`` (a list): each
    round's batch and step outputs are appended to it.  ``lookahead``
    (default: the driver's setting): 'tail' -- each round but the last also
    bounds the next batch after its split; 'overlap' -- while its alpha
    runs; False -- off (the same results every way)."""
    from vibecheck_amd import verify_graph as vg
    if lookahead is None:
        lookahead = LOOKAHEAD if LOOKAHEAD is not None else vg.LOOKAHEAD
    stats = []
    pre = None
    for r in range(N_ROUNDS):
        B = xl.shape[0]
        if B == 0:
            stats.append({'B': 0, 'closed': 0, 'alpha_leaves': 0, 'alpha_iters': 0})
            continue
        st = vg.bab_step(xl, xh, gg, spec_ew, table, crown_intermediate=True,
                         clip_enabled=True, alpha_iters=ALPHA_ITERS, alpha_all=True,
                         alpha_lr=ALPHA_LR, timers=timers,
                         lookahead=lookahead if r + 1 < N_ROUNDS else False, pre=pre)
        pre = st.get('lookahead')
        if keep is not None:
            keep.append((xl, xh, st))
        # next batch = the LIFO pop of [low chunk, high chunk]: high first
        # (the native round leaves them so in one block)
        if st.get('next') is not None:
            xl, xh = st['next']
        else:
            (lxl, lxh), (hxl, hxh) = st['low'], st['high']
            xl = torch.cat([hxl, lxl], 0)
            xh = torch.cat([hxh, lxh], 0)
        stats.append({'B': B, 'closed': B - int(st['unclosed'].numel()),
                      'alpha_leaves': st['n_alpha_leaves'],
                      'alpha_iters': st['n_alpha_iters']})
    return stats


def near_zero(lb, A, acc, xl, xh, rtol=1e-5, atol=1e-6):
    """Domains with a spec bound inside the bound tolerance of 0, |lb| <=
    atol + rtol * scale, scale = |acc| + sum_i |A_i| max(|xl_i|, |xh_i|): the
    domains whose verdict fp32 rounding could flip (closure is lb > 0)."""
    xm = torch.maximum(xl.abs(), xh.abs()).double()
    scale = acc.double().abs() + (A.double().abs() * xm.unsqueeze(1)).sum(-1)
    return int(((lb.double().abs() <= atol + rtol * scale).any(1)).sum())


def _events():
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def _timed(fn, reps=5):
    """Average seconds per call of fn with HIP events on the current stream
    (after one untimed call)."""
    fn()
    torch.cuda.synchronize()
    s, e = _events()
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / 1e3 / reps


def _roof(kernel, workload, sec, flop=None, nbytes=None, launches=1):
    if flop is not None:
        ach = flop / sec / 1e12
        return {'kernel': kernel, 'workload': workload, 'bound': 'mfma', 'achieved': ach,
                'peak': FP32_MFMA_PEAK, 'unit': 'TFLOP/s', 'frac': ach / FP32_MFMA_PEAK,
                'flop_per_launch': flop / launches, 'avg_launch_us': 1e6 * sec / launches}
    ach = nbytes / sec / 1e9
    return {'kernel': kernel, 'workload': workload, 'bound': 'hbm', 'achieved': ach,
            'peak': HBM_PEAK_GBS, 'unit': 'GB/s', 'frac': ach / HBM_PEAK_GBS,
            'bytes_per_launch': nbytes / launches, 'avg_launch_us': 1e6 * sec / launches}


def secondary_c1(gg, se, kept):
    """Rooflines of the step's other kernels on the step's own batches, each
    launch timed alone with HIP events (outside the timed step), plus
    alpha-CROWN's own rates: its loop on round 1's open leaves (as the step
    runs it), and on all 65,536 domains (the configuration's batch)."""
    from vibecheck_amd import _lib
    from vibecheck_amd import mlp_fused as mf
    from vibecheck_amd import verify_graph as vg
    from vibecheck_amd import verify_zono_bnb as vz
    import ctypes
    dev = torch.device('cuda:0')
    plan = mf.plan_for(gg, dev)
    dims = plan.dims
    n = plan.n
    Wq, bq = vz._spec_rows(se, dev)
    S, acc0 = mf.fold_spec(plan, Wq, bq)
    Q = S.shape[0]
    out = []
    # -- k_zono_tiled (+ the wide pass) on round 1's 65,536 boxes:
    #    sum_l 2 d_{l+1} d_l K_l per domain, K_l = 1 + n_in + unstable below l
    xl1, xh1, _ = kept[0]
    sb = vz._zono_sb(gg, xl1, xh1, dev, torch.float32)
    unst = torch.stack([((sb[L][0] < 0) & (sb[L][1] > 0)).sum(1) for L in range(n)], 1).double()
    below = torch.cat([torch.zeros_like(unst[:, :1]), unst.cumsum(1)[:, :-1]], 1)
    K = 1 + dims[0] + below
    w = torch.tensor([2.0 * dims[l + 1] * dims[l] for l in range(n)], device=dev,
                     dtype=torch.float64)
    zflop = float((K * w).sum())
    _lib.timing_begin(['vc_mlp_tiled_zono_bounds', 'vc_mlp_tiled_zono_wide'])
    for _ in range(5):
        mf.zono_bounds(plan, xl1, xh1, None)
    kt = _lib.timing_end()
    sec = kt['vc_mlp_tiled_zono_bounds']['seconds'] + kt['vc_mlp_tiled_zono_wide']['seconds']
    out.append(_roof('k_zono_tiled + k_zono_wide_tiled (vc_mlp_tiled_zono_bounds, '
                     '_zono_wide)', '65,536 ACAS boxes (round 1)', sec, flop=5 * zflop,
                     launches=5))
    # -- k_crown_dom on round 2's batch (small-batch kernel): spec rows +
    #    each domain's own seeded rows (counted by the kernel)
    xl2, xh2, _ = kept[1]
    B2 = xl2.shape[0]
    sb2 = vz._zono_sb(gg, xl2, xh2, dev, torch.float32)
    seeded = torch.zeros(8, 16, dtype=torch.int64, device=dev)
    mf.SEED_COUNTER, mf.SEED_ROW = seeded, 0
    _lib.timing_begin(CROWN_ENTRIES)
    for _ in range(5):
        mf.crown(plan, xl2, xh2, sb2, True, spec=(Wq, bq), want_linear=True, per_domain=True)
    lst = _crown_launches(_lib.timing_end())
    mf.SEED_COUNTER = None
    rows = seeded.tolist()
    cflop = sum(f + _lib.seed_flops([dims[0]] + dims[1:n + 1], rows[k])
                for k, (_, f, _) in enumerate(lst))
    out.append(_roof(crown_kernel_name(B2), f'{B2} boxes (round 2)',
                     sum(x[0] for x in lst), flop=cflop, launches=len(lst)))
    # -- one alpha iteration launch (vc_mlp_tiled_alpha_iter) at the open
    #    leaves of round 1 (small-batch kernel) and at 65,536 domains:
    #    2 Q sum_l 2 d_l d_{l+1} per domain (spec backward + gradient sweep)
    aflop_dom = 2.0 * Q * sum(2.0 * dims[l] * dims[l + 1] for l in range(n))
    st0 = vg.bab_step(xl1, xh1, gg, se, vg.DisjunctTable({0: list(range(Q))}, dev),
                      alpha_iters=0)
    open_idx = (~st0['closed']).nonzero(as_tuple=True)[0]
    xlo, xho = xl1[open_idx].contiguous(), xh1[open_idx].contiguous()
    sbo = {L: (a[open_idx].contiguous(), b[open_idx].contiguous()) for L, (a, b) in sb.items()}
    rates = {}
    for what, (xa, xb, sba) in (('open', (xlo, xho, sbo)), ('all', (xl1, xh1, sb))):
        B = xa.shape[0]
        lo = [sba[L][0] for L in range(n)]
        hi = [sba[L][1] for L in range(n)]
        st = [torch.zeros(B, dims[L + 1], device=dev) for L in range(n) for _ in range(3)]
        lb = torch.empty(B, Q, device=dev)
        keep = [_lib.host_array(ctypes.c_void_p, [_lib.ptr(t) for t in ts])
                for ts in (lo, hi, st[0::3], st[1::3], st[2::3])]

        def it():
            _lib.call('vc_mlp_tiled_alpha_iter', plan.dims_p, n, _lib.ptr(plan.tfrag),
                      _lib.ptr(plan.bias_cat), B, _lib.ptr(xa), _lib.ptr(xb),
                      *[k[1] for k in keep[:5]], None, Q, _lib.ptr(S), _lib.ptr(acc0),
                      _lib.ptr(lb), 0.9, 0.999, 1e-8, ALPHA_LR / 0.1, 0.0316, 1, None,
                      _lib.stream())
        sec = _timed(it, 10)
        n_cu = torch.cuda.get_device_properties(0).multi_processor_count
        kern = 'k_alpha_quad' if B <= 4 * n_cu else 'k_alpha_tiled'
        out.append(_roof(f'{kern} (vc_mlp_tiled_alpha_iter, one iteration)',
                         f'{B} domains ({"round 1 open leaves" if what == "open" else "all"})',
                         sec, flop=aflop_dom * B))
        # the whole alpha loop as the step runs it (20 iterations at most,
        # the reference's early stop): evaluated iterations per second
        res = {}

        def loop():
            best, n_it = vz._run_alpha_crown_inputsplit_batched(
                xa, xb, gg, se, dev, torch.float32, n_iters=ALPHA_ITERS, lr=ALPHA_LR,
                sb=sba, return_trace=True)
            res['n'] = n_it
        sec_loop = _timed(loop, 3)
        rates[what] = {'domains': B, 'iters': res['n'], 'ms': 1e3 * sec_loop,
                       'iters_per_s': res['n'] / sec_loop,
                       'domain_iters_per_s': B * res['n'] / sec_loop}
    return out, rates


def cpu_info():
    """The host's CPU model and the threads torch uses (OMP_NUM_THREADS when
    set: the GPU box's share of its host)."""
    model = None
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    model = line.split(':', 1)[1].strip()
                    break
    except OSError:
        pass
    return {'model': model, 'nproc': os.cpu_count(), 'threads': torch.get_num_threads()}


def _median_time(fn, warm, reps):
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts), ts


def _cpu_line(units, fn, warm, reps, sample, threads=None, units_1=None, fn_1=None, reps_1=1,
              sample_1=None):
    """cpu_baseline: the oracle (the op-for-op torch CPU restatement of the
    reference) timed with perf_counter, median of ``reps`` after ``warm``
    warm-ups, on ``threads`` threads; optionally a 1-thread run of fn_1."""
    n_thr = threads or torch.get_num_threads()
    torch.set_num_threads(n_thr)
    t, ts = _median_time(fn, warm, reps)
    out = {'value': units / t, 'unit': 'domains/s', 'cores': n_thr, 'kind': 'port',
           'sample': sample, 'seconds': ts, 'cpu': cpu_info()}
    if fn_1 is not None:
        torch.set_num_threads(1)
        t1, ts1 = _median_time(fn_1, 0, reps_1)
        out['one_thread'] = {'value': units_1 / t1, 'unit': 'domains/s', 'cores': 1,
                             'sample': sample_1, 'seconds': ts1}
        torch.set_num_threads(n_thr)
    return out


def cpu_baseline_c1(reps=3):
    """The oracle on the benchmark's own step: the three BaB rounds from the
    65,536 seeded boxes (each round's children are the next round's batch),
    median of ``reps`` after a warm-up round on a 2,048-box slice.  The
    oracle's per-domain cost grows with the batch (its union-seeded CROWN
    tensors of B x 100 x 50 floats), so a smaller sample would flatter it.
    The 1-thread figure (the reference's own BLAS default) is round 1 on all
    65,536 boxes, one run."""
    from oracle import ref_bab
    from vibecheck_amd import workloads as wk
    from vibecheck_amd.spec import dedup_queries
    gg = wk.acas_gg(dtype=torch.float32)
    xl0, xh0 = wk.acas_boxes(N_DOMAINS, seed=1)
    uq, dq = dedup_queries(wk.acas_spec().as_linear_queries(5))
    se = {i: (torch.tensor(w, dtype=torch.float32), b) for i, (w, b) in enumerate(uq)}
    kw = dict(crown_intermediate=True, clip_enabled=True, alpha_iters=ALPHA_ITERS,
              alpha_all=True, alpha_lr=ALPHA_LR)
    count = [0]

    def step():
        xl, xh = xl0, xh0
        count[0] = 0
        for r in range(N_ROUNDS):
            count[0] += xl.shape[0]
            t0 = time.perf_counter()
            st = ref_bab.bab_step(xl, xh, gg, se, dq, **kw)
            print(f'cpu_baseline: oracle round {r + 1} on {xl.shape[0]} boxes, '
                  f'{time.perf_counter() - t0:.1f} s', file=sys.stderr, flush=True)
            (lxl, lxh), (hxl, hxh) = st['low'], st['high']
            xl, xh = torch.cat([hxl, lxl], 0), torch.cat([hxh, lxh], 0)

    def slice_round():
        ref_bab.bab_step(xl0[:2048].contiguous(), xh0[:2048].contiguous(), gg, se, dq, **kw)

    def round_one():
        t0 = time.perf_counter()
        ref_bab.bab_step(xl0, xh0, gg, se, dq, **kw)
        print(f'cpu_baseline: oracle round 1 on {N_DOMAINS} boxes, 1 thread, '
              f'{time.perf_counter() - t0:.1f} s', file=sys.stderr, flush=True)
    slice_round()
    out = _cpu_line(67082, step, 0, reps,
                    f'the benchmark step itself: 3 BaB rounds from the 65,536 boxes '
                    f'(CROWN intermediate, alpha 20 it, clip, split), median of {reps} after a '
                    f'warm-up round on 2,048 boxes',
                    units_1=N_DOMAINS, fn_1=round_one, reps_1=1,
                    sample_1='round 1 of the step on all 65,536 boxes (CROWN intermediate, '
                             'alpha 20 it on the open leaves, clip, split), one run')
    out['value'] = count[0] / statistics.median(out['seconds'])
    return out


def measured_traffic(kernel):
    """HBM bytes per launch of the dominant kernel on this workload, from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (each counter scaled
    by what it reads for a plain copy of known size).  The summary records
    the sha256 of the kernel's source file it measured; a summary of an older
    source gives None (and the reason)."""
    import hashlib
    path = os.path.join(ROOT, 'profiles', f'{kernel}_acas_65536_traffic.md')
    src = os.path.join(ROOT, 'vibecheck-nn_amd', 'csrc', 'vc_mlp_tiled.hip')
    try:
        with open(src, 'rb') as f:
            cur = hashlib.sha256(f.read()).hexdigest()
        val = sha = None
        with open(path) as f:
            for line in f:
                if line.startswith('traffic_bytes_per_launch:'):
                    val = float(line.split(':', 1)[1])
                elif line.startswith('source_sha256:'):
                    sha = line.split(':', 1)[1].strip()
    except OSError:
        return None, 'no traffic summary'
    if sha != cur:
        return None, 'traffic summary measured an older vc_mlp_tiled.hip'
    return val, 'rocprofv3 FETCH_SIZE + WRITE_SIZE of this source (sha256 matches)'


def copy_probe(mib):
    """A plain device copy of known size (read mib MiB, write mib MiB), three
    times: the calibration dispatch for the FETCH_SIZE / WRITE_SIZE counters."""
    n = mib * (1 << 20) // 4
    src = torch.rand(n, device='cuda:0')
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({'copy_probe_bytes_read': n * 4, 'copy_probe_bytes_written': n * 4}))


ROTATE_BYTES = 768 << 20  # > 2x the 256 MB Infinity Cache


def _time_launches(fns, reps):
    """Average seconds per launch of fns (cycled) over reps launches, HIP
    events on the current stream (the launch stream of every entry point)."""
    for f in fns:
        f()
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for i in range(reps):
        fns[i % len(fns)]()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / 1e3 / reps


def _n_sets(bytes_per_set):
    """Independent input/output sets cycled per launch, so that a launch
    reads what the previous ones left in HBM, not in the 256 MB cache."""
    return max(1, min(32, -(-ROTATE_BYTES // max(1, bytes_per_set))))


def kernel_suite(reps):
    """The layer-wise kernels one at a time at workload shapes: one JSON line
    each with the algorithmic bytes (HBM-bound kernels) or FLOP (GEMM-shaped
    kernels) per launch, the average launch time and the fraction of the
    MI355X peak.  A plain device copy gives the achievable HBM rate."""
    from vibecheck_amd import _lib
    from vibecheck_amd._lib import call, load, ptr, stream

    dev = torch.device('cuda:0')
    _lib.load()
    st = stream()
    gen = torch.Generator(device=dev).manual_seed(7)

    def rnd(*shape):
        return torch.rand(*shape, device=dev, generator=gen)

    def rndn(*shape):
        return torch.randn(*shape, device=dev, generator=gen)

    def bounds(*shape):
        lo = rndn(*shape)
        return lo, lo + rnd(*shape) * 2.0

    def report(row, kernel, workload, sec, bound, amount):
        if bound == 'hbm':
            achieved, peak, unit = amount / sec / 1e9, HBM_PEAK_GBS, 'GB/s'
        else:
            achieved, peak, unit = amount / sec / 1e12, FP32_MFMA_PEAK, 'TFLOP/s'
        print(json.dumps({
            'row': row, 'kernel': kernel, 'workload': workload, 'bound': bound,
            'avg_launch_us': sec * 1e6, 'achieved': achieved, 'peak': peak, 'unit': unit,
            'frac': achieved / peak,
            ('bytes' if bound == 'hbm' else 'flop'): amount}), flush=True)

    # -- achievable: a plain 1 GiB device copy
    n = (1 << 30) // 4
    src = rnd(n)
    dst = torch.empty_like(src)
    sec = _time_launches([lambda: dst.copy_(src)], reps)
    report('-', 'device copy (torch copy_)', '1 GiB read + 1 GiB write', sec, 'hbm', 2.0 * n * 4)
    del src, dst
    # -- achievable at the narrow kernels' sizes (tens of MB per launch, where
    #    launch and drain take a larger share): 40 MiB copies, sets rotated
    #    past the 256 MB cache like the rows below
    n = (40 << 20) // 4
    sets = [(rnd(n), torch.empty(n, device=dev)) for _ in range(_n_sets(8 * n))]
    sec = _time_launches([lambda s=s: s[1].copy_(s[0]) for s in sets], reps)
    report('-', 'device copy (torch copy_)', '40 MiB read + 40 MiB write', sec, 'hbm', 2.0 * n * 4)
    del sets

    # -- a1: slopes of every (domain, neuron), 524,288 x 50
    n = 524288 * 50
    per = n * 23
    sets = []
    for _ in range(_n_sets(per)):
        lo, hi = bounds(n)
        outs = [torch.empty(n, device=dev) for _ in range(3)]
        flags = [torch.empty(n, dtype=torch.uint8, device=dev) for _ in range(3)]
        sets.append((lo, hi, outs, flags))
    fns = [lambda s=s: call('vc_make_slopes', ptr(s[0]), ptr(s[1]), n, *map(ptr, s[2]),
                            *map(ptr, s[3]), st) for s in sets]
    report('a1', 'k_make_slopes', '524,288 x 50 (lo, hi in; 3 slopes + 3 masks out)',
           _time_launches(fns, reps), 'hbm', per)
    del sets, fns

    # -- a8: concretization, A (B*R, n_in)
    for B, R, n_in, what in ((512, 2048, 784, '784-input MLP, 512 domains x 2048 seeded rows'),
                             (524288, 4, 5, '5-input MLP, 524,288 domains x 4 spec rows')):
        M = B * R
        per = 4 * (M * n_in + 2 * M + 2 * B * n_in)
        sets = []
        for _ in range(_n_sets(per)):
            A = rndn(M, n_in)
            acc = rndn(M)
            xl = rnd(B, n_in)
            sets.append((A, acc, xl, xl + 0.05, torch.empty(M, device=dev)))
        fns = [lambda s=s: call('vc_concretize', ptr(s[0]), ptr(s[1]), ptr(s[2]), ptr(s[3]),
                                M, R, n_in, 0, ptr(s[4]), st) for s in sets]
        kern = 'k_concretize_tile' if n_in <= 32 else 'k_concretize_wave'
        report('a8', kern, what, _time_launches(fns, reps), 'hbm', per)
        del sets, fns

    # -- a6: relaxation alone (the relu before a conv), 64 domains x 128 rows
    #    x 32,768 neurons (the 32x32x32 activation of the CNN)
    B, R, nn = 64, 128, 32768
    M = B * R
    per = 8 * M * nn + 8 * B * nn + 8 * M
    ew = rndn(M, nn)
    lo, hi = bounds(B, nn)
    out = torch.empty_like(ew)
    acc = torch.zeros(M, device=dev)
    fn = lambda: call('vc_backward_relu', ptr(ew), M, R, nn, ptr(lo), ptr(hi), None, 0, None,
                      ptr(out), ptr(acc), st)
    report('a6', 'k_backward_relu', '8,192 rows x 32,768 neurons (64 domains x 128 rows)',
           _time_launches([fn], reps), 'hbm', per)
    del ew, out, acc, lo, hi

    # -- a9: Adam step over every alpha of 524,288 domains x 6 x 50
    n = 524288 * 300
    per = 28 * n
    p, g, m, v = rnd(n), rndn(n), rndn(n) * 0.01, rnd(n) * 0.01
    fn = lambda: call('vc_adam_step', ptr(p), ptr(g), ptr(m), ptr(v), n, 0.9, 0.999, 1e-8,
                      0.1, 0.5, 0.0, 1.0, st)
    report('a9', 'k_adam', '157,286,400 alphas (524,288 domains x 6 x 50)',
           _time_launches([fn], reps), 'hbm', per)
    del p, g, m, v

    # -- a12-a14 on 524,288 5-dim boxes
    B, Q, nd = 524288, 4, 5
    d_ptr = torch.tensor([0, Q], dtype=torch.int32, device=dev)
    q_idx = torch.arange(Q, dtype=torch.int32, device=dev)
    per = B * (40 + 4 * Q * nd + 4 * Q + 40 + 1)
    sets = []
    for _ in range(_n_sets(per)):
        xl = rnd(B, nd) * 2 - 1
        xh = xl + rnd(B, nd) * 0.1
        A = rndn(B, Q, nd)
        b = rndn(B, Q) * 0.01 - 0.2
        sets.append((xl, xh, A, b, torch.empty_like(xl), torch.empty_like(xh),
                     torch.empty(B, dtype=torch.uint8, device=dev)))
    fns = [lambda s=s: call('vc_clip_box', ptr(s[0]), ptr(s[1]), ptr(s[2]), ptr(s[3]), B, Q, nd,
                            ptr(d_ptr), ptr(q_idx), 1, ptr(s[4]), ptr(s[5]), ptr(s[6]), st)
           for s in sets]
    report('a12', 'k_clip', '524,288 boxes, 5 dims, 4 halfspaces', _time_launches(fns, reps),
           'hbm', per)
    per = B * (40 + 8 + 1)
    outs = [(torch.empty(B, dtype=torch.int64, device=dev),
             torch.empty(B, dtype=torch.uint8, device=dev)) for _ in sets]
    fns = [lambda s=s, o=o: call('vc_widest_axis', ptr(s[0]), ptr(s[1]), B, nd, ptr(o[0]),
                                 ptr(o[1]), st) for s, o in zip(sets, outs)]
    report('a13', 'k_widest', '524,288 boxes, 5 dims', _time_launches(fns, reps), 'hbm', per)
    per = B * (40 + 8 + 8 + 80)
    idx = torch.arange(B, dtype=torch.int64, device=dev)
    kids = [[torch.empty(B, nd, device=dev) for _ in range(4)] for _ in sets]
    fns = [lambda s=s, o=o, c=c: call('vc_bisect', ptr(s[0]), ptr(s[1]), ptr(o[0]), ptr(idx), B,
                                      nd, *map(ptr, c), st)
           for s, o, c in zip(sets, outs, kids)]
    report('a14', 'k_bisect', '524,288 boxes, 5 dims', _time_launches(fns, reps), 'hbm', per)
    del sets, outs, kids
    flags = (rnd(B) < 0.5).to(torch.uint8)
    cnt_true = int(flags.sum())
    ws = torch.empty(max(8, _lib.load().vc_compact_workspace(B)), dtype=torch.uint8, device=dev)
    cidx = torch.empty(B, dtype=torch.int64, device=dev)
    cnt = torch.empty(1, dtype=torch.int64, device=dev)
    fn = lambda: call('vc_compact', ptr(flags), B, 0, ptr(cidx), ptr(cnt), ptr(ws), ws.numel(),
                      st)
    report('a14', 'k_compact_count + k_compact_scan + k_compact_write',
           '524,288 flags, half set', _time_launches([fn], reps), 'hbm', 2 * B + 8 * cnt_true)
    del flags, ws, cidx

    # -- a5 + a6: backward through relu -> fc (fp32 MFMA): the two-phase
    #    step the layer-wise path runs (k_relax_rows streams the relaxed rows,
    #    then the plain gemm_kernel), and the fused single-kernel form
    for B, R, n_out, n_in, what in (
            (512, 512, 1024, 1024, '1024x1024 fc, 512 domains x 512 seeded rows'),
            (8192, 9, 256, 256, '256x256 fc, 8,192 domains x 9 spec rows')):
        M = B * R
        ew = rndn(M, n_out)
        lo, hi = bounds(B, n_out)
        W = rndn(n_out, n_in) * (2.0 / n_in) ** 0.5
        bias = rndn(n_out) * 0.01
        out = torch.empty(M, n_in, device=dev)
        acc = torch.zeros(M, device=dev)
        rel = torch.empty(M, n_out, device=dev)
        for kern, r in (('k_relax_rows + rocBLAS sgemm (two-phase backward fc)', rel),
                        ('gemm_kernel (fused relaxation + backward fc)', None)):
            fn = lambda r=r: call('vc_backward_fc', ptr(ew), M, R, n_out, ptr(lo), ptr(hi), None,
                                  0, None, ptr(W), ptr(bias), n_in, ptr(out), ptr(acc), ptr(r),
                                  0, st)
            report('a5', kern, what, _time_launches([fn], max(3, reps // 4)), 'mfma',
                   2.0 * M * n_out * n_in)
        del ew, out, acc, rel

    # -- a9: alpha gradient sweep step (relaxation subgradient + fc^T)
    B, Q, n, n_next = 512, 9, 1024, 1024
    M = B * Q
    gE, P = rndn(M, n), rndn(M, n)
    lo, hi = bounds(B, n)
    alpha = rnd(B, n)
    Wn = rndn(n_next, n) * (2.0 / n) ** 0.5
    ls, us, ut = (torch.empty(B, n, device=dev) for _ in range(3))
    g2 = torch.empty(M, n_next, device=dev)

    def grad_step():
        call('vc_relax_slopes', ptr(lo), ptr(hi), ptr(alpha), B * n, ptr(ls), ptr(us), ptr(ut),
             st)
        call('vc_alpha_grad_step_slopes', ptr(gE), ptr(P), M, Q, n, ptr(ls), ptr(us), ptr(ut),
             0, ptr(Wn), None, n_next, ptr(g2), st)
    report('a9', 'k_relax_slopes + gemm_kernel (alpha gradient step)',
           '1024x1024 fc, 512 domains x 9 spec rows', _time_launches([grad_step], reps), 'mfma',
           2.0 * M * n * n_next)
    del gE, P, g2

    # -- a2: interval fc (two products: mid W^T, rad |W|^T)
    B, n_in, n_out = 8192, 784, 256
    l = rnd(B, n_in)
    h = l + 0.06
    W = rndn(n_out, n_in) * (2.0 / n_in) ** 0.5
    bias = torch.zeros(n_out, device=dev)
    lo, hi = torch.empty(B, n_out, device=dev), torch.empty(B, n_out, device=dev)
    fn = lambda: call('vc_ibp_fc', ptr(l), ptr(h), B, n_in, ptr(W), ptr(bias), n_out, ptr(lo),
                      ptr(hi), st)
    report('a2', 'gemm_kernel (interval fc, two products)', '784->256 fc, 8,192 boxes',
           _time_launches([fn], reps), 'mfma', 2.0 * 2 * B * n_in * n_out)

    # -- a7: backward through the CNN's convolutions (transposed conv as
    #    implicit GEMM by output parity class), 64 domains x 9 spec rows
    for C_in, H, C_out, k, cs, cp in ((3, 32, 32, 3, 1, 1), (32, 32, 64, 4, 2, 1),
                                      (64, 16, 64, 4, 2, 1)):
        Ho = (H + 2 * cp - k) // cs + 1
        M = 64 * 9
        ew = rndn(M, C_out * Ho * Ho)
        K = rndn(C_out, C_in, k, k) * (2.0 / (C_in * k * k)) ** 0.5
        bias = rndn(C_out) * 0.01
        out = torch.empty(M, C_in * H * H, device=dev)
        acc = torch.zeros(M, device=dev)
        KT = torch.empty(load().vc_conv_t_pack_floats(C_out, C_in, k, k, cs, cs), device=dev)
        call('vc_conv_t_pack', ptr(K), C_out, C_in, k, k, cs, cs, cp, cp, ptr(KT), st)
        fn = lambda: call('vc_backward_conv_packed', ptr(ew), M, ptr(K), ptr(KT), ptr(bias),
                          C_out, Ho, Ho, C_in, H, H, k, k, cs, cs, cp, cp, ptr(out), ptr(acc),
                          st)
        work = f'conv {C_in}->{C_out} {k}x{k} s{cs} p{cp} ({H}x{H} in), 576 rows (64 domains x 9)'
        flop = 2.0 * M * (C_out * Ho * Ho) * (C_in * k * k)
        if C_in <= 4:
            report('a7', 'k_conv_t_fold (MFMA GEMM + fold, bias dot fused)', work,
                   _time_launches([fn], max(3, reps // 4)), 'mfma', flop)
        else:
            report('a7', 'gemm_kernel<LoadPackedT> (transposed conv, packed taps) + '
                   'k_conv_bias_dot', work, _time_launches([fn], max(3, reps // 4)), 'mfma',
                   flop)
            fn = lambda: call('vc_backward_conv', ptr(ew), M, ptr(K), ptr(bias), C_out, Ho, Ho,
                              C_in, H, H, k, k, cs, cs, cp, cp, ptr(out), ptr(acc), st)
            report('a7', 'gemm_kernel<LoadKernelT> (transposed conv, taps from the kernel) + '
                   'k_conv_bias_dot', work, _time_launches([fn], max(3, reps // 4)), 'mfma',
                   flop)
        del ew, out, acc, KT

    # -- a6+a7: the relu relaxation fused into the first layer's conv
    #    backward, rows shared by the domains until that relu (the CROWN
    #    intermediate-bound chunks of the CNN): 64 domains x 512 rows
    C_in, H, C_out, k, cs, cp = 3, 32, 32, 3, 1, 1
    Ho, B, R = H, 64, 512
    n = C_out * Ho * Ho
    M = B * R
    x = rndn(R, n)
    lo = rndn(B, n)
    hi = lo + rnd(B, n) * 2
    ls, us, ut = (torch.empty(B, n, device=dev) for _ in range(3))
    call('vc_relax_slopes', ptr(lo), ptr(hi), None, B * n, ptr(ls), ptr(us), ptr(ut), st)
    K = rndn(C_out, C_in, k, k) * (2.0 / (C_in * k * k)) ** 0.5
    bias = rndn(C_out) * 0.01
    out = torch.empty(M, C_in * H * H, device=dev)
    acc = torch.zeros(M, device=dev)
    fn = lambda: call('vc_backward_relu_conv', ptr(x), M, R, 1, ptr(ls), ptr(us), ptr(ut), None,
                      ptr(K), ptr(bias), C_out, Ho, Ho, C_in, H, H, k, k, cs, cs, cp, cp,
                      ptr(out), ptr(acc), st)
    report('a7', 'k_conv_t_fold<relu> (relu relaxation + MFMA GEMM + fold + bias dot)',
           f'relu + conv {C_in}->{C_out} {k}x{k} s{cs} p{cp} ({H}x{H} in), {M:,} rows '
           f'({B} domains x {R} shared rows)', _time_launches([fn], max(3, reps // 4)), 'mfma',
           2.0 * M * n * (C_in * k * k))
    del x, lo, hi, ls, us, ut, out, acc

    # -- a2: interval forward through the CNN's second convolution, 64 boxes
    C_in, H, C_out, k, cs, cp, B = 32, 32, 64, 4, 2, 1, 64
    Ho = (H + 2 * cp - k) // cs + 1
    l = rnd(B, C_in * H * H)
    h = l + 0.01
    K = rndn(C_out, C_in, k, k) * (2.0 / (C_in * k * k)) ** 0.5
    bias = rndn(C_out) * 0.01
    lo, hi = torch.empty(B, C_out * Ho * Ho, device=dev), torch.empty(B, C_out * Ho * Ho,
                                                                      device=dev)
    fn = lambda: call('vc_ibp_conv', ptr(l), ptr(h), B, C_in, H, H, ptr(K), ptr(bias), C_out, k,
                      k, cs, cs, cp, cp, Ho, Ho, ptr(lo), ptr(hi), st)
    report('a2', 'gemm_kernel (interval conv, two products, implicit GEMM)',
           f'conv {C_in}->{C_out} {k}x{k} s{cs} p{cp} ({H}x{H} in), 64 boxes',
           _time_launches([fn], reps), 'mfma', 2.0 * 2 * B * (C_out * Ho * Ho) * (C_in * k * k))


def hybrid_replay_suite(reps=5, B=4096, spec_iters=10):
    """The hybrid replay (zonotope bounds, frozen per-query alpha layer
    tightening, ``spec_iters`` per-leaf spec alpha Adam iterations) on
    B ACAS-Xu-shaped leaves, each with its own group's alphas: one JSON line
    with the time per call, leaves/s and the algorithmic FLOP of the
    per-row backward GEMMs of the layer tightening (2 * B * 2 n_L * n_out *
    n_in per fc below the seeded one, Q = 2 n_L rows per leaf)."""
    from vibecheck_amd import verify_hybrid_acasxu as vh
    from vibecheck_amd import workloads as wk
    from vibecheck_amd.spec import dedup_queries

    dev = torch.device('cuda:0')
    gg = wk.acas_gg(device=dev, dtype=torch.float32)
    spec = wk.pairwise_spec(5, [0.0], [0.0], True)
    uq, _ = dedup_queries(spec.as_linear_queries(5))
    se = {i: (torch.tensor(w, dtype=torch.float32, device=dev), b) for i, (w, b) in enumerate(uq)}
    xl, xh = wk.acas_boxes(32, seed=3, device=dev, dtype=torch.float32)
    _, a_layer, a_spec, _ = vh._full_freeze(xl, xh, gg, se, dev, torch.float32,
                                            n_iters_per_layer=20, n_iters_spec=20)
    g = torch.Generator(device=dev).manual_seed(5)
    gid = torch.randint(0, 32, (B,), device=dev, generator=g)
    t = torch.rand(B, 5, device=dev, generator=g)
    c, r = (xl + xh)[gid] / 2, (xh - xl)[gid] / 2
    bxl, bxh = c - r * t, c + r * t
    fcs = [op for op in gg['ops'] if op['type'] == 'fc']
    flop = 0.0
    for L in a_layer:
        if a_layer[L]:
            q = 2 * fcs[L]['W'].shape[0]
            flop += sum(2.0 * B * q * f['W'].shape[0] * f['W'].shape[1] for f in fcs[:L])
    def timed(fn):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / reps

    # the driver's form: frozen layer alphas read by group index
    sec = timed(lambda: vh._replay_batched(bxl, bxh, gg, se, a_layer, a_spec, dev,
                                           torch.float32, spec_iters=spec_iters, group=gid))
    # per-leaf alpha copies (gathered inside the timed region)
    sec_copy = timed(lambda: vh._replay_batched(bxl, bxh, gg, se,
                                                *vh._gather_alphas(a_layer, a_spec, gid), dev,
                                                torch.float32, spec_iters=spec_iters))
    print(json.dumps({
        'row': 'f4', 'kernel': '_replay_batched (per-row alpha backward + spec alpha Adam)',
        'workload': f'ACAS-Xu 5-50x6-5, {B} leaves of 32 groups, {spec_iters} spec iterations',
        'ms_per_call': sec * 1e3, 'leaves_per_s': B / sec,
        'ms_per_call_per_leaf_alpha_copies': sec_copy * 1e3,
        'tighten_gemm_flop': flop, 'tighten_gemm_tflops_over_call': flop / sec / 1e12}),
        flush=True)


# Algorithmic FLOP per launch of the layer-wise MFMA entry points, from
# their arguments (the per-config bench lines time them with HIP events).
LAYERWISE_MFMA = {
    # 2 M n_out n_in
    'vc_backward_fc': lambda a: 2.0 * a[1] * a[3] * a[11],
    # 2 M (C_out H_out W_out)(C_in kh kw)
    'vc_backward_conv': lambda a: 2.0 * a[1] * a[4] * a[5] * a[6] * a[7] * a[10] * a[11],
    'vc_backward_conv_packed': lambda a: 2.0 * a[1] * a[5] * a[6] * a[7] * a[8] * a[11] * a[12],
    'vc_backward_relu_conv': lambda a: 2.0 * a[1] * a[10] * a[11] * a[12] * a[13] * a[16] * a[17],
    # 2 M n n_next
    'vc_alpha_grad_step_slopes': lambda a: 2.0 * a[2] * a[4] * a[11],
    'vc_alpha_grad_step': lambda a: 2.0 * a[2] * a[4] * a[11],
    # mid W^T and rad |W|^T: 4 B n_in n_out
    'vc_ibp_fc': lambda a: 4.0 * a[2] * a[3] * a[6],
    # centre and K generator columns through W: 2 B n_out n_in (K + 1)
    'vc_zono_fc': lambda a: 2.0 * a[2] * a[3] * a[7] * (a[4] + 1),
    # the same through a conv: 2 B (Kg + 1)(C_out H_out W_out)(C_in kh kw)
    'vc_zono_conv': lambda a: 2.0 * a[2] * (a[3] + 1) * a[9] * a[16] * a[17] * a[4] * a[10] * a[11],
    # 4 B (C_out H_out W_out)(C_in kh kw)
    'vc_ibp_conv': lambda a: 4.0 * a[2] * a[8] * a[15] * a[16] * a[3] * a[9] * a[10],
}


def layerwise_roofline(step, reps):
    """Run ``step`` with HIP events around every layer-wise MFMA entry
    point: per entry its time per step, algorithmic TFLOP/s and fraction of
    the fp32 MFMA peak; the roofline is the entry with the most time."""
    from vibecheck_amd import _lib
    for name, f in LAYERWISE_MFMA.items():
        _lib._FLOPS[name] = f
    _lib.timing_begin(list(LAYERWISE_MFMA))
    for _ in range(reps):
        step()
    kt = _lib.timing_end()
    rows = []
    for name, k in kt.items():
        if k['launches'] and k['seconds'] > 0:
            ach = k['flops'] / k['seconds'] / 1e12
            rows.append({'entry': name, 'ms_per_step': 1e3 * k['seconds'] / reps,
                         'launches_per_step': k['launches'] / reps, 'achieved': ach,
                         'frac': ach / FP32_MFMA_PEAK})
    rows.sort(key=lambda r: -r['ms_per_step'])
    return rows


def run_config(cfg, steps, warmup, cpu):
    """One JSON line for a non-headline configuration: value = domains
    bounded per second of the configuration's step (below), the roofline of
    its dominant kernel, the CPU oracle on the same step (full batch or a
    stated sample)."""
    from oracle import ref_bab, ref_bound as rb
    from vibecheck_amd import _lib
    from vibecheck_amd import mlp_fused as mf
    from vibecheck_amd import verify_graph as vg
    from vibecheck_amd import verify_milp as vm
    from vibecheck_amd import verify_zono_bnb as vz
    from vibecheck_amd import workloads as wk
    from vibecheck_amd.spec import dedup_queries
    dev = torch.device('cuda:0')
    F = torch.float32
    _lib.load()

    def specs(n_out, one):
        spec = wk.pairwise_spec(n_out, [0.0], [0.0], one)
        uq, dq = dedup_queries(spec.as_linear_queries(n_out))
        c = {i: (torch.tensor(w, dtype=F), b) for i, (w, b) in enumerate(uq)}
        return c, {k: (w.to(dev), b) for k, (w, b) in c.items()}, dq

    line = {'unit': 'domains/s', 'n_gpus': 1, 'steps': steps, 'warmup': warmup,
            'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f32',
            'data': 'synthetic (seeded boxes and Kaiming-normal weights)'}
    if cfg == 'c0':
        gg = wk.acas_gg(device=dev, dtype=F)
        ggc = wk.acas_gg(dtype=F)
        xlc, xhc = wk.acas_boxes(4096, seed=1)
        xl, xh = xlc.to(dev), xhc.to(dev)
        sec_c, se, dq = specs(5, True)
        table = vg.DisjunctTable(dq, dev)
        B = 4096

        def step():
            vg.bab_step(xl, xh, gg, se, table, crown_intermediate=True, clip_enabled=True,
                        alpha_iters=0)
        line.update(metric='CROWN-bounded domains/sec at 1 GPU (5-50x6-5 MLP, 4,096 domains, '
                           'one BaB step)',
                    config={'workload': '5-50x6-5 ReLU MLP, 4,096 input boxes, one BaB step: '
                                        'CROWN intermediate + spec bound + clip + widest split',
                            'domains_per_step': B})
        cpu_fn = lambda: ref_bab.bab_step(xlc, xhc, ggc, sec_c, dq)
        cpu_kw = dict(units=B, warm=1, reps=5, sample='the full step (4,096 boxes)',
                      units_1=1024, reps_1=3, sample_1='the step on the first 1,024 boxes',
                      fn_1=lambda: ref_bab.bab_step(xlc[:1024], xhc[:1024], ggc, sec_c, dq))
    elif cfg == 'c2':
        gg = wk.mnist_mlp_gg(device=dev, dtype=F)
        ggc = wk.mnist_mlp_gg(dtype=F)
        xlc, xhc = wk.mnist_mlp_boxes(512)
        xl, xh = xlc.to(dev), xhc.to(dev)
        sec_c, se, _ = specs(10, False)
        B = 512

        def step():
            sb = vz._crown_intermediate_batched(gg, xl, xh, dev, F)
            vz._run_alpha_crown_inputsplit_batched(xl, xh, gg, se, dev, F, n_iters=10,
                                                   lr=0.25, sb=sb)

        def cpu_step(n):
            sbc = rb.crown_intermediate_batched(ggc, xlc[:n], xhc[:n])
            rb.alpha_crown_batched(xlc[:n], xhc[:n], ggc, sec_c, n_iters=10, lr=0.25, sb=sbc)
        line.update(metric='CROWN-bounded domains/sec at 1 GPU (784-1024x4-10 MLP, 512 '
                           'domains, CROWN intermediate + alpha-CROWN 10 it)',
                    config={'workload': '784-[1024]x4-10 ReLU MLP, 512 L-inf boxes eps 0.02: '
                                        'CROWN intermediate bounds for every ReLU layer, '
                                        'then 10 alpha-CROWN iterations (lr 0.25)',
                            'domains_per_step': B})
        cpu_kw = dict(units=16, warm=1, reps=5,
                      sample='the step on the first 16 of the 512 boxes (the oracle seeds '
                             'the union of those 16 boxes\' unstable neurons, fewer rows per '
                             'domain than the GPU\'s 512-box union)',
                      units_1=4, reps_1=1, sample_1='the step on the first 4 boxes',
                      fn_1=lambda: cpu_step(4))
        cpu_fn = lambda: cpu_step(16)
    elif cfg == 'c3':
        gg = wk.cifar_cnn_gg(device=dev, dtype=F)
        ggc = wk.cifar_cnn_gg(dtype=F)
        xlc, xhc = wk.cifar_cnn_boxes(64)
        xl, xh = xlc.to(dev), xhc.to(dev)
        sec_c, se, _ = specs(10, False)
        B = 64

        def step():
            ibp = vz._ibp_forward_graph_batched(xl, xh, gg, dev, F)
            sb = vz._crown_intermediate_batched(gg, xl, xh, dev, F, sb=ibp)
            vz._spec_backward_graph_batched(sb, xl, xh, gg, se, dev, F)

        def cpu_step(n):
            ibp = rb.ibp_forward_batched(xlc[:n], xhc[:n], ggc)
            sbc = rb.crown_intermediate_batched(ggc, xlc[:n], xhc[:n], sb=ibp)
            rb.spec_backward_batched(sbc, xlc[:n], xhc[:n], ggc, sec_c)
        line.update(metric='CROWN-bounded domains/sec at 1 GPU (3x32x32 CNN, 64 domains, '
                           'CROWN with intermediate bounds)',
                    config={'workload': 'CNN conv 3-32 3x3, 32-64 4x4 s2, 64-64 4x4 s2, fc '
                                        '4096-512-10; 64 L-inf boxes eps 2/255: IBP, CROWN '
                                        'intermediate bounds (IBP-seeded), spec bound',
                            'domains_per_step': B})
        cpu_fn = lambda: cpu_step(1)
        cpu_kw = dict(units=1, warm=1, reps=3, sample='the step on the first of the 64 boxes')
    elif cfg == 'c4':
        widths = wk.DEEP_MLP_WIDTHS
        Ws, bs = wk.mlp_params(widths, seed=0)
        gg = wk.mlp_gg(Ws, bs, device=dev, dtype=F)
        ggc = wk.mlp_gg(Ws, bs, dtype=F)
        x_l, x_h = wk.linf_boxes(1, 784, 0.03, seed=1, dtype=F)
        root_c = {L: (lo[0], hi[0]) for L, (lo, hi) in
                  rb.ibp_forward_batched(x_l, x_h, ggc).items()}
        root = {L: (a.to(dev), b.to(dev)) for L, (a, b) in root_c.items()}
        un = [(L, int(j)) for L in sorted(root_c)
              for j in ((root_c[L][0] < 0) & (root_c[L][1] > 0)).nonzero().flatten().tolist()]
        layer, neuron, side = wk.relu_split_domains(un, n_domains=8192, n_splits=8, seed=2)
        cl, _ = vm._split_clamps_batched(layer.to(dev), neuron.to(dev), side.to(dev),
                                         widths[1:-1], dev)
        sec_c, se, _ = specs(10, False)
        xl, xh = x_l[0].to(dev), x_h[0].to(dev)
        B = 8192

        def step():
            vm._ibp_crown_bab_bound(gg, xl, xh, root, cl, se, dev, F, alpha_iters=10, lr=0.25)

        def cpu_step(n):
            clamps = wk.relu_clamps_from_splits(layer[:n], neuron[:n], side[:n], widths[1:-1])
            xlb, xhb = x_l.expand(n, -1).clone(), x_h.expand(n, -1).clone()
            sbc = rb.split_domain_bounds(xlb, xhb, ggc, root_c, clamps)
            rb.beta_crown_bound(sbc, xlb, xhb, ggc, sec_c, rb.beta_signs_from_clamps(clamps),
                                n_iters=10, lr=0.25)
        line.update(metric='CROWN-bounded domains/sec at 1 GPU (784-256x6-10 MLP, 8,192 '
                           'ReLU-split subdomains, alpha/beta 10 it)',
                    config={'workload': '784-[256]x6-10 ReLU MLP, one L-inf box eps 0.03 split '
                                        'into 8,192 subdomains of 8 ReLU splits: IBP with the '
                                        'split clamps, joint alpha/beta-CROWN 10 Adam '
                                        'iterations (lr 0.25)',
                            'domains_per_step': B})
        cpu_fn = lambda: cpu_step(8192)
        cpu_kw = dict(units=8192, warm=1, reps=3, sample='the full step (8,192 subdomains)',
                      units_1=1024, reps_1=1, sample_1='the step on the first 1,024 subdomains',
                      fn_1=lambda: cpu_step(1024))
    else:
        raise SystemExit(f'unknown config {cfg}')
    # setup objects to the permanent generation (see main)
    gc.collect()
    gc.freeze()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    per_step = (time.perf_counter() - t0) / steps
    line.update(value=B / per_step, ms_per_step=1e3 * per_step)
    # alpha's own rates at the configuration's batch (outside the timed step)
    if cfg == 'c2':
        sb = vz._crown_intermediate_batched(gg, xl, xh, dev, F)
        res = {}

        def alpha_only():
            _, res['n'] = vz._run_alpha_crown_inputsplit_batched(
                xl, xh, gg, se, dev, F, n_iters=10, lr=0.25, sb=sb, return_trace=True)
        sec = _timed(alpha_only, 3)
        line['alpha'] = {'domains': B, 'iters': int(res['n']), 'ms': 1e3 * sec,
                         'iters_per_s': res['n'] / sec, 'domain_iters_per_s': B * res['n'] / sec,
                         'sample': 'the alpha-CROWN loop alone from the step\'s CROWN bounds'}
    elif cfg == 'c4':
        res = {}

        def ab_only():
            _, res['n'] = vm._ibp_crown_bab_bound(gg, xl, xh, root, cl, se, dev, F,
                                                  alpha_iters=10, lr=0.25, return_trace=True)
        sec = _timed(ab_only, 3)
        line['alpha_beta'] = {'domains': B, 'iters': int(res['n']), 'ms': 1e3 * sec,
                              'iters_per_s': res['n'] / sec,
                              'domain_iters_per_s': B * res['n'] / sec,
                              'sample': 'the whole bound call: IBP with the split clamps, '
                                        'then the joint alpha/beta iterations'}
    if cfg == 'c0':
        seeded = torch.zeros(steps + 4, 16, dtype=torch.int64, device=dev)
        mf.SEED_COUNTER, mf.SEED_ROW = seeded, 0
        _lib.timing_begin(CROWN_ENTRIES)
        for _ in range(steps):
            step()
        lst = _crown_launches(_lib.timing_end())
        mf.SEED_COUNTER = None
        dims = mf.plan_for(gg, dev).dims
        flop = sum(f + _lib.seed_flops(dims, seeded.tolist()[_seed_row(k, a)])
                   for k, (_, f, a) in enumerate(lst))
        sec = sum(x[0] for x in lst)
        line['roofline'] = _roof(crown_kernel_name(B), f'{B:,} boxes', sec,
                                 flop=flop, launches=len(lst))
        line['roofline'].update(traffic=None, share_of_step=sec / steps / per_step)
    else:
        rows = layerwise_roofline(step, steps)
        top = rows[0]
        how = {'vc_backward_fc': 'relaxation pass + rocBLAS sgemm',
               'vc_zono_fc': 'rocBLAS strided-batched sgemm for the generators'}.get(
                   top['entry'], 'MFMA GEMM core')
        line['roofline'] = {'kernel': f'{top["entry"]} ({how})', 'bound': 'mfma',
                            'achieved': top['achieved'], 'peak': FP32_MFMA_PEAK,
                            'unit': 'TFLOP/s', 'frac': top['frac'], 'traffic': None,
                            'share_of_step': top['ms_per_step'] / (1e3 * per_step)}
        line['mfma_entries'] = rows
    if cpu:
        line['cpu_baseline'] = _cpu_line(fn=cpu_fn, **cpu_kw)
    return line


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=5)
    ap.add_argument('--warmup', type=int, default=2)
    ap.add_argument('--config', default='c1', choices=['c0', 'c1', 'c2', 'c3', 'c4'],
                    help='c1 (default): the headline 65,536-box ACAS step; the others print '
                         'their own line')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--lookahead', choices=['off', 'tail', 'overlap'], default=None,
                    help="how each round but the last bounds the next batch (the same "
                         "results): 'tail' after its split, on the same stream (the "
                         "driver's default); 'overlap' on the main stream while its alpha "
                         "runs on a second one; 'off' each round bounds its own batch")
    ap.add_argument('--no-secondary', action='store_true',
                    help='after the timed steps, skip the extra pass over the rounds '
                         '(near-zero counts, secondary rooflines, alpha rates): a profile '
                         'of the run then holds the warm-up and timed steps only')
    ap.add_argument('--cpu-reps', type=int, default=3,
                    help='timed CPU runs of the headline step (median)')
    ap.add_argument('--no-configs', action='store_true',
                    help='skip the other configurations (C0, C2, C3, C4), which the default '
                         'run carries under "configs", each with its roofline and CPU line')
    ap.add_argument('--copy-probe', type=int, default=0, metavar='MIB',
                    help='only run a plain copy of MIB MiB (counter calibration)')
    ap.add_argument('--kernels', action='store_true',
                    help='only time the layer-wise kernels one at a time (one JSON line each)')
    ap.add_argument('--hybrid', action='store_true',
                    help='only time the hybrid replay on ACAS-Xu-shaped leaves (one JSON line)')
    args = ap.parse_args()
    global LOOKAHEAD
    LOOKAHEAD = {None: None, 'off': False}.get(args.lookahead, args.lookahead)
    if args.gpus != 1:
        print(f'bench.py measures one GPU only (this build has no multi-GPU path); '
              f'got --gpus {args.gpus}', file=sys.stderr)
        sys.exit(2)
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.kernels:
        kernel_suite(max(4, args.steps * 4))
        hybrid_replay_suite()
        return
    if args.hybrid:
        hybrid_replay_suite(reps=max(1, args.steps))
        return
    if args.config != 'c1':
        print(json.dumps(run_config(args.config, args.steps, args.warmup,
                                    not args.no_cpu_baseline)), flush=True)
        return

    from vibecheck_amd import _lib
    from vibecheck_amd import mlp_fused as mf
    from vibecheck_amd import verify_graph as vg
    from vibecheck_amd import workloads as wk
    from vibecheck_amd.spec import dedup_queries

    dev = torch.device('cuda:0')
    _lib.load()
    gg = wk.acas_gg(device=dev, dtype=torch.float32)
    xl0, xh0 = wk.acas_boxes(N_DOMAINS, seed=1)
    xl0, xh0 = xl0.to(dev), xh0.to(dev)
    uq, dq = dedup_queries(wk.acas_spec().as_linear_queries(5))
    se = {i: (torch.tensor(w, dtype=torch.float32, device=dev), b) for i, (w, b) in enumerate(uq)}
    table = vg.DisjunctTable(dq, dev)

    # The objects of torch's and this setup's imports go to the permanent
    # generation: otherwise the collector's first full pass over them (~45 ms,
    # about 1.5 s after start) can land inside the timed steps.  The
    # collector stays on.
    gc.collect()
    gc.freeze()
    # The shape-specialised CROWN kernels count the neurons they seed per
    # layer (one atomic per wavefront per layer), one counter row per call:
    # the work of the seeded rows depends on each domain's bounds.  The
    # warm-up runs with the same counters and HIP events as the timed steps.
    seeded = torch.zeros(max(args.steps, args.warmup) * N_ROUNDS + 8, 16, dtype=torch.int64,
                         device=dev)
    mf.SEED_COUNTER, mf.SEED_ROW = seeded, 0
    # only the large round's CROWN pass is the roofline's unit: the small
    # rounds' launches are not bracketed by events
    lib = _lib.load()
    large = lambda b: lib.vc_mlp_tiled_crown_mode(b) == 0
    when = {'vc_mlp_tiled_crown': large, 'zonotope_pass': large}
    timed_names = ['vc_mlp_crown', 'vc_mlp_tiled_crown', 'zonotope_pass']
    _lib.timing_begin(timed_names, when=when)
    for _ in range(max(1, args.warmup)):
        run_rounds(gg, xl0, xh0, se, table)
    _lib.timing_end()
    seeded.zero_()
    mf.SEED_ROW = 0
    torch.cuda.synchronize()
    _lib.timing_begin(timed_names, when=when)
    t0 = time.perf_counter()
    stats = None
    for _ in range(args.steps):
        stats = run_rounds(gg, xl0, xh0, se, table)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kt = _lib.timing_end()
    mf.SEED_COUNTER = None
    zt = kt.pop('zonotope_pass', {})
    if kt.get('vc_mlp_tiled_crown', {}).get('launches'):
        # the dominant work is the CROWN pass of the large batch (the
        # layer-synchronous rows form); the small rounds run k_crown_dom
        dims = [op['W'].shape[1] for op in gg['ops'] if op['type'] == 'fc']
        rows = seeded.tolist()
        sel = [(sec, fl + _lib.seed_flops(dims, rows[_seed_row(k, a)]))
               for k, (sec, fl, a) in enumerate(kt['vc_mlp_tiled_crown']['per_launch'])
               if lib.vc_mlp_tiled_crown_mode(a[4]) == 0]
        kt = {'vc_mlp_tiled_crown': {'launches': len(sel), 'seconds': sum(x[0] for x in sel),
                                     'flops': sum(x[1] for x in sel)}}

    per_step = wall / args.steps
    domains = sum(s['B'] for s in stats)
    entry = max(kt, key=lambda n: kt[n]['launches'])
    k = kt[entry]
    kernel = {'vc_mlp_crown': 'k_mlp_crown', 'vc_mlp_tiled_crown': 'crown_rows_pass'}[entry]
    achieved = k['flops'] / k['seconds'] / 1e12 if k['seconds'] > 0 else 0.0
    traffic, traffic_note = measured_traffic(kernel)
    roof_crown = {'kernel': (crown_kernel_name(N_DOMAINS) if entry == 'vc_mlp_tiled_crown'
                             else 'k_mlp_crown (vc_mlp_crown)')
                            + ': CROWN intermediate bounds + spec backward, fp32 MFMA',
                  'bound': 'mfma', 'achieved': achieved, 'peak': FP32_MFMA_PEAK,
                  'unit': 'TFLOP/s', 'frac': achieved / FP32_MFMA_PEAK,
                  'traffic': traffic,
                  'traffic_unit': 'bytes per launch (HBM, rocprofv3 FETCH_SIZE + WRITE_SIZE)',
                  'traffic_note': traffic_note,
                  'launches_per_step': k['launches'] / args.steps,
                  'avg_launch_us': 1e6 * k['seconds'] / max(1, k['launches']),
                  'ms_per_step': 1e3 * k['seconds'] / args.steps}
    # the zonotope passes of the 65,536-box round, timed in the same steps
    # (from an event before the native round to the CROWN pass's start):
    # sum_l 2 d_{l+1} d_l K_l FLOP per domain, K_l = 1 + n_in + the domain's
    # unstable neurons below layer l, from the round's bounds (outside the
    # timed region; the same boxes every step)
    roof_zono = None
    if zt.get('launches'):
        plan = mf.plan_for(gg, dev)
        dims, n = plan.dims, plan.n
        sbz = vz_sb(gg, xl0, xh0, dev)
        unst = torch.stack([((sbz[L][0] < 0) & (sbz[L][1] > 0)).sum(1) for L in range(n)],
                           1).double()
        below = torch.cat([torch.zeros_like(unst[:, :1]), unst.cumsum(1)[:, :-1]], 1)
        wz = torch.tensor([2.0 * dims[l + 1] * dims[l] for l in range(n)], device=dev,
                          dtype=torch.float64)
        zflop = float(((1 + dims[0] + below) * wz).sum())
        zsec = zt['seconds'] / zt['launches']
        ztraffic, znote = measured_traffic('zonotope_pass')
        roof_zono = {'kernel': 'zonotope pass (k_zono_init, k_zono_tiled, k_zono_wide_tiled for '
                               'the domains past 128 generator columns): the zonotope bounds '
                               'of every relu, fp32 MFMA',
                     'bound': 'mfma', 'achieved': zflop / zsec / 1e12, 'peak': FP32_MFMA_PEAK,
                     'unit': 'TFLOP/s', 'frac': zflop / zsec / 1e12 / FP32_MFMA_PEAK,
                     'traffic': ztraffic,
                     'traffic_unit': 'bytes per launch (HBM, rocprofv3 FETCH_SIZE + WRITE_SIZE)',
                     'traffic_note': znote,
                     'launches_per_step': zt['launches'] / args.steps,
                     'avg_launch_us': 1e6 * zsec,
                     'ms_per_step': 1e3 * zt['seconds'] / args.steps}

    # outside the timed region: the rounds' outputs once more, for the
    # domains inside the zero band and the other kernels' rooflines
    nz, secondary, alpha_rates = [None] * len(stats), None, None
    if not args.no_secondary:
        kept = []
        run_rounds(gg, xl0, xh0, se, table, keep=kept)
        nz = [near_zero(st['lb'], st['A'], st['acc'], xl, xh) for xl, xh, st in kept]
        secondary, alpha_rates = secondary_c1(gg, se, kept)
    out = {
        'metric': 'CROWN-bounded domains/sec at 1 GPU (5-50x6-5 MLP, 65,536 domains)',
        'value': domains / per_step, 'unit': 'domains/s', 'n_gpus': 1,
        'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': per_step * 1e3,
        'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None,
        'dtype': 'f32', 'data': 'synthetic (seeded boxes and Kaiming-normal weights)',
        'config': {'workload': '5-50x6-5 ReLU MLP, 65,536 input boxes, 3 BaB rounds, '
                               'CROWN intermediate + alpha-CROWN 20 it lr 0.1 + clip + '
                               'widest split', 'domains_per_step': domains,
                   'lookahead': _lookahead_mode()},
        'alpha_iters_per_s': alpha_rates['open']['iters_per_s'] if alpha_rates else None,
        'alpha': ({'step_open_leaves': alpha_rates['open'], 'all_65536': alpha_rates['all']}
                  if alpha_rates else None),
        'rounds': [dict(s, near_zero=z) for s, z in zip(stats, nz)],
        # the work that takes the most time per step (both timed live)
        'roofline': (roof_zono if roof_zono is not None
                     and roof_zono['ms_per_step'] >= roof_crown['ms_per_step'] else roof_crown),
        'rooflines_timed': [r for r in (roof_zono, roof_crown) if r is not None],
        'secondary': secondary,
    }
    if not args.no_cpu_baseline:
        out['cpu_baseline'] = cpu_baseline_c1(args.cpu_reps)
    if not args.no_configs:
        # the parity-test configurations, each one line as with --config
        out['configs'] = {}
        for cfg in ('c0', 'c2', 'c3', 'c4'):
            print(f'bench: configuration {cfg}', file=sys.stderr, flush=True)
            out['configs'][cfg] = run_config(cfg, args.steps, args.warmup,
                                             not args.no_cpu_baseline)
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()
