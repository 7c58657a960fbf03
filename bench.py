"""Benchmark: CROWN-bounded domains/s on the 5-50x6-5 ReLU MLP.

One step = three input-split BaB rounds starting from 65,536 seeded boxes
(centres U[-1,1]^5, half-widths U[0.005,0.05]): per round CROWN
intermediate bounds, CROWN spec bounds with input linearization, closure,
alpha-CROWN (20 Adam iterations, lr 0.1, decay 0.98) on every unclosed
leaf, one halfspace clip, widest-dimension bisection; the children are the
next round's batch.  value = domains bounded / wall time of the step.

Prints one JSON line (rank 0).  Extra keys: roofline (dominant kernel,
measured with HIP events on the launch stream), cpu_baseline (CPU oracle on
a bounded sample of the same workload), alpha_iters_per_s, rounds.
"""
import argparse
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


def run_rounds(gg, xl, xh, spec_ew, table, timers=None):
    """Three BaB rounds; returns per-round stats."""
    from vibecheck_amd import verify_graph as vg
    stats = []
    for _ in range(N_ROUNDS):
        B = xl.shape[0]
        if B == 0:
            stats.append({'B': 0, 'closed': 0, 'alpha_leaves': 0, 'alpha_iters': 0})
            continue
        st = vg.bab_step(xl, xh, gg, spec_ew, table, crown_intermediate=True,
                         clip_enabled=True, alpha_iters=ALPHA_ITERS, alpha_all=True,
                         alpha_lr=ALPHA_LR, timers=timers)
        (lxl, lxh), (hxl, hxh) = st['low'], st['high']
        # next batch = the LIFO pop of [low chunk, high chunk]: high first
        xl = torch.cat([hxl, lxl], 0)
        xh = torch.cat([hxh, lxh], 0)
        stats.append({'B': B, 'closed': B - int(st['unclosed'].numel()),
                      'alpha_leaves': st['n_alpha_leaves'],
                      'alpha_iters': st['n_alpha_iters']})
    return stats


def cpu_baseline(sample_B=2048, reps=3):
    """Oracle (op-for-op torch CPU restatement) on one BaB round of a
    sample_B-box slice of the same workload, all host threads."""
    from oracle import ref_bab
    from vibecheck_amd import workloads as wk
    from vibecheck_amd.spec import dedup_queries
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    gg = wk.acas_gg(dtype=torch.float32)
    xl, xh = wk.acas_boxes(N_DOMAINS, seed=1)
    xl, xh = xl[:sample_B].contiguous(), xh[:sample_B].contiguous()
    uq, dq = dedup_queries(wk.acas_spec().as_linear_queries(5))
    se = {i: (torch.tensor(w, dtype=torch.float32), b) for i, (w, b) in enumerate(uq)}
    ts = []
    for r in range(reps + 1):
        t0 = time.perf_counter()
        ref_bab.bab_step(xl, xh, gg, se, dq, crown_intermediate=True, clip_enabled=True,
                         alpha_iters=ALPHA_ITERS, alpha_all=True, alpha_lr=ALPHA_LR)
        if r > 0:
            ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    return {'value': sample_B / t, 'unit': 'domains/s', 'cores': cores, 'kind': 'port',
            'sample': f'one BaB round (CROWN-intermediate, spec bound, alpha 20 it, clip, '
                      f'split) on the first {sample_B} of the 65,536 boxes, median of {reps}'}


def measured_traffic(kernel):
    """HBM bytes per launch of the dominant kernel on this workload, from the
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (each counter scaled
    by what it reads for a plain copy of known size); None when absent."""
    path = os.path.join(ROOT, 'profiles', f'{kernel}_acas_65536_traffic.md')
    try:
        with open(path) as f:
            for line in f:
                if line.startswith('traffic_bytes_per_launch:'):
                    return float(line.split(':', 1)[1])
    except OSError:
        pass
    return None


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
    from vibecheck_amd._lib import call, ptr, stream

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
        kern = 'k_concretize_thread' if n_in <= 32 else 'k_concretize_wave'
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
        for kern, r in (('k_relax_rows + gemm_kernel (two-phase backward fc)', rel),
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
        fn = lambda: call('vc_backward_conv', ptr(ew), M, ptr(K), ptr(bias), C_out, Ho, Ho, C_in,
                          H, H, k, k, cs, cs, cp, cp, ptr(out), ptr(acc), st)
        kern = ('k_conv_t_smallc' if C_in <= 4 else
                'gemm_kernel (transposed conv, implicit GEMM)') + ' + k_conv_bias_dot'
        report('a7', kern,
               f'conv {C_in}->{C_out} {k}x{k} s{cs} p{cp} ({H}x{H} in), 576 rows '
               '(64 domains x 9)', _time_launches([fn], max(3, reps // 4)), 'mfma',
               2.0 * M * (C_out * Ho * Ho) * (C_in * k * k))
        del ew, out, acc

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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=5)
    ap.add_argument('--warmup', type=int, default=2)
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--cpu-sample', type=int, default=2048)
    ap.add_argument('--copy-probe', type=int, default=0, metavar='MIB',
                    help='only run a plain copy of MIB MiB (counter calibration)')
    ap.add_argument('--kernels', action='store_true',
                    help='only time the layer-wise kernels one at a time (one JSON line each)')
    ap.add_argument('--hybrid', action='store_true',
                    help='only time the hybrid replay on ACAS-Xu-shaped leaves (one JSON line)')
    args = ap.parse_args()
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

    for _ in range(args.warmup):
        run_rounds(gg, xl0, xh0, se, table)
    torch.cuda.synchronize()

    # The shape-specialised CROWN kernels count the neurons they seed per
    # layer (one atomic per wavefront per layer), one counter row per call:
    # the work of the seeded rows depends on each domain's bounds.
    seeded = torch.zeros(args.steps * N_ROUNDS + 8, 16, dtype=torch.int64, device=dev)
    mf.SEED_COUNTER, mf.SEED_ROW = seeded, 0
    _lib.timing_begin(['vc_mlp_crown', 'vc_mlp_tiled_crown'])
    t0 = time.perf_counter()
    stats = None
    for _ in range(args.steps):
        stats = run_rounds(gg, xl0, xh0, se, table)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kt = _lib.timing_end()
    mf.SEED_COUNTER = None
    if kt.get('vc_mlp_tiled_crown', {}).get('launches'):
        # the dominant kernel is k_crown_tiled, the one-wavefront-per-domain
        # kernel of the large batches; the small rounds run k_crown_dom
        lib = _lib.load()
        dims = [op['W'].shape[1] for op in gg['ops'] if op['type'] == 'fc']
        rows = seeded.tolist()
        sel = [(sec, fl + _lib.seed_flops(dims, rows[k]))
               for k, (sec, fl, a) in enumerate(kt['vc_mlp_tiled_crown']['per_launch'])
               if lib.vc_mlp_tiled_crown_mode(a[4]) == 0]
        kt = {'vc_mlp_tiled_crown': {'launches': len(sel), 'seconds': sum(x[0] for x in sel),
                                     'flops': sum(x[1] for x in sel)}}

    per_step = wall / args.steps
    domains = sum(s['B'] for s in stats)
    alpha_iters = sum(s['alpha_iters'] for s in stats)
    entry = max(kt, key=lambda n: kt[n]['launches'])
    k = kt[entry]
    kernel = {'vc_mlp_crown': 'k_mlp_crown', 'vc_mlp_tiled_crown': 'k_crown_tiled'}[entry]
    achieved = k['flops'] / k['seconds'] / 1e12 if k['seconds'] > 0 else 0.0
    out = {
        'metric': 'CROWN-bounded domains/sec at 1 GPU (5-50x6-5 MLP, 65,536 domains)',
        'value': domains / per_step, 'unit': 'domains/s', 'n_gpus': 1,
        'steps': args.steps, 'warmup': args.warmup, 'ms_per_step': per_step * 1e3,
        'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None,
        'dtype': 'f32', 'data': 'synthetic (seeded boxes and Kaiming-normal weights)',
        'config': {'workload': '5-50x6-5 ReLU MLP, 65,536 input boxes, 3 BaB rounds, '
                               'CROWN intermediate + alpha-CROWN 20 it lr 0.1 + clip + '
                               'widest split', 'domains_per_step': domains},
        'alpha_iters_per_s': alpha_iters / per_step,
        'rounds': stats,
        'roofline': {'kernel': f'{kernel} ({entry}: CROWN intermediate bounds + spec '
                               'backward, whole network per wavefront, fp32 MFMA)',
                     'bound': 'mfma', 'achieved': achieved, 'peak': FP32_MFMA_PEAK,
                     'unit': 'TFLOP/s', 'frac': achieved / FP32_MFMA_PEAK,
                     'traffic': measured_traffic(kernel),
                     'traffic_unit': 'bytes per launch (HBM, rocprofv3 FETCH_SIZE + WRITE_SIZE)',
                     'launches_per_step': k['launches'] / args.steps,
                     'avg_launch_us': 1e6 * k['seconds'] / max(1, k['launches'])},
    }
    if not args.no_cpu_baseline:
        out['cpu_baseline'] = cpu_baseline(args.cpu_sample)
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()
