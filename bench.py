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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=5)
    ap.add_argument('--warmup', type=int, default=2)
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--cpu-sample', type=int, default=2048)
    ap.add_argument('--copy-probe', type=int, default=0, metavar='MIB',
                    help='only run a plain copy of MIB MiB (counter calibration)')
    args = ap.parse_args()
    if args.gpus != 1:
        print(f'bench.py measures one GPU only (this build has no multi-GPU path); '
              f'got --gpus {args.gpus}', file=sys.stderr)
        sys.exit(2)
    if args.copy_probe:
        copy_probe(args.copy_probe)
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
