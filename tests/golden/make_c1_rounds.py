"""Writes tests/golden/c1_rounds.npz: the oracle's three input-split BaB
rounds on the 65,536-box ACAS-Xu-shaped workload (5-50x6-5 ReLU MLP,
seeded weights and boxes; CROWN intermediate bounds, clip, alpha-CROWN 20
iterations at lr 0.1 / decay 0.98 on every unclosed leaf, widest-dimension
bisection), as `bench.py` runs them.  Round r + 1 starts from round r's
children in the worklist's pop order (the high chunk, then the low chunk).

The oracle takes about two minutes per 65,536-box round on eight host
threads, far too long for a GPU test, so its results are kept here.  The
first round's boxes are regenerated from their seed by the test; later
rounds' boxes are the stored children.

Per round the file holds (prefix r<k>_):
  B                 batch size
  closed            packed closure verdicts after alpha (B bits)
  crown_closed      packed closure verdicts of the CROWN bound (B bits)
  near0             packed flags: some spec row's CROWN bound within the
                    bound tolerance of 0, |lb| <= 1e-6 + 1e-5 scale with
                    scale = |acc| + sum_i |A_i| max(|xl_i|, |xh_i|)
  crown_lb          the CROWN pass's spec bounds of every box, (B, Q)
  sub               a seeded subset of at most 4,096 boxes, int32 ascending
  sub_A, sub_acc    the CROWN pass's input linearization on those boxes,
                    (n, Q, 5) and (n, Q)
  sub_A64           the same A from the oracle in fp64 on the same (fp32)
                    boxes, (n, Q, 5) float64
  alpha_idx         the alpha-CROWN leaves (CROWN-unclosed), int32
  alpha_lb          their bounds after the max-merge with alpha, (n, Q)
  alpha_scale       the scale above for those rows, (n, Q)
  n_alpha_iters     alpha's evaluated iterations (global early stop)
  unclosed          leaves open after alpha, int32
  feasible          their clip feasibility, bool
  xl_split/xh_split the clipped boxes of the feasible leaves
  ax                their split dimensions, int8
  low_xl/low_xh/high_xl/high_xh  the children

Run from the repository root:  python tests/golden/make_c1_rounds.py
"""
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
for _p in (ROOT, os.path.join(ROOT, 'vibecheck-nn_amd')):
    if _p not in sys.path:
        sys.path.insert(0, _p)

from oracle import ref_bab  # noqa: E402
from vibecheck_amd import workloads as wk  # noqa: E402
from vibecheck_amd.spec import dedup_queries  # noqa: E402

N_DOMAINS = 65536
N_ROUNDS = 3
ALPHA_ITERS = 20
ALPHA_LR = 0.1
RTOL, ATOL = 1e-5, 1e-6
N_SUB = 4096
OUT = os.environ.get('C1_ROUNDS_OUT') or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                     'c1_rounds.npz')


def spec_scale(A, acc, xl, xh):
    xm = torch.maximum(xl.double().abs(), xh.double().abs())
    return acc.double().abs() + (A.double().abs() * xm.unsqueeze(1)).sum(-1)


def main():
    torch.set_num_threads(os.cpu_count() or 1)
    gg = wk.acas_gg(dtype=torch.float32)
    xl, xh = wk.acas_boxes(N_DOMAINS, seed=1)
    uq, dq = dedup_queries(wk.acas_spec().as_linear_queries(5))
    se = {i: (torch.tensor(w, dtype=torch.float32), b) for i, (w, b) in enumerate(uq)}
    gg64 = wk.acas_gg(dtype=torch.float64)
    se64 = {i: (torch.tensor(w, dtype=torch.float64), b) for i, (w, b) in enumerate(uq)}
    out = {'n_rounds': np.int64(N_ROUNDS)}
    for r in range(N_ROUNDS):
        t0 = time.perf_counter()
        B = xl.shape[0]
        st = ref_bab.bab_step(xl, xh, gg, se, dq, crown_intermediate=True, clip_enabled=True,
                              alpha_iters=ALPHA_ITERS, alpha_all=True, alpha_lr=ALPHA_LR)
        lb_c, crown_closed = st['crown_lb'], st['crown_closed']
        scale = spec_scale(st['A'], st['acc'], xl, xh)
        near0 = ((lb_c.double().abs() <= ATOL + RTOL * scale).any(1))
        aidx = (~crown_closed).nonzero(as_tuple=True)[0]
        p = f'r{r}_'
        out[p + 'B'] = np.int64(B)
        out[p + 'closed'] = np.packbits(st['closed'].numpy())
        out[p + 'crown_closed'] = np.packbits(crown_closed.numpy())
        out[p + 'near0'] = np.packbits(near0.numpy())
        out[p + 'crown_lb'] = lb_c.numpy().astype(np.float32)
        g = torch.Generator().manual_seed(100 + r)
        sub = (torch.randperm(B, generator=g)[:N_SUB].sort().values if B > N_SUB
               else torch.arange(B))
        out[p + 'sub'] = sub.numpy().astype(np.int32)
        out[p + 'sub_A'] = st['A'][sub].numpy().astype(np.float32)
        out[p + 'sub_acc'] = st['acc'][sub].numpy().astype(np.float32)
        _, A64, _ = ref_bab.bound_batch(xl[sub].double(), xh[sub].double(), gg64, se64)
        out[p + 'sub_A64'] = A64.numpy()
        out[p + 'alpha_idx'] = aidx.numpy().astype(np.int32)
        out[p + 'alpha_lb'] = st['lb'][aidx].numpy().astype(np.float32)
        out[p + 'alpha_scale'] = scale[aidx].numpy().astype(np.float32)
        out[p + 'n_alpha_iters'] = np.int64(st['n_alpha_iters'])
        out[p + 'unclosed'] = st['unclosed'].numpy().astype(np.int32)
        out[p + 'feasible'] = st['feasible'].numpy()
        out[p + 'xl_split'] = st['xl_split'].numpy()
        out[p + 'xh_split'] = st['xh_split'].numpy()
        out[p + 'ax'] = st['ax'].numpy().astype(np.int8)
        (lxl, lxh), (hxl, hxh) = st['low'], st['high']
        out[p + 'low_xl'], out[p + 'low_xh'] = lxl.numpy(), lxh.numpy()
        out[p + 'high_xl'], out[p + 'high_xh'] = hxl.numpy(), hxh.numpy()
        print(f'round {r}: B={B} closed={int(st["closed"].sum())} '
              f'crown_closed={int(crown_closed.sum())} near0={int(near0.sum())} '
              f'alpha_leaves={st["n_alpha_leaves"]} alpha_iters={st["n_alpha_iters"]} '
              f'feasible={int(st["feasible"].sum())} children={2 * lxl.shape[0]} '
              f'({time.perf_counter() - t0:.1f} s)', flush=True)
        # the next round pops the whole worklist: the high chunk, then the low
        xl = torch.cat([hxl, lxl], 0).contiguous()
        xh = torch.cat([hxh, lxh], 0).contiguous()
    np.savez_compressed(OUT, **out)
    print(f'wrote {OUT} ({os.path.getsize(OUT)} bytes)')


if __name__ == '__main__':
    main()
