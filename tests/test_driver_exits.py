"""The input-split driver's exits (verify_graph.py:12834-13464), host logic
only: the step is replaced by a stand-in that raises or returns what a
case needs, so these run without a GPU.

  - a RuntimeError or OOM in a step halves the batch size and retries the
    popped batch (12872-12897); at batch size 1 an OOM is re-raised unless
    raise_on_oom is off, and anything else ends 'unknown' / batched_oom;
  - the worklist overflow exit after a push (13424-13429);
  - the timeout exit before a pop (12836-12838);
  - degenerate leaves (no usable split width) left open: 'unknown' even
    with an empty worklist (13366-13369, 13452-13464);
  - the details keys of every exit are the reference's.
"""
import pytest
import torch

from vibecheck_amd import verify_graph as vg
from vibecheck_amd import workloads as wk

VERIFIED_KEYS = {'phase', 'batched_n_leaves', 'batched_n_iters', 'batched_batch_size'}
TIMEOUT_KEYS = {'phase', 'batched_n_leaves', 'batched_n_iters', 'batched_worklist_left',
                'batched_open_degenerate', 'batched_batch_size'}
OVERFLOW_KEYS = {'phase', 'batched_n_leaves', 'batched_n_iters', 'worklist_size'}
OOM_KEYS = {'phase', 'batch_size'}


class Steps:
    """Stand-in for bab_step: ``plan(call_no, B)`` returns 'close', 'split',
    'degenerate' or an exception to raise."""

    def __init__(self, plan):
        self.plan = plan
        self.calls = []

    def __call__(self, xl, xh, gg, spec_ew, table, *args, **kw):
        B = xl.shape[0]
        self.calls.append((B, kw.get('clip_iters')))
        what = self.plan(len(self.calls), B)
        if isinstance(what, BaseException):
            raise what
        out = {'n_degenerate': 0, 'chunks': []}
        if what == 'split':
            mid = (xl + xh) / 2
            out['chunks'] = [(xl, mid), (mid, xh)]
        elif what == 'degenerate':
            out['n_degenerate'] = B
        return out


@pytest.fixture
def driver(monkeypatch):
    # the output-width probe is the only other device call of the driver
    monkeypatch.setattr(vg, '_forward_zonotope_graph_batched',
                        lambda xl, xh, gg, dev, dt: ({}, (torch.zeros(1, 5), None)))

    def run(plan, **settings):
        steps = Steps(plan)
        monkeypatch.setattr(vg, 'bab_step', steps)
        spec = wk.acas_spec([0.0] * 5, [0.1] * 5)
        s = {'input_split_batch_size': 4096, 'total_timeout': 60.0}
        s.update(settings)
        verdict, det = vg._input_split_batched(None, spec, s, {}, 'cpu', torch.float32)
        return verdict, det, steps.calls
    return run


def test_oom_once_halves_the_batch_and_retries(driver):
    oom = torch.cuda.OutOfMemoryError('test')
    verdict, det, calls = driver(lambda k, B: oom if k == 1 else 'close')
    assert verdict == 'verified' and set(det) == VERIFIED_KEYS
    assert det['batched_batch_size'] == 2048
    assert det['batched_n_leaves'] == 1 and det['batched_n_iters'] == 1
    assert [B for B, _ in calls] == [1, 1]


def test_runtime_error_halves_down_to_one_then_unknown(driver):
    verdict, det, calls = driver(lambda k, B: RuntimeError('launch failed'))
    assert verdict == 'unknown' and det == {'phase': 'batched_oom', 'batch_size': 1}
    # 4096, 2048, ..., 2, 1: thirteen attempts
    assert len(calls) == 13


def test_not_implemented_is_a_runtime_error_too(driver):
    # the reference's `except (OutOfMemoryError, RuntimeError)` also takes
    # NotImplementedError, a RuntimeError subclass
    verdict, det, _ = driver(lambda k, B: NotImplementedError('op'),
                             input_split_batch_size=4)
    assert verdict == 'unknown' and det == {'phase': 'batched_oom', 'batch_size': 1}


def test_oom_at_batch_one_is_raised_unless_tolerated(driver):
    oom = torch.cuda.OutOfMemoryError('test')
    with pytest.raises(torch.cuda.OutOfMemoryError):
        driver(lambda k, B: oom, input_split_batch_size=2)
    verdict, det, calls = driver(lambda k, B: oom, input_split_batch_size=2, raise_on_oom=False)
    assert verdict == 'unknown' and det == {'phase': 'batched_oom', 'batch_size': 1}
    assert set(det) == OOM_KEYS and len(calls) == 2


def test_worklist_overflow_exit(driver):
    verdict, det, calls = driver(lambda k, B: 'split', input_split_batched_max_worklist=3)
    # root -> 2 children (size 2), then both popped -> 4 children > 3
    assert verdict == 'unknown' and set(det) == OVERFLOW_KEYS
    assert det['phase'] == 'batched_worklist_overflow'
    assert det['batched_n_leaves'] == 3 and det['batched_n_iters'] == 2
    assert det['worklist_size'] == 4
    assert [B for B, _ in calls] == [1, 2]


def test_timeout_exit_before_any_pop(driver):
    verdict, det, calls = driver(lambda k, B: 'close', total_timeout=0.0)
    assert verdict == 'unknown' and set(det) == TIMEOUT_KEYS
    assert det['phase'] == 'batched_timeout'
    assert det['batched_worklist_left'] == 1 and det['batched_open_degenerate'] == 1
    assert det['batched_n_leaves'] == 0 and det['batched_n_iters'] == 0
    assert calls == []


def test_degenerate_leaves_keep_the_run_open(driver):
    verdict, det, calls = driver(lambda k, B: 'split' if k == 1 else 'degenerate')
    assert verdict == 'unknown' and set(det) == TIMEOUT_KEYS
    assert det['phase'] == 'batched_timeout'
    assert det['batched_worklist_left'] == 0 and det['batched_open_degenerate'] == 2
    assert det['batched_n_leaves'] == 3 and det['batched_n_iters'] == 2


def test_clip_iters_setting_reaches_the_step(driver):
    _, _, calls = driver(lambda k, B: 'close', input_split_batched_clip_iters=4)
    assert calls == [(1, 4)]
    _, _, calls = driver(lambda k, B: 'close')
    assert calls == [(1, 1)]


def test_errors_after_the_bound_phase_propagate(driver):
    """The reference's try covers the bound phase only (verify_graph.py:
    12853-12897): a clip- or split-phase error (the step tags it with
    vc_phase) ends the run with that error instead of halving the batch."""
    for phase in ('clip', 'split'):
        err = vg._tag_phase(RuntimeError('clip kernel failed'), phase)
        assert err.vc_phase == phase
        with pytest.raises(RuntimeError, match='clip kernel failed'):
            driver(lambda k, B: err)
    # an error tagged once keeps its first phase
    err = vg._tag_phase(vg._tag_phase(RuntimeError('x'), 'split'), 'clip')
    assert err.vc_phase == 'split'
    # untagged (bound phase): halves as before
    verdict, det, calls = driver(lambda k, B: RuntimeError('bound'), input_split_batch_size=4)
    assert verdict == 'unknown' and len(calls) == 3


def test_worklist_pop_joins_adjacent_chunks_without_copy():
    """The product worklist pops [high, low] chunks that lie back to back in
    one storage (the native round's layout) as a view of that block, with
    the values torch.cat would give; chunks elsewhere are concatenated, and
    the LIFO order (verify_graph.py:12695-12726) holds either way."""
    blk = torch.arange(40, dtype=torch.float32)
    high, low = blk[:12].view(3, 4), blk[12:20].view(2, 4)
    other = torch.arange(100, 108, dtype=torch.float32).view(2, 4)
    wl = vg.ChunkWorklist(torch.zeros(4), torch.ones(4))
    wl.pop(1)
    wl.push(low, low)
    wl.push(high, high)
    xl, xh = wl.pop(5)
    assert torch.equal(xl, torch.cat([high, low], 0)) and torch.equal(xh, xl)
    assert xl.untyped_storage().data_ptr() == blk.untyped_storage().data_ptr()
    assert not wl
    # a partial pop takes the lower chunk's last rows, which do not follow
    # the upper chunk: concatenated
    wl.push(other, other)
    wl.push(low, low)
    wl.push(high, high)
    xl, _ = wl.pop(4)
    assert xl.tolist() == torch.cat([high, low[-1:]], 0).tolist()
    assert xl.untyped_storage().data_ptr() != blk.untyped_storage().data_ptr()
    xl, _ = wl.pop(3)
    assert xl.tolist() == torch.cat([low[:1], other], 0).tolist()
    assert not wl
