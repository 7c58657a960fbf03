import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, 'vibecheck-nn_amd')):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line(
        'markers', 'gpu: needs an MI355X GPU and the built HIP library')


@pytest.fixture(scope='session')
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.fail('GPU test run without a visible GPU')
    from vibecheck_amd import _lib
    _lib.load()
    return torch.device('cuda:0')


def pytest_terminal_summary(terminalreporter):
    """The escape counts of the GPU bound comparisons (entries within the
    tolerance only relative to their scale, or only as close to fp64 as the
    fp32 oracle), summed over the run."""
    mod = sys.modules.get('test_gpu_parity')
    esc = getattr(mod, 'ESCAPES', None)
    if not esc:
        _c1_summary(terminalreporter)
        return
    n = sum(e[3] for e in esc)
    n_sc = sum(e[1] for e in esc)
    n_64 = sum(e[2] for e in esc)
    worst = max(esc, key=lambda e: (e[1] + e[2]) / max(1, e[3]))
    terminalreporter.write_line(
        f'bound comparisons: {len(esc)} calls, {n} entries; escapes: {n_sc} by scale, '
        f'{n_64} by fp64 ({100.0 * (n_sc + n_64) / max(1, n):.4f}%); worst call '
        f'{worst[0]!r}: {worst[1] + worst[2]} of {worst[3]}')
    _c1_summary(terminalreporter)


def _c1_summary(terminalreporter):
    """The C1 workload's comparison counts per round (test_gpu_c1_rounds)."""
    mod = sys.modules.get('test_gpu_c1_rounds')
    stats = getattr(mod, 'C1_STATS', None)
    if not stats:
        return
    for r, (B, fc, ff, esc, esc_a, na, n5, n54, nf, nb) in enumerate(stats):
        terminalreporter.write_line(
            f'C1 round {r}: B={B}, closure flips in the zero band: CROWN {fc}, final {ff}; '
            f'escapes: CROWN lb {esc}, A {esc_a}; alpha on {na} leaves, '
            f'entries within 1e-5: {n5}, 1e-5..1e-4: {n54}, beyond 1e-4: {nf}; {nb} '
            f'both-open feasible leaves')
