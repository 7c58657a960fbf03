"""The C-ABI library loads on the CPU host and exports every entry point
declared in include/*.h; the ctypes table matches the declarations."""
import ctypes
import glob
import os
import re

import pytest

from vibecheck_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = {}
    for h in glob.glob(os.path.join(ROOT, 'include', '*.h')):
        text = open(h).read()
        text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
        for m in re.finditer(r'\b(int|int64_t)\s+(vc_\w+)\s*\(([^)]*)\)\s*;', text):
            args = [a for a in m.group(3).split(',') if a.strip() and a.strip() != 'void']
            names[m.group(2)] = len(args)
    return names


def test_header_declares_entry_points():
    assert len(_declared()) >= 30


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail('libvibecheck_amd.so is not built (run __graft_entry__.build())')
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_table_matches_header():
    decl = _declared()
    assert set(decl) == set(_lib.SIGNATURES), set(decl) ^ set(_lib.SIGNATURES)
    for name, nargs in decl.items():
        assert len(_lib.SIGNATURES[name]) == nargs, name


def test_abi_version_callable_without_gpu():
    lib = _lib.load()
    assert lib.vc_abi_version() == 1


def test_argument_errors_map_to_exceptions():
    # null pointers are rejected before any launch: no GPU needed
    with pytest.raises(ValueError):
        _lib.call('vc_make_slopes', None, None, 4, None, None, None, None,
                  None, None, None)
    lib = _lib.load()
    assert lib.vc_compact_workspace(1 << 20) >= 8


def test_work_accounting_closed_forms():
    """Flop accounting of the whole-network CROWN launches: a 2-layer chain
    worked by hand, and the per-layer seed totals of the shape-specialised
    kernel (union seeding: B * cnt[L]) giving the same figure as the
    argument-based count of the untiled kernel."""
    dims = [3, 4, 5]
    # fc_0: 2*3*4 = 24 per row, fc_1: 2*4*5 = 40 per row.
    # layer 1 seeds 2 neurons -> 4 rows through fc_0; Q = 2 spec rows
    # through fc_1, fc_0; B = 7 domains.
    want = 7 * (4 * 24 + 2 * (24 + 40))
    assert _lib.mlp_crown_flops(dims, 2, 7, [0, 2], 1, 2) == want
    cnt = [5, 3]
    B, Q = 11, 4
    full = _lib.mlp_crown_flops(dims, 2, B, cnt, 1, Q)
    spec = _lib.mlp_crown_flops(dims, 2, B, [0, 0], 0, Q)
    assert spec + _lib.seed_flops(dims, [B * c for c in cnt] + [0] * 14) == full


def test_zono_wide_capacity_matches_header():
    text = open(os.path.join(ROOT, 'include', 'vibecheck_amd.h')).read()
    m = re.search(r'#define VC_ZONO_WIDE_COLS (\d+)', text)
    assert m and int(m.group(1)) == _lib.VC_ZONO_WIDE_COLS


def test_round_handoff_offsets_layout():
    """The handed-over spec bound, A and acc of B children inside la_work:
    each array 256-byte aligned, in that order and back to back (sizes
    rounded up to 256 bytes), so a caller can point a round's lb, A and
    acc there; host arithmetic only."""
    dims = (ctypes.c_int32 * 8)(5, 50, 50, 50, 50, 50, 50, 5)
    for B, Q in ((810, 4), (1, 1), (65536, 9)):
        off = (ctypes.c_int64 * 3)()
        _lib.call('vc_mlp_bab_round_handoff_offsets', ctypes.addressof(dims), 6, B, Q,
                  ctypes.addressof(off))
        up = lambda nbytes: (nbytes + 255) // 256 * 256
        assert list(off) == [0, up(4 * B * Q), up(4 * B * Q) + up(4 * B * Q * 5)], (B, Q)
    with pytest.raises(ValueError):
        _lib.call('vc_mlp_bab_round_handoff_offsets', ctypes.addressof(dims), 6, 4, 0,
                  ctypes.addressof(off))
