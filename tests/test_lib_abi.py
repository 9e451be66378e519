"""CPU-side checks of the C-ABI library: it is built, loads, and exports every entry point include/treeattn.h
declares (no compute calls: there is no GPU here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, 'include', 'treeattn.h')


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(ta_[a-z_0-9]+)\s*\(', text)))


def test_header_declares_entry_points():
    names = declared_functions()
    for n in ('ta_level_sums', 'ta_tree_descend', 'ta_gather_dot', 'ta_gather_dot_blocks', 'ta_sparse_attn_fwd',
              'ta_seg_attn_fwd', 'ta_kv_append', 'ta_last_error', 'ta_abi_version'):
        assert n in names


def test_library_exports_every_declared_symbol():
    import torch  # noqa: F401  (the library binds to the HIP runtime torch loads)
    from treeattn_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail('libtreeattn.so is not built (python -m treeattn_amd.build)')
    L = _lib.lib()
    for n in declared_functions():
        assert hasattr(L, n), n
    assert set(_lib.SIGNATURES) == set(declared_functions())
    assert L.ta_abi_version() == 3


def test_build_entry_checks_the_declared_abi_version():
    """__graft_entry__.build() compares the library's ABI version with the one include/treeattn.h declares (no
    number of its own to fall behind the header); the built library matches it."""
    import torch  # noqa: F401
    from treeattn_amd import _lib
    src = open(os.path.join(ROOT, '__graft_entry__.py')).read()
    assert 'TA_ABI_VERSION' in src and 'ta_abi_version() == ' not in src
    declared = int(re.search(r'#define TA_ABI_VERSION (\d+)', open(HEADER).read()).group(1))
    assert _lib.lib().ta_abi_version() == declared


def test_library_rejects_bad_arguments_without_gpu():
    """Argument validation runs on the host: a bad size returns an error code and a message."""
    import torch  # noqa: F401
    from treeattn_amd import _lib
    L = _lib.lib()
    rc = L.ta_tree_descend(None, 0, 0, 0, 0, 1, 1, 4, 64, None, 0, 0, None, None, None, 100, 1, 1, 4, 4,
                           None, None, None, None)
    assert rc == 1
    assert b'bad sizes' in L.ta_last_error()
    rc = L.ta_seg_attn_fwd(None, None, None, 2, 0, 0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 1, 64, 64, None, 0, None, None, None, 4,
                           64, 200, 0.1, None, 0, 0, 0, None, None, 1, None, 0, None, None)
    assert rc == 2
    assert b'local window' in L.ta_last_error()
    # candidate rows wider than 320 entries (leaf 4 x 64 leaves + 128 neighbour keys + 4 static keys + 4 own keys)
    import ctypes
    one = ctypes.c_void_p(8)   # never dereferenced: the sizes are refused first
    rc = L.ta_assemble_candidates(one, one, one, one, one, 0, 1, 1, 8, 64, 4, 128, 3, one, one, None)
    assert rc == 1
    assert b'at most 320 candidates' in L.ta_last_error()
    # LaneTree workspace: T a power of two in [4, 262144], chunk dividing T, head size 16 / 32 / 64 / 128
    nb = ctypes.c_int64(0)
    assert L.ta_lanetree_workspace_size(1, 6, 131072, 64, 4096, ctypes.byref(nb)) == 0
    assert nb.value == 6 * 32 * 131072 * (64 * 4 + 8)
    assert L.ta_lanetree_workspace_size(2, 3, 4096, 128, 64, ctypes.byref(nb)) == 0
    assert nb.value == 2 * 3 * 64 * 4096 * (128 * 4 + 8)
    for bad in [(1, 1, 100, 64, 4), (1, 1, 524288, 64, 4096), (1, 1, 4096, 48, 64), (1, 1, 4096, 64, 48),
                (1, 1, 2, 16, 1), (0, 1, 4096, 64, 64)]:
        assert L.ta_lanetree_workspace_size(*bad, ctypes.byref(nb)) == 1, bad
        assert b'ta_lanetree_workspace_size' in L.ta_last_error()


def test_product_refuses_cpu_tensors():
    import torch
    from treeattn_amd import kernels
    q = torch.zeros(1, 1, 4, 64)
    with pytest.raises(RuntimeError, match='GPU'):
        kernels.gather_dot(q, q, torch.zeros(1, 1, 4, 2, dtype=torch.long), 1.0)


def test_backward_route_choice():
    """The default dk/dv route: the fixed-order (bit-reproducible) scan while its candidate-row reads stay within
    DKDV_SCAN_LIMIT, the atomic adds beyond (the scan is quadratic in T).  Causal scans skip the queries before a
    key block: sum over blocks of (T - block start) rows."""
    from treeattn_amd import kernels as K
    # T = 512, D = 64 (blocks of 64 keys), KC = 100: 8 blocks x 512 rows, or 512 + 448 + ... + 64 causally
    assert K.dkdv_scan_ints(1, 1, 512, 512, 100, 64, False) == 8 * 512 * 100
    assert K.dkdv_scan_ints(1, 1, 512, 512, 100, 64, True) == sum(512 - 64 * j for j in range(8)) * 100
    assert K.dkdv_scan_ints(2, 6, 512, 512, 100, 64, True) <= K.DKDV_SCAN_LIMIT          # the reference's size
    assert K.dkdv_scan_ints(1, 16, 16384, 16384, 2100, 128, True) > K.DKDV_SCAN_LIMIT    # config 3's shape


def test_tracing_builds_are_separate():
    """The phase marks are nothing in the library build: it exports no trace buffer accessor, and a tracing build
    of one source lives in its own library beside it."""
    from treeattn_amd import _lib, build, phase_trace  # noqa: F401
    L = _lib.lib()
    assert not hasattr(L, 'ta_trace_read')
    assert build.trace_lib_path('attend.hip') != _lib.LIB_PATH
    assert build.trace_lib_path('attend.hip').endswith('libtreeattn_trace_attend.so')
