"""The C ABI: libveda_hip.so loads, exports every entry point declared in
include/veda_hip.h with the arity the ctypes binding uses, and rejects bad
arguments on the host before any launch (these paths make no HIP call, so
they run without a GPU)."""

import ctypes
import pathlib
import re
import threading

import pytest

from miowtion_amd import _native

HEADER = pathlib.Path(__file__).resolve().parent.parent / 'include' / 'veda_hip.h'


def _declared():
    text = re.sub(r'/\*.*?\*/', '', HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r'\b(?:int|const char\*)\s+(veda_\w+)\s*\(([^;]*?)\)\s*;', text, re.S):
        args = [a.strip() for a in m.group(2).split(',') if a.strip() and a.strip() != 'void']
        out[m.group(1)] = len(args)
    return out


def test_library_built_and_exports_every_declared_symbol():
    lib = _native.load()
    declared = _declared()
    assert {'veda_gather_tiles', 'veda_block_sparse_fwd', 'veda_block_heat',
            'veda_select_topk', 'veda_index_lists'} <= set(declared)
    for name in declared:
        assert hasattr(lib, name), name
    # the binding covers every compute entry point with the declared arity
    for name, n in declared.items():
        if name in ('veda_last_error', 'veda_abi_version'):
            continue
        assert len(_native.SIGNATURES[name]) == n, name
    assert set(_native.SIGNATURES) <= set(declared)
    assert lib.veda_abi_version() == _native.ABI_VERSION == 5


def test_host_side_argument_checks():
    lib = _native.load()
    # head_dim 96 is refused before anything is launched
    with pytest.raises(ValueError, match='head_dim'):
        _native.call('veda_gather_tiles', None, 0, 0, 0, 0, None, None, None, 1, None, 1, 96,
                     None, 0, 0, None, None, None, None)
    with pytest.raises(ValueError, match='k_lo'):
        _native.call('veda_select_topk', None, 1, 1, 0, 0, 0, 10, None, None, 5, 4, None, 0,
                     None, None, 0, 0, 0, None)
    with pytest.raises(ValueError, match='head_dim'):
        _native.call('veda_block_sparse_fwd', None, 0, 0, None, 0, 0, None, 0, 0, 1, 64, 1, 1,
                     None, None, None, None, 1, None, 1.0, None, 0, 0, None, 0, 0, 0, None)
    with pytest.raises(ValueError, match='front_tiles'):
        _native.call('veda_block_sparse_fwd', None, 0, 0, None, 0, 0, None, 0, 0, 1, 128, 1, 1,
                     None, None, None, None, 1, None, 1.0, None, 0, 0, None, 0, 0, 2, None)
    with pytest.raises(ValueError, match='reduce'):
        _native.call('veda_block_heat', None, 0, 0, None, 0, 0, None, 0, 0, None, None, 1, 1,
                     1, 128, 3, 1.0, None, None)
    with pytest.raises(ValueError, match='used'):
        _native.call('veda_dense_fwd', None, 0, 0, None, 0, 0, None, 0, 0, 10, 11, 1, 128, 1.0,
                     None, 0, 0, None, 0, 0, None)
    with pytest.raises(ValueError, match='head_dim'):
        _native.call('veda_dense_heat_fwd', None, 0, 0, 1, None, 0, 0, None, 0, 0, 1, 64, None,
                     1, 1, None, 1.0, 0, None, 0, 0, None, 0, 0, None, None)
    with pytest.raises(ValueError, match='reduce'):
        _native.call('veda_dense_heat_fwd', None, 0, 0, 1, None, 0, 0, None, 0, 0, 1, 128, None,
                     1, 1, None, 1.0, 2, None, 0, 0, None, 0, 0, None, None)
    with pytest.raises(ValueError, match='out and v'):
        _native.call('veda_dense_heat_fwd', 16, 0, 0, 1, 16, 0, 0, 16, 0, 0, 1, 128, None,
                     1, 1, None, 1.0, 0, None, 0, 0, 16, 0, 0, 16, None)
    with pytest.raises(ValueError, match='head_dim'):
        _native.call('veda_block_sparse_bwd', *([None, 0, 0] * 7), 1, 64, 1, 1, None, None,
                     None, None, 1, None, None, None, None, 1, None, 1.0, *([None, 0, 0] * 3),
                     None, 0, 0, None)
    with pytest.raises(ValueError, match='workspace'):
        _native.call('veda_block_sparse_bwd', *([16, 0, 0] * 5), 16, 0, 0, None, 0, 0, 1, 128,
                     1, 1, None, None, None, None, 1, None, None, None, None, 1, None, 1.0,
                     *([16, 0, 0] * 3), 16, 1024, 0, None)
    with pytest.raises(ValueError, match='head_dim'):
        _native.call('veda_compensated_attention', None, 0, 0, None, 0, 0, None, 0, 0, 1, 64, 1, 1,
                     None, None, None, None, 1, None, None, 0, 0, None, None, 1.0, None, 0, 0, 0,
                     None)
    with pytest.raises(ValueError, match='front_tiles'):
        _native.call('veda_compensated_attention', None, 0, 0, None, 0, 0, None, 0, 0, 1, 128, 1,
                     1, None, None, None, None, 1, None, None, 0, 0, None, None, 1.0, None, 0, 0,
                     -1, None)
    with pytest.raises(ValueError, match='front_tiles'):
        _native.call('veda_block_sparse_bwd', *([16, 0, 0] * 5), 16, 0, 0, None, 0, 0, 1, 128,
                     2, 1, None, None, None, None, 2, None, None, None, None, 2, None, 1.0,
                     *([16, 0, 0] * 3), 16, 1 << 20, 2, None)
    with pytest.raises(ValueError, match='reduce'):
        _native.call('veda_heat_combine', None, None, 0, 0, None, None, 1, 1, 1, 5, None, None)
    assert isinstance(lib.veda_last_error(), bytes)


def test_supports_refuses_cpu_tensors_and_unknown_ops():
    import torch
    from miowtion_amd import kernels
    x = torch.zeros(4, 2, 128, dtype=torch.bfloat16)
    for op in ('gather', 'attention', 'heat'):
        assert not kernels.supports(x, op)
    with pytest.raises(ValueError, match='op must be'):
        kernels.supports(x, 'dense')


def test_error_messages_are_per_thread():
    """The library keeps no host state shared between calls; a failed call's
    message is the calling thread's own (threads that each drive a GPU need
    no lock around the calls). Two threads fail different entry points
    thousands of times and each always reads its own message."""
    lib = _native.load()
    failures = []

    def heat():
        for _ in range(3000):
            rc = lib.veda_block_heat(None, 0, 0, None, 0, 0, None, 0, 0, None, None, 1, 1,
                                     1, 128, 3, 1.0, None, None)
            msg = lib.veda_last_error().decode()
            if rc != -1 or 'reduce' not in msg:
                failures.append(('heat', rc, msg))

    def gather():
        for _ in range(3000):
            rc = lib.veda_gather_tiles(None, 0, 0, 0, 0, None, None, None, 1, None, 1, 96,
                                       None, 0, 0, None, None, None, None)
            msg = lib.veda_last_error().decode()
            if rc != -1 or 'head_dim' not in msg:
                failures.append(('gather', rc, msg))

    threads = [threading.Thread(target=f) for f in (heat, gather)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not failures, failures[:3]
