"""ctypes binding of libveda_hip.so (the C ABI declared in include/veda_hip.h).

The library is the only compute path of this package. If it is missing, or
the process has no GPU, every op raises: there is no CPU fallback and no
silent dense fallback (the reference's own rule, `miowtion/kernels/fa4.py:
327-335`, `miowtion/veda/attention.py:713-717`).
"""

from __future__ import annotations

import ctypes
import pathlib
import threading

LIB_PATH = pathlib.Path(__file__).resolve().parent / 'libveda_hip.so'
# the signatures below are those of this ABI version (veda_abi_version())
ABI_VERSION = 5

_P = ctypes.c_void_p
_I = ctypes.c_int64
_F = ctypes.c_float
_C = ctypes.c_int

# name -> argument types, in the order of include/veda_hip.h.
SIGNATURES: dict[str, list] = {
    'veda_gather_tiles': [_P, _I, _I, _I, _I, _P, _P, _P, _I, _P, _I, _I, _P, _I, _I,
                          _P, _P, _P, _P],
    'veda_scatter_tiles': [_P, _I, _I, _P, _P, _I, _P, _I, _I, _P, _I, _I, _I, _I, _P],
    'veda_gather_lse': [_P, _I, _I, _I, _I, _P, _P, _I, _P, _I, _P, _P],
    'veda_select_topk': [_P, _I, _I, _I, _I, _I, _I, _P, _P, _I, _I, _P, _I, _P, _P,
                         _I, _I, _I, _P],
    'veda_dense_block_mask': [_P, _P, _I, _I, _I, _P, _I, _I, _C, _P, _P],
    'veda_index_lists': [_P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P],
    'veda_block_sparse_fwd': [_P, _I, _I, _P, _I, _I, _P, _I, _I, _I, _I, _I, _I,
                              _P, _P, _P, _P, _I, _P, _F, _P, _I, _I, _P, _I, _I, _I, _P],
    'veda_block_sparse_fwd_seq': [_P, _I, _I, _I, _I, _P, _P, _P, _P, _I, _P, _I, _I, _P, _I, _I,
                                  _I, _I, _I, _P, _P, _P, _P, _I, _P, _F, _P, _I, _I, _I, _I,
                                  _P],
    'veda_block_sparse_fwd_seq_kv': [_P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _I, _I, _I,
                                     _I, _P, _P, _P, _P, _I, _P, _F, _P, _I, _I, _I, _I, _P],
    'veda_dense_fwd': [_P, _I, _I, _P, _I, _I, _P, _I, _I, _I, _I, _I, _I, _F, _P,
                       _I, _I, _P, _I, _I, _P],
    'veda_block_heat': [_P, _I, _I, _P, _I, _I, _P, _I, _I, _P, _P, _I, _I, _I, _I,
                        _C, _F, _P, _P],
    'veda_dense_heat_fwd': [_P, _I, _I, _I, _P, _I, _I, _P, _I, _I, _I, _I, _P, _I, _I,
                            _P, _F, _C, _P, _I, _I, _P, _I, _I, _P, _P],
    'veda_heat_combine': [_P, _P, _I, _I, _P, _P, _I, _I, _I, _C, _P, _P],
    'veda_tile_summaries': [_P, _I, _I, _P, _I, _I, _P, _I, _I, _I, _P, _P, _I, _I, _P],
    'veda_zero_order_compensation': [_P, _I, _I, _P, _I, _I, _P, _I, _I, _P, _P, _I, _I, _P, _P,
                                     _I, _I, _I, _I, _F, _P, _I, _I, _P],
    'veda_block_sparse_bwd': [_P, _I, _I, _P, _I, _I, _P, _I, _I, _P, _I, _I, _P, _I, _I,
                              _P, _I, _I, _P, _I, _I, _I, _I, _I, _I,
                              _P, _P, _P, _P, _I, _P, _P, _P, _P, _I, _P, _F,
                              _P, _I, _I, _P, _I, _I, _P, _I, _I, _P, _I, _I, _P],
    'veda_block_sparse_bwd_noalloc': [_P, _I, _I, _P, _I, _I, _P, _I, _I, _P, _I, _I, _P, _I,
                                      _I, _P, _I, _I, _P, _I, _I, _I, _I, _I, _I,
                                      _P, _P, _P, _P, _I, _P, _P, _P, _P, _I, _P, _F,
                                      _P, _I, _I, _P, _I, _I, _P, _I, _I, _I, _P],
    'veda_compensated_attention': [_P, _I, _I, _P, _I, _I, _P, _I, _I, _I, _I, _I, _I,
                                   _P, _P, _P, _P, _I, _P, _P, _I, _I, _P, _P, _F,
                                   _P, _I, _I, _I, _P],
    'veda_predictor_embed': [_P, _I, _I, _I, _P, _C, _P, _I, _P, _I, _C, _P, _P],
    'veda_predictor_logits': [_P, _P, _I, _I, _I, _I, _F, _P, _P, _P, _C, _P, _P],
}

_lock = threading.Lock()
_lib = None


class NativeError(RuntimeError):
    """A HIP launch failed inside libveda_hip.so."""


def load() -> ctypes.CDLL:
    """Loads the library once; raises ImportError if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f'{LIB_PATH} is missing: build it with '
                    '`python -m miowtion_amd.csrc.build` (there is no CPU fallback)')
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, args in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = ctypes.c_int
            lib.veda_last_error.restype = ctypes.c_char_p
            lib.veda_last_error.argtypes = []
            lib.veda_abi_version.restype = ctypes.c_int
            lib.veda_abi_version.argtypes = []
            found = lib.veda_abi_version()
            if found != ABI_VERSION:
                raise ImportError(
                    f'{LIB_PATH} has ABI version {found}, this package binds version '
                    f'{ABI_VERSION}: rebuild it with `python -m miowtion_amd.csrc.build`')
            _lib = lib
        return _lib


def call(name: str, *args) -> None:
    """Calls one entry point; maps its status to ValueError / NativeError."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        msg = lib.veda_last_error().decode()
        if status == -1:
            raise ValueError(msg)
        raise NativeError(msg)
