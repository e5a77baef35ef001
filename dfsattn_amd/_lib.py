"""ctypes binding of libdfsattn_amd.so (declarations: include/dfsattn_amd.h).

The library is loaded lazily and is mandatory: every GPU op raises if it is
missing, there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libdfsattn_amd.so")

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# name -> argument types (all return int status unless listed in _RESTYPES).
SIGNATURES = {
    "dfs_last_error": [],
    "dfs_abi_version": [],
    "dfs_hilbert3d_perm": [_i64, _i64, _i64, _p],
    "dfs_permute_gather": [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p],
    "dfs_permute_scatter": [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p],
    "dfs_prepare_qkv": [_p, _p, _p, _p, _i64, _i64, _i64, _i32, _i64, _i64, _i64, _i32,
                        _p, _p, _p, _p, _p, _p, _p, _p, _p],
    "dfs_block_score_topk_workspace_size": [_i64, _i64, _i64, _i64, _i64],
    "dfs_block_score_topk": [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                             _i64, _i64, _i64, _p, _p, _p, _p, _p, _i64, _p],
    "dfs_block_score_topk_noalloc": [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                     _i64, _i64, _i64, _p, _p, _p, _p],
    "dfs_topk_from_scores": [_p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p, _p],
    "dfs_prepare_fixup": [_p, _p, _p, _p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p],
    "dfs_bsa_fwd": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _f32, _p, _i32, _p, _p, _p, _p, _i64, _p,
                    _p, _p, _i32, _p],
    "dfs_mask_row_counts": [_p, _i64, _i64, _p, _p],
    "dfs_mask_to_csr": [_p, _i64, _i64, _p, _p, _p],
    "dfs_csr_to_mask": [_p, _p, _i64, _i64, _p, _p],
    "dfs_norm_rope": [_p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32,
                      _p, _i32, _f32, _p, _p, _i64, _p],
    "dfs_head_norm_rope": [_p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32,
                           _p, _i32, _f32, _p, _p, _i64, _p],
    "dfs_adaln_modulate": [_p, _i64, _i64, _i32, _p, _p, _p, _p, _f32, _p, _p],
    "dfs_gated_residual": [_p, _p, _p, _i64, _i64, _i32, _p, _p],
}
_RESTYPES = {"dfs_last_error": ctypes.c_char_p, "dfs_block_score_topk_workspace_size": ctypes.c_int64}
ABI_VERSION = 5

_lock = threading.Lock()
_lib = None


class DfsKernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""


def lib() -> ctypes.CDLL:
    """The loaded library; raises ImportError when it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise ImportError(
                        f"{LIB_PATH} is missing; build it with `python -m dfsattn_amd.build` "
                        "(the DFS HIP kernels have no CPU fallback)")
                handle = ctypes.CDLL(LIB_PATH)
                for name, args in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.argtypes = args
                    fn.restype = _RESTYPES.get(name, ctypes.c_int)
                if handle.dfs_abi_version() != ABI_VERSION:
                    raise ImportError(f"{LIB_PATH} has ABI {handle.dfs_abi_version()}, expected {ABI_VERSION}")
                _lib = handle
    return _lib


def call(name: str, *args) -> None:
    """Calls entry point ``name`` and raises DfsKernelError on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().dfs_last_error().decode(errors="replace")
        raise DfsKernelError(f"{name} failed (status {rc}): {msg}")
