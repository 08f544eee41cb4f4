"""ctypes binding of the C ABI declared in include/mi355_fa.h.

The product path loads only the in-tree ``libmi355_fa.so`` built by
``custom_ops_amd.build``; there is no fallback implementation. ``torch`` is
imported first so the process already holds PyTorch's HIP runtime
(``libamdhip64.so.7``) and the library binds to that same runtime by SONAME.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the dlopen below, see module docstring)

from .build import lib_path

FP16 = 0
BF16 = 1

OK = 0
EINVAL = 1
EWORKSPACE = 2
ELAUNCH = 3
EDEVICE = 4

# Every function include/mi355_fa.h declares (checked by tests/test_host.py).
EXPORTED = (
    "mi355_fa_fwd",
    "mi355_fa_fwd_noalloc",
    "mi355_fa_num_splits",
    "mi355_fa_workspace_bytes",
    "mi355_fa_cost_model_splits",
    "mi355_fa_abi_version",
    "mi355_fa_build_info",
)
ABI_VERSION = 3


class Variant(ctypes.Structure):
    """Mirror of ``mi355_fa_variant`` (include/mi355_fa.h): kernel-variant
    selection for parity tests and tuning. Every field 0 = the library's plan;
    see the header for the meaning of each value."""

    _fields_ = [(name, ctypes.c_int32) for name in
                ("waves", "pack", "order", "loop", "fuse", "live", "deep", "mask_mfma", "stream",
                 "live_map", "stage")]

    def __repr__(self) -> str:
        set_ = {n: getattr(self, n) for n, _ in self._fields_ if getattr(self, n)}
        return f"Variant({', '.join(f'{k}={v}' for k, v in set_.items())})"


class Params(ctypes.Structure):
    """Mirror of ``mi355_fa_params`` (include/mi355_fa.h)."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("mask", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("q_batch_stride", ctypes.c_int64), ("q_head_stride", ctypes.c_int64),
        ("q_row_stride", ctypes.c_int64),
        ("k_batch_stride", ctypes.c_int64), ("k_head_stride", ctypes.c_int64),
        ("k_row_stride", ctypes.c_int64),
        ("v_batch_stride", ctypes.c_int64), ("v_head_stride", ctypes.c_int64),
        ("v_row_stride", ctypes.c_int64),
        ("o_batch_stride", ctypes.c_int64), ("o_head_stride", ctypes.c_int64),
        ("o_row_stride", ctypes.c_int64),
        ("mask_batch_stride", ctypes.c_int64), ("mask_row_stride", ctypes.c_int64),
        ("b", ctypes.c_int32), ("h", ctypes.c_int32), ("h_k", ctypes.c_int32),
        ("seqlen_q", ctypes.c_int32), ("seqlen_k", ctypes.c_int32),
        ("mask_seqlen_q", ctypes.c_int32), ("mask_seqlen_k", ctypes.c_int32),
        ("d", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("scale_softmax", ctypes.c_float),
        ("num_splits", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("variant", ctypes.POINTER(Variant)),
    ]


_lock = threading.Lock()
_lib = None
_lib_file: str | None = None
_load_error: str | None = None


def load(path: str | None = None) -> ctypes.CDLL:
    """Open the library once per process; raise RuntimeError (with the reason)
    if it is absent or incompatible.

    ``path`` names the file to open (default: the in-tree build, or
    MI355_FA_LIB). Once a library is open, asking for a different file raises:
    one library serves the process."""
    global _lib, _load_error, _lib_file
    lib = _lib
    if lib is not None and path is None:      # per-call fast path: no lock, no path lookup
        return lib
    with _lock:
        want = os.path.realpath(path if path is not None else lib_path())
        if _lib is not None:
            if path is not None and want != _lib_file:
                raise RuntimeError(f"{_lib_file} is already loaded in this process; "
                                   f"cannot also load {want}")
            return _lib
        if not os.path.exists(want):
            _load_error = (f"{want} is missing: build it with `python -m custom_ops_amd.build` "
                           f"(or __graft_entry__.build())")
            raise RuntimeError(_load_error)
        try:
            lib = ctypes.CDLL(want)
        except OSError as e:
            _load_error = f"failed to load {want}: {e}"
            raise RuntimeError(_load_error) from e
        missing = [n for n in EXPORTED if not hasattr(lib, n)]
        if missing:
            _load_error = f"{want} does not export {missing}"
            raise RuntimeError(_load_error)
        P = ctypes.POINTER(Params)
        lib.mi355_fa_fwd.argtypes = [P, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]
        lib.mi355_fa_fwd.restype = ctypes.c_int
        lib.mi355_fa_fwd_noalloc.argtypes = [P, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]
        lib.mi355_fa_fwd_noalloc.restype = ctypes.c_int
        lib.mi355_fa_num_splits.argtypes = [P]
        lib.mi355_fa_num_splits.restype = ctypes.c_int
        lib.mi355_fa_workspace_bytes.argtypes = [P]
        lib.mi355_fa_workspace_bytes.restype = ctypes.c_size_t
        lib.mi355_fa_cost_model_splits.argtypes = [ctypes.c_int] * 5
        lib.mi355_fa_cost_model_splits.restype = ctypes.c_int
        lib.mi355_fa_abi_version.argtypes = []
        lib.mi355_fa_abi_version.restype = ctypes.c_int
        lib.mi355_fa_build_info.argtypes = []
        lib.mi355_fa_build_info.restype = ctypes.c_char_p
        ver = lib.mi355_fa_abi_version()
        if ver != ABI_VERSION:
            _load_error = f"{want}: ABI version {ver}, expected {ABI_VERSION}; rebuild it"
            raise RuntimeError(_load_error)
        _lib = lib
        _lib_file = want
        _load_error = None
        return lib


def loaded_path() -> str | None:
    """The file this process opened, if any."""
    return _lib_file if _lib is not None else None


def load_error() -> str | None:
    return _load_error


_tls = threading.local()


def _err_buffer() -> ctypes.Array:
    """Per-thread message buffer, reused across calls (the library writes it only on failure)."""
    buf = getattr(_tls, "err", None)
    if buf is None:
        buf = _tls.err = ctypes.create_string_buffer(512)
    return buf


def fwd(params: Params, stream: int) -> None:
    """Call mi355_fa_fwd; raise RuntimeError carrying the library's message on failure."""
    lib = load()
    err = _err_buffer()
    rc = lib.mi355_fa_fwd(ctypes.byref(params), stream, err, 512)
    if rc != OK:
        raise RuntimeError(err.value.decode(errors="replace") or f"mi355_fa_fwd failed ({rc})")


def workspace_bytes(params: Params) -> int:
    return int(load().mi355_fa_workspace_bytes(ctypes.byref(params)))


def num_splits(params: Params) -> int:
    return int(load().mi355_fa_num_splits(ctypes.byref(params)))


def cost_model_splits(total_mblocks: int, num_n_blocks: int, block_m: int, head_dim: int,
                      num_cus: int) -> int:
    return int(load().mi355_fa_cost_model_splits(total_mblocks, num_n_blocks, block_m, head_dim,
                                                 num_cus))
