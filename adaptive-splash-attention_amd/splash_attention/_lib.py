"""ctypes binding of libadasplash (C ABI in include/adasplash.h).

The library is loaded from ``splash_attention/lib/libadasplash.so`` (built
in-tree by ``splash_attention._build``).  There is no fallback: if the
library is missing or stale, every call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

from . import _build

ABI_VERSION = 8

ASA_OK = 0
ASA_ERR_INVALID_ARGUMENT = 1
ASA_ERR_UNSUPPORTED = 2
ASA_ERR_DEVICE = 3

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2

TAU_REFERENCE = 0
TAU_EXACT = 1
GRAD_ENTMAX = 0
GRAD_REFERENCE = 1

# workspace held by asa_forward_noalloc (ASA_NOALLOC_WORKSPACE_BYTES)
NOALLOC_WORKSPACE_BYTES = 64 << 20

# bits of asa_state.status (ASA_STATUS_* in adasplash.h)
STATUS_SELECT_ROUNDS = 0x1
STATUS_REFINE_SWEEPS = 0x2

# Every symbol the header declares (checked by the CPU test suite).
EXPORTS = (
    "asa_abi_version",
    "asa_last_error",
    "asa_query_sizes",
    "asa_forward",
    "asa_forward_noalloc",
    "asa_backward",
    "asa_select_from_scores",
    "asa_set_pairing",
    "asa_profile_enable",
    "asa_profile_read",
)


class Problem(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("nq", ctypes.c_int32),
        ("nk", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("k_keep", ctypes.c_int32),
        ("block_m", ctypes.c_int32),
        ("block_n", ctypes.c_int32),
        ("alpha", ctypes.c_float),
        ("sm_scale", ctypes.c_float),
        ("dtype", ctypes.c_int32),
        ("tau_mode", ctypes.c_int32),
        # element strides {batch, head, row}; zeros: contiguous
        ("q_strides", ctypes.c_int64 * 3),
        ("k_strides", ctypes.c_int64 * 3),
        ("v_strides", ctypes.c_int64 * 3),
        ("dout_strides", ctypes.c_int64 * 3),
    ]


class State(ctypes.Structure):
    _fields_ = [
        ("taus", ctypes.c_void_p),
        ("norms", ctypes.c_void_p),
        ("mask", ctypes.c_void_p),
        ("q_ptr", ctypes.c_void_p),
        ("q_list", ctypes.c_void_p),
        ("k_ptr", ctypes.c_void_p),
        ("k_list", ctypes.c_void_p),
        ("topk_idx", ctypes.c_void_p),
        ("topk_val", ctypes.c_void_p),
        ("sup_mask", ctypes.c_void_p),
        ("status", ctypes.c_void_p),
    ]


class Sizes(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in (
        "taus", "norms", "mask", "q_ptr", "q_list", "k_ptr", "k_list", "topk_idx", "topk_val",
        "sup_mask", "workspace")]


class ASAError(RuntimeError):
    """Error reported by libadasplash; `code` is the asa_status value."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


_lock = threading.Lock()
_handle: ctypes.CDLL | None = None

_V = ctypes.c_void_p
_I = ctypes.c_int32


def library_path() -> str:
    return _build.LIB


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it is not built."""
    global _handle
    if _handle is not None:
        return _handle
    with _lock:
        if _handle is not None:
            return _handle
        path = library_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"libadasplash is not built ({path} missing); run "
                "`python -c 'import __graft_entry__ as g; g.build()'` or "
                "`python adaptive-splash-attention_amd/splash_attention/_build.py`")
        lib = ctypes.CDLL(path)
        lib.asa_abi_version.restype = ctypes.c_int
        lib.asa_abi_version.argtypes = []
        if lib.asa_abi_version() != ABI_VERSION:
            raise RuntimeError(f"libadasplash ABI {lib.asa_abi_version()} != {ABI_VERSION}; rebuild")
        lib.asa_last_error.restype = ctypes.c_char_p
        lib.asa_last_error.argtypes = []
        lib.asa_query_sizes.restype = ctypes.c_int
        lib.asa_query_sizes.argtypes = [ctypes.POINTER(Problem), ctypes.POINTER(Sizes)]
        lib.asa_forward.restype = ctypes.c_int
        lib.asa_forward.argtypes = [ctypes.POINTER(Problem), _V, _V, _V, _V, _V, _V,
                                    ctypes.POINTER(State), _V, _V]
        lib.asa_forward_noalloc.restype = ctypes.c_int
        lib.asa_forward_noalloc.argtypes = [ctypes.POINTER(Problem), _V, _V, _V, _V, _V, _V,
                                            ctypes.POINTER(State), _V]
        lib.asa_backward.restype = ctypes.c_int
        lib.asa_backward.argtypes = [ctypes.POINTER(Problem), _I, _V, _V, _V, _V, _V, _V, _V,
                                     ctypes.POINTER(State), _V, _V, _V, _V, _V]
        lib.asa_select_from_scores.restype = ctypes.c_int
        lib.asa_select_from_scores.argtypes = [ctypes.POINTER(Problem), _V, _V, _V,
                                               ctypes.POINTER(State), _V, _V]
        lib.asa_set_pairing.restype = ctypes.c_int
        lib.asa_set_pairing.argtypes = [ctypes.c_int]
        lib.asa_profile_enable.restype = ctypes.c_int
        lib.asa_profile_enable.argtypes = [ctypes.c_int]
        lib.asa_profile_read.restype = ctypes.c_int
        lib.asa_profile_read.argtypes = [ctypes.c_int, _V, _V, _V]
        _handle = lib
        return lib


def check(rc: int) -> None:
    if rc != ASA_OK:
        msg = load().asa_last_error().decode(errors="replace")
        if rc == ASA_ERR_INVALID_ARGUMENT:
            raise ValueError(msg)
        raise ASAError(rc, msg)


def query_sizes(p: Problem) -> Sizes:
    z = Sizes()
    check(load().asa_query_sizes(ctypes.byref(p), ctypes.byref(z)))
    return z


PAIRING = {"auto": 0, "always": 1, "never": 2}  # asa_pairing


def set_pairing(mode: str) -> None:
    """Forward kernel for 16-bit inputs (asa_set_pairing, process-wide):
    "auto" (default) pairs query blocks when the pairs fill the GPU,
    "always" wherever the paired kernel applies, "never" not at all."""
    if mode not in PAIRING:
        raise ValueError(f"pairing must be one of {sorted(PAIRING)}, got {mode!r}")
    check(load().asa_set_pairing(PAIRING[mode]))


def profile_enable(on: bool) -> None:
    check(load().asa_profile_enable(1 if on else 0))


def profile_read(max_kernels: int = 32) -> dict[str, tuple[int, float]]:
    """{kernel name: (launches, total ms)} since the last read (synchronises)."""
    names = (ctypes.c_char * 64 * max_kernels)()
    counts = (ctypes.c_int * max_kernels)()
    total = (ctypes.c_double * max_kernels)()
    n = load().asa_profile_read(max_kernels, ctypes.cast(names, _V), ctypes.cast(counts, _V),
                                ctypes.cast(total, _V))
    out = {}
    for i in range(n):
        out[bytes(names[i]).split(b"\0", 1)[0].decode()] = (counts[i], total[i])
    return out
