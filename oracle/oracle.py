"""Python front end of the CPU oracle (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this module, and only as the checker.  The product path
(``splash_attention``) never imports it.

Two back ends are loaded with ctypes from ``oracle/lib`` (built by
``oracle/Makefile``): ``liboracle_f32.so`` restates the reference algorithm in
fp32 and ``liboracle_f64.so`` runs the same recurrences in fp64.  The
arrays are numpy, C-contiguous, shaped like the reference's tensors:
Q, K, V ``[BH, N, d]`` and Q_idx, K_idx ``[BH, N]`` int32
(source/adasplashattention.cu:164, :182, :571-572).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIBDIR = os.path.join(_HERE, "lib")
_ABI = 4

_libs: dict[str, ctypes.CDLL] = {}

_P = ctypes.c_void_p
_I = ctypes.c_int


def build() -> None:
    """Compile both oracle back ends with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _lib(precision: str) -> ctypes.CDLL:
    if precision in _libs:
        return _libs[precision]
    name = {"f32": "liboracle_f32.so", "f64": "liboracle_f64.so"}[precision]
    path = os.path.join(_LIBDIR, name)
    if not os.path.exists(path):
        build()
    lib = ctypes.CDLL(path)
    lib.asao_abi_version.restype = _I
    if lib.asao_abi_version() != _ABI:
        build()
        raise RuntimeError("oracle library was stale; rebuilt it, restart the process")
    R = ctypes.c_float if precision == "f32" else ctypes.c_double
    lib.asao_entmax_threshold.restype = R
    lib.asao_entmax_threshold.argtypes = [_P, _I, R]
    lib.asao_scores.restype = None
    lib.asao_scores.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, R, _P, _P]
    lib.asao_select.restype = None
    lib.asao_select.argtypes = [_P, _P, _I, _I, _I, _I, R, _I, _I, _P, _P, _P, _P]
    lib.asao_csr.restype = None
    lib.asao_csr.argtypes = [_P, _I, _I, _I, _P, _P, _P, _P]
    lib.asao_forward.restype = None
    lib.asao_forward.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I, R, R, _I, _I, _I,
                                 _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]
    lib.asao_set_threads.restype = None
    lib.asao_set_threads.argtypes = [_I]
    lib.asao_max_threads.restype = _I
    lib.asao_backward.restype = None
    lib.asao_backward.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, R, R, _I, _I,
                                  _P, _P, _P, _I, _P, _P, _P]
    _libs[precision] = lib
    return lib


def _dt(precision: str):
    return np.float32 if precision == "f32" else np.float64


def _arr(x, dtype) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=dtype))


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def entmax_threshold(s, alpha: float, precision: str = "f32") -> float:
    """tau of one row from its top-k values (descending; sentinel -1e6 pads)."""
    lib = _lib(precision)
    a = _arr(s, _dt(precision))
    return float(lib.asao_entmax_threshold(_ptr(a), a.shape[0], alpha))


def scores(Q, K, Q_idx, K_idx, sm_scale: float, precision: str = "f32"):
    """Clamped scores S[BH, NQ, NK] and visibility vis[BH, NQ, NK] (uint8)."""
    lib = _lib(precision)
    dt = _dt(precision)
    Q, K = _arr(Q, dt), _arr(K, dt)
    qi, ki = _arr(Q_idx, np.int32), _arr(K_idx, np.int32)
    BH, NQ, d = Q.shape
    NK = K.shape[1]
    S = np.empty((BH, NQ, NK), dt)
    vis = np.empty((BH, NQ, NK), np.uint8)
    lib.asao_scores(_ptr(Q), _ptr(K), _ptr(qi), _ptr(ki), BH, NQ, NK, d, sm_scale,
                    _ptr(S), _ptr(vis))
    return S, vis


@dataclass
class Selection:
    taus: np.ndarray       # [BH, NQ]
    topk_idx: np.ndarray   # [BH, NQ, k] int32, -1 for empty slots
    topk_val: np.ndarray   # [BH, NQ, k], -1e6 for empty slots
    mask: np.ndarray       # [BH, nQB, nKB] uint8


def select(S, vis, k: int, alpha: float, block_m: int = 64, block_n: int = 64,
           precision: str = "f32") -> Selection:
    """Top-k, tau and block mask from given scores."""
    lib = _lib(precision)
    dt = _dt(precision)
    S = _arr(S, dt)
    vis = _arr(vis, np.uint8)
    BH, NQ, NK = S.shape
    nQB = -(-NQ // block_m)
    nKB = -(-NK // block_n)
    taus = np.empty((BH, NQ), dt)
    ti = np.empty((BH, NQ, k), np.int32)
    tv = np.empty((BH, NQ, k), dt)
    mask = np.zeros((BH, nQB, nKB), np.uint8)
    lib.asao_select(_ptr(S), _ptr(vis), BH, NQ, NK, k, alpha, block_m, block_n,
                    _ptr(taus), _ptr(ti), _ptr(tv), _ptr(mask))
    return Selection(taus, ti, tv, mask)


@dataclass
class CSR:
    q_ptr: np.ndarray   # [BH, nQB+1]
    q_list: np.ndarray  # [BH, nQB*nKB]
    k_ptr: np.ndarray   # [BH, nKB+1]
    k_list: np.ndarray  # [BH, nKB*nQB]


def csr(mask, precision: str = "f32") -> CSR:
    lib = _lib(precision)
    m = _arr(mask, np.uint8)
    BH, nQB, nKB = m.shape
    qp = np.empty((BH, nQB + 1), np.int32)
    ql = np.empty((BH, nQB * nKB), np.int32)
    kp = np.empty((BH, nKB + 1), np.int32)
    kl = np.empty((BH, nKB * nQB), np.int32)
    lib.asao_csr(_ptr(m), BH, nQB, nKB, _ptr(qp), _ptr(ql), _ptr(kp), _ptr(kl))
    return CSR(qp, ql, kp, kl)


@dataclass
class Forward:
    out: np.ndarray
    taus: np.ndarray
    norms: np.ndarray
    topk_idx: np.ndarray
    topk_val: np.ndarray
    mask: np.ndarray
    csr: CSR


def forward(Q, K, V, Q_idx, K_idx, alpha: float, sm_scale: float, k: int,
            block_m: int = 64, block_n: int = 64, taus_in=None,
            precision: str = "f32") -> Forward:
    """Whole forward pass (scores, top-k, tau, mask, CSR, output)."""
    lib = _lib(precision)
    dt = _dt(precision)
    Q, K, V = _arr(Q, dt), _arr(K, dt), _arr(V, dt)
    qi, ki = _arr(Q_idx, np.int32), _arr(K_idx, np.int32)
    BH, NQ, d = Q.shape
    NK = K.shape[1]
    if K.shape != (BH, NK, d) or V.shape != (BH, NK, d):
        raise ValueError("K and V must be [BH, NK, d] matching Q")
    if qi.shape != (BH, NQ) or ki.shape != (BH, NK):
        raise ValueError("Q_idx must be [BH, NQ] and K_idx [BH, NK]")
    nQB = -(-NQ // block_m)
    nKB = -(-NK // block_n)
    tin = None if taus_in is None else _arr(taus_in, dt)
    taus = np.empty((BH, NQ), dt)
    norms = np.empty((BH, NQ), dt)
    ti = np.empty((BH, NQ, k), np.int32)
    tv = np.empty((BH, NQ, k), dt)
    mask = np.zeros((BH, nQB, nKB), np.uint8)
    c = CSR(np.empty((BH, nQB + 1), np.int32), np.empty((BH, nQB * nKB), np.int32),
            np.empty((BH, nKB + 1), np.int32), np.empty((BH, nKB * nQB), np.int32))
    out = np.empty((BH, NQ, d), dt)
    lib.asao_forward(_ptr(Q), _ptr(K), _ptr(V), _ptr(qi), _ptr(ki), BH, NQ, NK, d, alpha,
                     sm_scale, k, block_m, block_n, _ptr(tin), _ptr(taus), _ptr(norms),
                     _ptr(ti), _ptr(tv), _ptr(mask), _ptr(c.q_ptr), _ptr(c.q_list),
                     _ptr(c.k_ptr), _ptr(c.k_list), _ptr(out))
    return Forward(out, taus, norms, ti, tv, mask, c)


GRAD_ENTMAX = 0
GRAD_REFERENCE = 1


def backward(Q, K, V, Q_idx, K_idx, dO, alpha: float, sm_scale: float, taus, q_ptr, q_list,
             mode: int = GRAD_ENTMAX, block_m: int = 64, block_n: int = 64,
             precision: str = "f32"):
    """dQ, dK, dV for given taus and query-major CSR (mode 0 entmax, 1 reference)."""
    lib = _lib(precision)
    dt = _dt(precision)
    Q, K, V, dO = _arr(Q, dt), _arr(K, dt), _arr(V, dt), _arr(dO, dt)
    qi, ki = _arr(Q_idx, np.int32), _arr(K_idx, np.int32)
    taus = _arr(taus, dt)
    qp, ql = _arr(q_ptr, np.int32), _arr(q_list, np.int32)
    BH, NQ, d = Q.shape
    NK = K.shape[1]
    dQ = np.empty_like(Q)
    dK = np.empty_like(K)
    dV = np.empty_like(V)
    lib.asao_backward(_ptr(Q), _ptr(K), _ptr(V), _ptr(qi), _ptr(ki), _ptr(dO), BH, NQ, NK, d,
                      alpha, sm_scale, block_m, block_n, _ptr(taus), _ptr(qp), _ptr(ql),
                      int(mode), _ptr(dQ), _ptr(dK), _ptr(dV))
    return dQ, dK, dV


def host_fixup(x: np.ndarray) -> tuple[np.ndarray, bool, bool]:
    """The reference's host fix-up of one result tensor
    (source/adasplashattention.cu:599-606 for Out, :684-697 for dQ, dK, dV):
    NaN elements become 0 (``masked_fill_``); then, if any element is
    infinite, the whole tensor is clamped to [-100, 100] (``torch::clamp``).
    Returns (fixed array, had NaN, had Inf)."""
    x = np.array(x, copy=True)
    nan = bool(np.isnan(x).any())
    if nan:
        x[np.isnan(x)] = 0
    inf = bool(np.isinf(x).any())
    if inf:
        x = np.clip(x, -100.0, 100.0)
    return x, nan, inf


def set_num_threads(n: int) -> int:
    """Set the OpenMP thread count of both back ends; returns the previous
    count of the f32 one."""
    prev = _lib("f32").asao_max_threads()
    for p in ("f32", "f64"):
        _lib(p).asao_set_threads(int(n))
    return prev


def attention(Q, K, V, Q_idx, K_idx, dO, alpha: float, sm_scale: float, k: int,
              mode: int = GRAD_ENTMAX, block_m: int = 64, block_n: int = 64,
              precision: str = "f32"):
    """Forward and backward in one call: returns (Forward, (dQ, dK, dV))."""
    fw = forward(Q, K, V, Q_idx, K_idx, alpha, sm_scale, k, block_m, block_n,
                 precision=precision)
    grads = backward(Q, K, V, Q_idx, K_idx, dO, alpha, sm_scale, fw.taus, fw.csr.q_ptr,
                     fw.csr.q_list, mode, block_m, block_n, precision)
    return fw, grads
