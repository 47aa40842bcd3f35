"""Tensor-level entry points over the C ABI.

Every function here validates its torch tensors the way the reference
extension does (source/adasplashattention.cu:542-558), allocates the
outputs and per-call state with torch, and launches on the current HIP
stream of the input's device.  Nothing synchronises.
"""
from __future__ import annotations

import ctypes
import math
import warnings
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import _lib

BLOCK_M = 64             # default query rows per mask block
BLOCK_MS = (64, 32)      # supported block_m values
BLOCK_N = 64
MAX_HEAD_DIM = 128
MAX_K_KEEP = 128

# dtypes the kernels compute in
_DTYPES = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16,
           torch.float16: _lib.DTYPE_F16}
# dtypes the Python entry points accept (each has its own kernels)
INPUT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)

GRAD_MODES = {"entmax": _lib.GRAD_ENTMAX, "reference": _lib.GRAD_REFERENCE}
# "reference": the reference's top-k threshold; "exact": the alpha-entmax
# threshold over the whole visible row (asa_tau_mode in adasplash.h)
TAU_MODES = {"reference": _lib.TAU_REFERENCE, "exact": _lib.TAU_EXACT}
# How the backward runs (the forward records the support masks only for
# "support"):
#   "support": over each row's (row, key) pairs with nonzero weight, from
#              the support masks the forward records (512 bytes per active
#              tile); VALU and gather work per pair, fastest when supports
#              are small (headline: 0.33 ms against 0.83 ms)
#   "tiles":   over whole active 64 x 64 tiles on MFMA, no masks; fastest
#              when most entries of the active tiles are in the support
#              (near-uniform rows: 1x4x4096x64, N(0,1)*0.1 inputs, k 8,
#              block_m 32: 0.21 ms against 3.9 ms)
BWD_PASSES = ("support", "tiles")


@dataclass
class SplashState:
    """Selection state of one forward call (see asa_state in adasplash.h)."""
    taus: torch.Tensor       # [BH, NQ] float32
    norms: torch.Tensor      # [BH, NQ] float32, sum of p per row
    mask: torch.Tensor       # [BH, nQB, nKB] uint8, nQB = ceil(NQ / block_m)
    q_ptr: torch.Tensor      # [BH, nQB+1] int32 (reference Qi_ptr)
    q_list: torch.Tensor     # [BH, nQB*nKB] int32 (reference Qi_idx)
    k_ptr: torch.Tensor      # [BH, nKB+1] int32
    k_list: torch.Tensor     # [BH, nKB*nQB] int32
    topk_idx: torch.Tensor | None = None  # [BH, NQ, k] int32
    topk_val: torch.Tensor | None = None  # [BH, NQ, k] float32
    # support masks (asa_state.sup_mask): the (row, key) pairs with u > 0,
    # 16 bits per (tile, 16-row wave, lane) as uint16 bit patterns
    sup_mask: torch.Tensor | None = None  # [BH, ceil(NQ/64)*nKB, 4, 64] int16
    # per-call status word (asa_state.status): written on the stream by the
    # forward, read only by check_status()
    status: torch.Tensor | None = None    # [1] int32

    SUPPORT = ("sup_mask",)

    def c_struct(self) -> _lib.State:
        def ptr(t):
            return None if t is None else t.data_ptr()
        return _lib.State(ptr(self.taus), ptr(self.norms), ptr(self.mask), ptr(self.q_ptr),
                          ptr(self.q_list), ptr(self.k_ptr), ptr(self.k_list),
                          ptr(self.topk_idx), ptr(self.topk_val), ptr(self.sup_mask),
                          ptr(self.status))

    def status_word(self) -> int:
        """The forward's status word (synchronises with the device)."""
        if self.status is None:
            return 0
        return int(self.status.item()) & 0xFFFFFFFF

    def overflow_rounds(self) -> int:
        """Largest number of candidate overflow rounds a query block of the
        score pass ran (information; synchronises)."""
        return (self.status_word() >> 8) & 0xFF

    def check_status(self) -> None:
        """Debug check (synchronises): raises RuntimeError if the forward
        reported a truncated iteration (ASA_STATUS_* in adasplash.h)."""
        w = self.status_word()
        msgs = []
        if w & _lib.STATUS_SELECT_ROUNDS:
            msgs.append("score pass stopped at its candidate round bound (top-k may be incomplete)")
        if w & _lib.STATUS_REFINE_SWEEPS:
            msgs.append("exact tau: a row's iteration stopped at the sweep cap (tau not converged)")
        if msgs:
            raise RuntimeError("; ".join(msgs))

    def tensors(self) -> tuple:
        """The tensors a backward needs (support lists included when present)."""
        base = (self.taus, self.norms, self.mask, self.q_ptr, self.q_list, self.k_ptr,
                self.k_list)
        if self.sup_mask is None:
            return base
        return base + tuple(getattr(self, n) for n in self.SUPPORT)

    @classmethod
    def from_tensors(cls, ts) -> "SplashState":
        """A state from tensors() (an empty support-mask tensor, as the custom
        operator returns without masks, reads as none)."""
        st = cls(*ts[:7])
        if len(ts) > 7:
            for n, t in zip(cls.SUPPORT, ts[7:]):
                setattr(st, n, t if t.numel() else None)
        return st


def fix_nonfinite(t: torch.Tensor, name: str) -> torch.Tensor:
    """The reference's host fix-up of a result (adasplashattention.cu:599-606
    for the output, :684-697 for dQ, dK, dV): NaN elements become 0, and if
    any element is infinite the whole tensor is clamped to [-100, 100]; each
    step warns.  Synchronises with the device (two reductions read back), as
    the reference's ``.item()`` calls do.

    The kernels already zero non-finite outputs and dQ elements, as the
    reference's kernels do (:335-337, :529-531); a dK or dV sum that
    overflows stays +-inf, as the reference's atomic sums do, and is what
    this clamp acts on.
    """
    if bool(torch.isnan(t).any()):
        warnings.warn(f"NaN values detected in {name}, setting to zero", RuntimeWarning,
                      stacklevel=3)
        t = t.masked_fill(torch.isnan(t), 0.0)
    if bool(torch.isinf(t).any()):
        warnings.warn(f"Inf values detected in {name}, clamping", RuntimeWarning, stacklevel=3)
        t = torch.clamp(t, -100.0, 100.0)
    return t


def clamp_alpha(alpha: float) -> float:
    """alpha as the kernels use it (adasplashattention.cu:547)."""
    return max(1.05, min(float(alpha), 3.0))


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _index(idx, BH: int, N: int, B: int, H: int, device, name: str) -> torch.Tensor:
    """Position indices as int32 [BH, N] on `device` (reference: Q_idx/K_idx [B*H, N])."""
    if idx is None:
        return torch.arange(N, device=device, dtype=torch.int32).unsqueeze(0).expand(BH, N).contiguous()
    if not isinstance(idx, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if idx.dtype.is_floating_point or idx.dtype == torch.bool:
        raise TypeError(f"{name} must be an integer tensor, got {idx.dtype}")
    if idx.dim() == 1 and idx.shape[0] == N:
        idx = idx.unsqueeze(0).expand(BH, N)
    elif idx.dim() == 3 and tuple(idx.shape) == (B, H, N):
        idx = idx.reshape(BH, N)
    if tuple(idx.shape) != (BH, N):
        raise ValueError(f"{name} must have shape [B*H, N] = [{BH}, {N}], got {tuple(idx.shape)}")
    if idx.dtype != torch.int32:
        if idx.numel() and (int(idx.min()) < -(2 ** 31) or int(idx.max()) >= 2 ** 31):
            raise ValueError(f"{name} values do not fit int32")
        idx = idx.to(torch.int32)
    if idx.device != device:
        raise RuntimeError("All tensors must be on same device")
    return idx.contiguous()


class HeadDimError(RuntimeError, ValueError):
    """Head dimension above the kernels' limit.  The reference raises it as a
    RuntimeError (TORCH_CHECK, adasplashattention.cu:542); it is also a
    ValueError, like this module's other argument errors."""


def check_shapes(Q, K, V, k_keep=None):
    """The reference's argument checks (adasplashattention.cu:542-558) that
    need no tensor data: ranks, shapes, dtypes, head dimension, device."""
    for name, t in (("Q", Q), ("K", K), ("V", V)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a tensor")
        if t.dim() != 4:
            raise ValueError(f"{name} must be 4-D [B, H, N, d], got shape {tuple(t.shape)}")
    if Q.size(3) > MAX_HEAD_DIM:
        raise HeadDimError("Head dimension too large; increase D_MAX")
    if Q.dtype not in INPUT_DTYPES:
        raise TypeError(f"unsupported dtype {Q.dtype}; use torch.float32, torch.bfloat16 "
                        "or torch.float16")
    if K.dtype != Q.dtype or V.dtype != Q.dtype:
        raise TypeError("Q, K and V must have the same dtype")
    B, H, NQ, d = Q.shape
    if K.shape[0] != B or K.shape[1] != H or K.shape[3] != d:
        raise ValueError(f"K shape {tuple(K.shape)} does not match Q shape {tuple(Q.shape)}")
    if V.shape != K.shape:
        raise ValueError(f"V shape {tuple(V.shape)} must equal K shape {tuple(K.shape)}")
    if d < 1:
        raise ValueError("head dimension must be at least 1")
    NK = K.shape[2]
    if NQ < 1 or NK < 1 or B < 1 or H < 1:
        raise ValueError("empty attention problem")
    if not Q.is_cuda:
        raise RuntimeError("Tensors must be on CUDA device")
    if K.device != Q.device or V.device != Q.device:
        raise RuntimeError("All tensors must be on same device")
    if k_keep is not None and not (1 <= int(k_keep) <= MAX_K_KEEP):
        raise ValueError(f"k_keep {k_keep} out of range [1, {MAX_K_KEEP}]")


def check_inputs(Q, K, V, Q_idx=None, K_idx=None):
    """Validate and normalise (Q, K, V, Q_idx, K_idx).  Q, K, V come back as
    the kernels read them (kernel_operand): the caller's tensors themselves,
    views included, unless their head dimension needs padding or their
    layout cannot be read in place."""
    check_shapes(Q, K, V)
    B, H, NQ, _ = Q.shape
    NK = K.shape[2]
    BH = B * H
    qi = _index(Q_idx, BH, NQ, B, H, Q.device, "Q_idx")
    ki = _index(K_idx, BH, NK, B, H, Q.device, "K_idx")
    Q, K, V = to_kernel_layout(Q, K, V)
    return kernel_operand(Q), kernel_operand(K), kernel_operand(V), qi, ki


def chunk_elems(dtype: torch.dtype) -> int:
    """Elements of a 16-byte chunk, the kernels' unit of every load and store."""
    return 4 if dtype == torch.float32 else 8


def kernel_head_dim(d: int, dtype: torch.dtype) -> int:
    """The head dimension the kernels take for a caller's d <= 128: d itself
    when it is a whole number of 16-byte chunks, else d rounded up to one."""
    e = chunk_elems(dtype)
    return -(-d // e) * e


def to_kernel_layout(*ts):
    """Tensors [..., d] as the kernels take them: the head dimension
    zero-padded to a whole number of 16-byte chunks (kernel_head_dim; no
    change for d a multiple of 8, or of 4 in fp32).

    The reference accepts any d <= 128 (adasplashattention.cu:542); the
    kernels read any d that is a whole number of 16-byte chunks, in place.
    Zero columns add exact zeros to every dot product, so scores, weights
    and tau are those of the unpadded problem, and the padded columns of
    the outputs and of dQ, dK, dV are zero.  The padding is a
    differentiable torch op: gradients reach the caller's tensors through it.
    """
    dk = kernel_head_dim(ts[0].size(-1), ts[0].dtype)
    out = []
    for t in ts:
        if t.size(-1) != dk:
            t = F.pad(t, (0, dk - t.size(-1)))
        out.append(t)
    return out


def from_kernel_layout(t: torch.Tensor, d: int, dtype: torch.dtype) -> torch.Tensor:
    """Undo to_kernel_layout on an output: first d columns, caller's dtype."""
    if t.size(-1) != d:
        t = t[..., :d]
    if t.dtype != dtype:
        t = t.to(dtype)
    return t


def strides_of(t: torch.Tensor) -> tuple:
    """Element strides {batch, head, row} of a [B, H, N, d] operand, as the
    C ABI takes them.  A dimension of size 1 gets its contiguous stride (its
    stride is never used), so the ABI's mark for a contiguous operand, all
    three strides 0, comes out only for an operand broadcast along all
    three dimensions, which readable_in_place rejects."""
    B, H, N, d = t.shape
    contiguous = (H * N * d, N * d, d)
    return tuple(st if n > 1 else c for n, st, c in zip((B, H, N), t.stride()[:3], contiguous))


def readable_in_place(t: torch.Tensor) -> bool:
    """Whether the kernels can read a [B, H, N, d] operand where it is (the
    C ABI's stride rules, asa_problem.q_strides): contiguous head dimension,
    16-byte aligned start, non-negative batch, head and row strides that are
    whole 16-byte chunks, not all three 0, and a head's rows within 2^31
    bytes of its first."""
    e = chunk_elems(t.dtype)
    if t.size(-1) > 1 and t.stride(-1) != 1:
        return False
    if t.data_ptr() % 16:
        return False
    st = strides_of(t)
    if any(x < 0 or x % e for x in st):
        return False
    if st == (0, 0, 0):  # broadcast along batch, heads and rows: the ABI's "contiguous" mark
        return False
    return ((t.size(2) - 1) * st[2] + t.size(-1)) * t.element_size() < 2 ** 31


def kernel_operand(t: torch.Tensor) -> torch.Tensor:
    """t itself if readable_in_place, else a contiguous, 16-byte aligned copy."""
    if readable_in_place(t):
        return t
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """Contiguous with a 16-byte aligned base (the C ABI's Out, dQ, dK, dV)."""
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _set_strides(p: _lib.Problem, **ts) -> None:
    """The operands' strides into the problem descriptor; raises for an
    operand the kernels cannot read in place (pass it through check_inputs
    or kernel_operand first)."""
    for name, t in ts.items():
        if not readable_in_place(t):
            raise ValueError(f"{name}: shape {tuple(t.shape)} with strides {tuple(t.stride())} "
                             "cannot be read in place; pass it through check_inputs first")
        arr = getattr(p, name + "_strides")
        for i, x in enumerate(strides_of(t)):
            arr[i] = x


def check_tau_mode(tau_mode: str) -> int:
    if tau_mode not in TAU_MODES:
        raise ValueError(f"tau_mode must be one of {sorted(TAU_MODES)}")
    return TAU_MODES[tau_mode]


def check_bwd_passes(bwd_passes: str) -> str:
    if bwd_passes not in BWD_PASSES:
        raise ValueError(f"bwd_passes must be one of {BWD_PASSES}, got {bwd_passes!r}")
    return bwd_passes


def check_block_m(block_m) -> int:
    """Query rows per mask block: 64, or 32 (the reference's compile-time
    BLOCK_M, adasplashattention.cu:8-9)."""
    if int(block_m) not in BLOCK_MS:
        raise ValueError(f"block_m must be one of {BLOCK_MS}, got {block_m}")
    return int(block_m)


def block_m_of(st: "SplashState", NQ: int) -> int:
    """The block_m a state was written with, from its mask's row count (for
    NQ <= 32 both give one identical row; 64 is returned)."""
    return 64 if st.mask.shape[1] == -(-NQ // 64) else 32


def make_problem(B, H, NQ, NK, d, dtype, alpha, k_keep, sm_scale,
                 tau_mode: str = "reference", block_m: int = BLOCK_M) -> _lib.Problem:
    if not (1 <= int(k_keep) <= MAX_K_KEEP):
        raise ValueError(f"k_keep {k_keep} out of range [1, {MAX_K_KEEP}]")
    block_m = check_block_m(block_m)
    if block_m == 32 and tau_mode == "exact":
        raise ValueError("tau_mode 'exact' needs block_m = 64")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    return _lib.Problem(B, H, NQ, NK, d, int(k_keep), block_m, BLOCK_N, float(alpha),
                        float(sm_scale), _DTYPES[dtype] if isinstance(dtype, torch.dtype) else dtype,
                        check_tau_mode(tau_mode))


def alloc_state(p: _lib.Problem, device, with_topk: bool = False,
                with_support: bool = False) -> SplashState:
    BH = p.batch * p.heads
    nQB = -(-p.nq // p.block_m)   # rows of the mask and CSR lists
    nQ64 = -(-p.nq // 64)         # 64-row tiles of the support masks
    nKB = -(-p.nk // BLOCK_N)
    i32 = dict(device=device, dtype=torch.int32)
    f32 = dict(device=device, dtype=torch.float32)
    st = SplashState(
        taus=torch.empty((BH, p.nq), **f32),
        norms=torch.empty((BH, p.nq), **f32),
        mask=torch.empty((BH, nQB, nKB), device=device, dtype=torch.uint8),
        q_ptr=torch.empty((BH, nQB + 1), **i32),
        q_list=torch.empty((BH, nQB * nKB), **i32),
        k_ptr=torch.empty((BH, nKB + 1), **i32),
        k_list=torch.empty((BH, nKB * nQB), **i32),
        status=torch.empty((1,), **i32),
    )
    if with_topk:
        st.topk_idx = torch.empty((BH, p.nq, p.k_keep), **i32)
        st.topk_val = torch.empty((BH, p.nq, p.k_keep), **f32)
    if with_support:
        st.sup_mask = torch.empty((BH, nQ64 * nKB, 4, 64), device=device, dtype=torch.int16)
    return st


def workspace(p: _lib.Problem, device) -> torch.Tensor:
    """Scratch memory the entry points need for problem `p` (asa_sizes.workspace)."""
    z = _lib.query_sizes(p)
    return torch.empty(max(z.workspace, 16), device=device, dtype=torch.uint8)


def splash_forward(Q, K, V, Q_idx, K_idx, alpha: float, k_keep: int, sm_scale=None,
                   with_topk: bool = False, with_support: bool = True,
                   tau_mode: str = "reference", noalloc: bool = False,
                   block_m: int = BLOCK_M):
    """Forward pass; returns (out, SplashState).  Inputs as check_inputs() returns them.
    with_support records the rows' support masks for the sparse backward
    (skip it for inference).  tau_mode "exact" solves tau over the whole
    visible row instead of the top-k (see TAU_MODES).  noalloc=True calls
    asa_forward_noalloc, whose workspace is the library's own device array
    (no workspace tensor is allocated; calls that overlap on one GPU race).
    block_m = 32 gives the reference's 32-row mask blocks."""
    lib = _lib.load()
    B, H, NQ, d = Q.shape
    p = make_problem(B, H, NQ, K.shape[2], d, Q.dtype, alpha, k_keep, sm_scale, tau_mode,
                     block_m)
    _set_strides(p, q=Q, k=K, v=V)
    st = alloc_state(p, Q.device, with_topk, with_support)
    out = torch.empty(Q.shape, dtype=Q.dtype, device=Q.device)
    cst = st.c_struct()
    if noalloc:
        with torch.cuda.device(Q.device):
            rc = lib.asa_forward_noalloc(ctypes.byref(p), Q.data_ptr(), K.data_ptr(), V.data_ptr(),
                                         Q_idx.data_ptr(), K_idx.data_ptr(), out.data_ptr(),
                                         ctypes.byref(cst), _stream(Q.device))
        _lib.check(rc)
        return out, st
    ws = workspace(p, Q.device)
    with torch.cuda.device(Q.device):
        rc = lib.asa_forward(ctypes.byref(p), Q.data_ptr(), K.data_ptr(), V.data_ptr(),
                             Q_idx.data_ptr(), K_idx.data_ptr(), out.data_ptr(),
                             ctypes.byref(cst), ws.data_ptr(), _stream(Q.device))
    _lib.check(rc)
    return out, st


def _as_kernel_operand(t: torch.Tensor, Q: torch.Tensor, name: str, contiguous: bool = False):
    """A [B, H, NQ, d'] operand of the backward (dOut, Out) in the layout of
    the kernel-layout Q: padded to Q's head dimension, in Q's dtype, read in
    place where the C ABI allows (dOut) or contiguous (Out)."""
    dq = Q.size(-1)
    if (t.dim() != 4 or tuple(t.shape[:3]) != tuple(Q.shape[:3]) or t.size(-1) > dq
            or kernel_head_dim(t.size(-1), Q.dtype) != dq):
        raise ValueError(f"{name} shape {tuple(t.shape)} must equal Q shape {tuple(Q.shape)}")
    (t,) = to_kernel_layout(t.to(Q.dtype))
    return _aligned(t) if contiguous else kernel_operand(t)


def splash_backward(Q, K, V, Q_idx, K_idx, out, dout, st: SplashState, alpha: float,
                    k_keep: int, sm_scale=None, grad_mode: str = "entmax"):
    """Gradients (dQ, dK, dV) from a forward's state (of either block_m)."""
    lib = _lib.load()
    if grad_mode not in GRAD_MODES:
        raise ValueError(f"grad_mode must be one of {sorted(GRAD_MODES)}")
    B, H, NQ, d = Q.shape
    p = make_problem(B, H, NQ, K.shape[2], d, Q.dtype, alpha, k_keep, sm_scale,
                     block_m=block_m_of(st, NQ))
    dout = _as_kernel_operand(dout, Q, "dOut")
    if out is not None:
        out = _as_kernel_operand(out, Q, "Out", contiguous=True)
    _set_strides(p, q=Q, k=K, v=V, dout=dout)
    ws = workspace(p, Q.device)
    dQ = torch.empty(Q.shape, dtype=Q.dtype, device=Q.device)
    dK = torch.empty(K.shape, dtype=K.dtype, device=K.device)
    dV = torch.empty(V.shape, dtype=V.dtype, device=V.device)
    cst = st.c_struct()
    with torch.cuda.device(Q.device):
        rc = lib.asa_backward(ctypes.byref(p), GRAD_MODES[grad_mode], Q.data_ptr(), K.data_ptr(),
                              V.data_ptr(), Q_idx.data_ptr(), K_idx.data_ptr(),
                              None if out is None else out.data_ptr(), dout.data_ptr(),
                              ctypes.byref(cst), dQ.data_ptr(), dK.data_ptr(), dV.data_ptr(),
                              ws.data_ptr(), _stream(Q.device))
    _lib.check(rc)
    return dQ, dK, dV


def select_from_scores(scores, Q_idx, K_idx, alpha: float, k_keep: int, batch: int = 1,
                       heads: int | None = None, with_topk: bool = True,
                       block_m: int = BLOCK_M) -> SplashState:
    """Top-k, tau, block mask and CSR lists from given fp32 scores [BH, NQ, NK]
    (no reference counterpart: exposes the reference's selection stage,
    adasplashattention.cu:199-216, for checks on identical scores).
    with_topk=False leaves the top-k index/value outputs out, which is the
    selection path asa_forward takes."""
    lib = _lib.load()
    if scores.dim() == 4:
        batch, heads = scores.shape[0], scores.shape[1]
        scores = scores.reshape(-1, scores.shape[2], scores.shape[3])
    if scores.dim() != 3:
        raise ValueError("scores must be [BH, NQ, NK] or [B, H, NQ, NK]")
    if scores.dtype != torch.float32:
        raise TypeError("scores must be float32")
    if not scores.is_cuda:
        raise RuntimeError("Tensors must be on CUDA device")
    BH, NQ, NK = scores.shape
    if heads is None:
        heads = BH // batch
    if batch * heads != BH:
        raise ValueError("batch * heads must equal scores.shape[0]")
    qi = _index(Q_idx, BH, NQ, batch, heads, scores.device, "Q_idx")
    ki = _index(K_idx, BH, NK, batch, heads, scores.device, "K_idx")
    p = make_problem(batch, heads, NQ, NK, 64, torch.float32, alpha, k_keep, 1.0,
                     block_m=block_m)
    st = alloc_state(p, scores.device, with_topk=with_topk)
    scores = scores.contiguous()
    ws = workspace(p, scores.device)
    cst = st.c_struct()
    with torch.cuda.device(scores.device):
        rc = lib.asa_select_from_scores(ctypes.byref(p), scores.data_ptr(), qi.data_ptr(),
                                        ki.data_ptr(), ctypes.byref(cst), ws.data_ptr(),
                                        _stream(scores.device))
    _lib.check(rc)
    return st
