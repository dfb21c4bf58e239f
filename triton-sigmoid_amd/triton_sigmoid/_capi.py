"""ctypes binding of libsigattn.so (the C ABI in include/sigattn.h).

The op bodies call `forward` / `backward` here.  They build one
`sigattn_problem`, pass raw device pointers and torch's current HIP stream,
and turn a non-zero status into RuntimeError.  There is no fallback: without
the built library or a gfx950 device the call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
import warnings
from pathlib import Path
from typing import Optional

import torch

# The library built next to this file; the environment variable
# SIGATTN_LIBRARY may name another build of the same sources (a tile-
# configuration variant from _build.py --out ... -D...).
LIB_PATH = Path(os.environ.get("SIGATTN_LIBRARY") or Path(__file__).resolve().parent / "libsigattn.so")
ABI_VERSION = 2

F16, BF16, F32 = 0, 1, 2
_DTYPE_CODE = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}

_c_i32, _c_i64, _c_vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p


class SigattnProblem(ctypes.Structure):
    """Mirror of `struct sigattn_problem` (include/sigattn.h)."""

    _fields_ = [
        ("abi_version", _c_i32),
        ("dtype", _c_i32),
        ("B", _c_i64),
        ("Tq", _c_i64),
        ("Tk", _c_i64),
        ("H", _c_i64),
        ("D", _c_i64),
        ("q_stride_b", _c_i64),
        ("q_stride_t", _c_i64),
        ("q_stride_h", _c_i64),
        ("k_stride_b", _c_i64),
        ("k_stride_t", _c_i64),
        ("k_stride_h", _c_i64),
        ("q", _c_vp),
        ("k", _c_vp),
        ("v", _c_vp),
        ("bias", _c_vp),
        ("scale", _c_vp),
        ("score_mod", _c_vp),
        ("seq_lens_q", _c_vp),
        ("seq_lens_k", _c_vp),
        ("causal", _c_i32),
        ("cu_seqlens_q", _c_vp),
        ("cu_seqlens_k", _c_vp),
        ("rows_q", _c_i64),
        ("rows_k", _c_i64),
    ]


# Exported symbols and their signatures (every function in include/sigattn.h).
SIGNATURES = {
    "sigattn_abi_version": ([], _c_i32),
    "sigattn_strerror": ([_c_i32], ctypes.c_char_p),
    "sigattn_check": ([ctypes.POINTER(SigattnProblem)], _c_i32),
    "sigattn_fwd": ([ctypes.POINTER(SigattnProblem), _c_vp, _c_vp], _c_i32),
    "sigattn_fwd_workspace_bytes": ([ctypes.POINTER(SigattnProblem)], ctypes.c_size_t),
    "sigattn_fwd_ws": ([ctypes.POINTER(SigattnProblem), _c_vp, _c_vp, ctypes.c_size_t, _c_vp], _c_i32),
    "sigattn_fwd_noalloc": ([ctypes.POINTER(SigattnProblem), _c_vp, _c_vp], _c_i32),
    "sigattn_bwd": ([ctypes.POINTER(SigattnProblem), _c_vp, _c_vp, _c_vp, _c_vp, _c_vp], _c_i32),
    "sigattn_bwd_dq": ([ctypes.POINTER(SigattnProblem), _c_vp, _c_vp, _c_vp], _c_i32),
    "sigattn_bwd_dkdv": ([ctypes.POINTER(SigattnProblem), _c_vp, _c_vp, _c_vp, _c_vp], _c_i32),
    "sigattn_bwd_workspace_bytes": ([ctypes.POINTER(SigattnProblem)], ctypes.c_size_t),
    "sigattn_bwd_ws": ([ctypes.POINTER(SigattnProblem), _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, ctypes.c_size_t,
                        _c_vp], _c_i32),
    "sigattn_bwd_dkdv_ws": ([ctypes.POINTER(SigattnProblem), _c_vp, _c_vp, _c_vp, _c_vp, ctypes.c_size_t,
                             _c_vp], _c_i32),
    "sigattn_bwd_dq_ws": ([ctypes.POINTER(SigattnProblem), _c_vp, _c_vp, ctypes.c_size_t, _c_vp], _c_i32),
    "sigattn_bwd_split_workspace_bytes": ([ctypes.POINTER(SigattnProblem)], ctypes.c_size_t),
    "sigattn_bwd_split": ([ctypes.POINTER(SigattnProblem), _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, ctypes.c_size_t,
                           _c_vp], _c_i32),
}

_lib = None
_lib_lock = threading.Lock()
_checked_devices: set[int] = set()


def load_library(path: Optional[Path] = None) -> ctypes.CDLL:
    """Loads (once) and returns the C ABI library; raises if it is not built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lib_lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"{p.name} is not built ({p}); build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` at the repository root"
            )
        lib = ctypes.CDLL(str(p))
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = restype
        if lib.sigattn_abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"{p.name} ABI version {lib.sigattn_abi_version()} != expected {ABI_VERSION}"
            )
        if path is None:
            _lib = lib
        return lib


# C++ autograd node of the eager public APIs (csrc/torch_autograd.cpp,
# _sigattn_autograd next to this file): the same kernels, launch policy,
# saved tensors and gradients as the Python nodes (torch.autograd.Function
# in the op modules) with far less host time per call, and a backward that
# runs on the autograd engine's device thread without taking the GIL.  The
# environment variable SIGATTN_EAGER_BINDING=python selects the Python nodes;
# so does a node that fails to import (with a warning).
_EAGER_ENV = "SIGATTN_EAGER_BINDING"
_AUTOGRAD_FNS = ("sigattn_strerror", "sigattn_fwd_workspace_bytes", "sigattn_fwd_ws",
                 "sigattn_bwd_workspace_bytes", "sigattn_bwd_ws", "sigattn_bwd_split_workspace_bytes",
                 "sigattn_bwd_split")
_autograd = None  # the bound module, or False after a failed import


def autograd_node():
    """The bound C++ autograd module, or None when the Python nodes serve."""
    global _autograd
    if os.environ.get(_EAGER_ENV, "").strip().lower() == "python":
        return None
    if _autograd is None:
        lib = load_library()
        try:
            from . import _sigattn_autograd as mod
        except ImportError as e:
            warnings.warn(f"sigmoid attention: C++ autograd node not loaded ({e}); the Python node serves the "
                          "eager APIs, with more host time per call")
            _autograd = False
            return None
        mod.bind({n: ctypes.cast(getattr(lib, n), ctypes.c_void_p).value for n in _AUTOGRAD_FNS},
                 list(TWO_PASS_HEAD_DIMS), _DQ_DS_ROWS)
        _autograd = mod
    return _autograd or None


def attention_node(node, Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k, causal) -> torch.Tensor:
    """O with autograd through the C++ node on the canonical op inputs."""
    Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k = _prepare(
        Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k)
    return node.attention(Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k, bool(causal),
                          bwd_workspace_limit())


def attention_node_packed(node, Q, K, V, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, bias,
                          score_mod, sm_scale, causal) -> torch.Tensor:
    """attention_node for packed [rows, H, D] tensors (cu_seqlens layout)."""
    Q, K, V, bias, score_mod, sm_scale, _, _ = _prepare(Q, K, V, bias, score_mod, sm_scale, None, None)
    cu_q, cu_k = _prepare_packed(cu_seqlens_q, cu_seqlens_k, Q.device)
    return node.attention(Q, K, V, bias, score_mod, sm_scale, None, None, bool(causal), bwd_workspace_limit(),
                          cu_q, cu_k, int(max_seqlen_q), int(max_seqlen_k))


def strerror(code: int) -> str:
    return load_library().sigattn_strerror(code).decode()


def _check_device(t: torch.Tensor) -> None:
    if t.device.type != "cuda" or torch.version.hip is None:
        raise RuntimeError(
            "sigmoid attention kernels need tensors on an AMD gfx950 (MI355X) GPU under "
            f"PyTorch-ROCm; got a tensor on '{t.device}'"
        )
    idx = t.device.index if t.device.index is not None else torch._C._cuda_getDevice()
    if idx in _checked_devices:
        return
    arch = torch.cuda.get_device_properties(idx).gcnArchName.split(":")[0]
    if arch != "gfx950":
        raise RuntimeError(f"sigmoid attention kernels are built for gfx950 only; device {idx} is {arch}")
    _checked_devices.add(idx)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _problem(Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k, causal,
             packed=None) -> SigattnProblem:
    """One sigattn_problem.  `packed` = (cu_seqlens_q, cu_seqlens_k,
    max_seqlen_q, max_seqlen_k) for [rows, H, D] tensors, else [B, T, H, D]."""
    pr = SigattnProblem()
    if packed is None:
        B, Tq, H, D = Q.shape
        Tk = K.shape[1]
        qs, ks = Q.stride(), K.stride()
    else:
        cu_q, cu_k, Tq, Tk = packed
        B = cu_q.numel() - 1
        H, D = Q.shape[1], Q.shape[2]
        qs, ks = (0,) + Q.stride(), (0,) + K.stride()
        pr.cu_seqlens_q, pr.cu_seqlens_k = _ptr(cu_q), _ptr(cu_k)
        pr.rows_q, pr.rows_k = Q.shape[0], K.shape[0]
    pr.abi_version = ABI_VERSION
    pr.dtype = _DTYPE_CODE[Q.dtype]
    pr.B, pr.Tq, pr.Tk, pr.H, pr.D = B, Tq, Tk, H, D
    pr.q_stride_b, pr.q_stride_t, pr.q_stride_h = qs[0], qs[1], qs[2]
    pr.k_stride_b, pr.k_stride_t, pr.k_stride_h = ks[0], ks[1], ks[2]
    pr.q, pr.k, pr.v = _ptr(Q), _ptr(K), _ptr(V)
    pr.bias, pr.scale = _ptr(bias), _ptr(sm_scale)
    pr.score_mod = _ptr(score_mod)
    pr.seq_lens_q, pr.seq_lens_k = _ptr(seq_lens_q), _ptr(seq_lens_k)
    pr.causal = 1 if causal else 0
    return pr


def _prepare(Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k):
    """Canonicalises op inputs: contiguous rows, fp32 bias/scale/score_mod,
    int32 seq_lens, everything on Q's device."""
    if Q.dtype not in _DTYPE_CODE:
        raise RuntimeError(f"unsupported dtype {Q.dtype}; expected float16, bfloat16 or float32")
    if K.dtype != Q.dtype or V.dtype != Q.dtype:
        raise RuntimeError(f"Q, K, V must share a dtype, got {Q.dtype}, {K.dtype}, {V.dtype}")
    _check_device(Q)
    dev = Q.device
    Q, K, V = Q.contiguous(), K.contiguous(), V.contiguous()
    for name, t in (("K", K), ("V", V)):
        if t.device != dev:
            raise RuntimeError(f"{name} is on {t.device}, expected {dev}")
    bias = _as(bias, torch.float32, dev)
    sm_scale = _as(sm_scale, torch.float32, dev)
    if sm_scale.dim() != 0:
        sm_scale = sm_scale.reshape(())
    score_mod = _as(score_mod, torch.float32, dev)
    seq_lens_q = _as(seq_lens_q, torch.int32, dev)
    seq_lens_k = _as(seq_lens_k, torch.int32, dev)
    return Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k


def _as(t: Optional[torch.Tensor], dtype: torch.dtype, dev: torch.device) -> Optional[torch.Tensor]:
    """t as a contiguous `dtype` tensor on `dev` (t itself when it already is)."""
    if t is None or (t.dtype == dtype and t.device == dev and t.is_contiguous()):
        return t
    return t.to(device=dev, dtype=dtype).contiguous()


def _on_device(dev: torch.device, fn):
    """fn(stream) with `dev` current and torch's current HIP stream of it.

    Reads the device and raw stream through torch's C bindings (the ones
    Triton's launcher uses): torch.cuda.current_stream() resolves the device
    through several Python layers and costs ~20 µs per call."""
    cur = torch._C._cuda_getDevice()
    idx = cur if dev.index is None else dev.index
    if idx == cur:
        return fn(torch._C._cuda_getCurrentRawStream(idx))
    with torch.cuda.device(idx):
        return fn(torch._C._cuda_getCurrentRawStream(idx))


def _launch_fwd(lib, pr: SigattnProblem, out: torch.Tensor) -> None:
    """sigattn_fwd_ws with the workspace the problem asks for (decode shapes
    split their keys over several workgroups; others need none), allocated
    from torch's caching allocator on the output's device."""
    def run(stream):
        nbytes = int(lib.sigattn_fwd_workspace_bytes(ctypes.byref(pr)))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=out.device) if nbytes else None
        _raise(lib.sigattn_fwd_ws(ctypes.byref(pr), out.data_ptr(), _ptr(ws), nbytes, stream), "sigattn_fwd")

    _on_device(out.device, run)


# Two-pass backward (dS stored by the dK/dV kernel, dQ = dS·K read back):
# head dims it is used for, and the most workspace it may take (larger
# problems run their heads in groups that fit).  At D = 128 it replaces the dQ
# kernel's 4·D-FLOP recomputation of S and dP per pair with 2 bytes of dS
# written and read back.
TWO_PASS_HEAD_DIMS = (128,)
_WS_ENV = "SIGATTN_BWD_WORKSPACE_MB"
_WS_DEFAULT_MB = 2048


def bwd_workspace_limit() -> int:
    """Largest two-pass backward workspace in bytes (0 disables the path);
    environment variable SIGATTN_BWD_WORKSPACE_MB, default 2048."""
    raw = os.environ.get(_WS_ENV)
    mb = _WS_DEFAULT_MB if raw is None or raw.strip() == "" else int(raw)
    return max(mb, 0) << 20


# Query rows per workgroup of the D = 128 dQ-from-dS kernel on grids that
# would not fill the GPU with its 512-row workgroups (the library then
# launches 256-row ones).
_DQ_DS_ROWS = 256
_CU_COUNT: dict = {}


def _compute_units(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch._C._cuda_getDevice()
    n = _CU_COUNT.get(idx)
    if n is None:
        n = _CU_COUNT[idx] = int(torch.cuda.get_device_properties(idx).multi_processor_count)
    return n


def bwd_workspace_bytes(lib, pr: SigattnProblem, device: torch.device) -> int:
    """Workspace this layer gives sigattn_bwd_ws (0: the recompute backward).

    The whole problem's dS when it fits bwd_workspace_limit(); otherwise the
    largest whole number of heads that fits, run by the library one group
    after another.  Groups whose dQ-from-dS grid (in workgroups of 256 query
    rows) has fewer workgroups than the GPU has compute units take the
    recompute backward instead.  Measured at D=128 bf16 (ms, two-pass in
    head groups against recompute): non-causal B=1 L=16384 H=16 in groups
    of 4 heads (256 workgroups) 6.04-6.05 against 6.90-6.91, B=2 L=8192
    H=16 in groups of 8 3.00-3.02 against 3.49; causal B=1 L=16384 H=16 in
    groups of 4 3.57-3.59 against 3.56-3.57."""
    if pr.D not in TWO_PASS_HEAD_DIMS:
        return 0
    full = int(lib.sigattn_bwd_workspace_bytes(ctypes.byref(pr)))
    limit = bwd_workspace_limit()
    if full <= limit:
        return full
    per_head = full // pr.H
    heads = limit // per_head
    grid = heads * pr.B * -(-pr.Tq // _DQ_DS_ROWS)
    if heads == 0 or grid < _compute_units(device):
        return 0
    return heads * per_head


def _bwd_workspace(nbytes: int, device: torch.device):
    """The two-pass backward's dS workspace, or None when it is not used or
    the device cannot hold it: the recompute backward needs no workspace, so
    an allocation failure falls back to it instead of failing the backward
    (the reference's backward allocates only its outputs)."""
    if nbytes == 0:
        return None, 0
    try:
        return torch.empty(nbytes, dtype=torch.uint8, device=device), nbytes
    except torch.OutOfMemoryError:
        return None, 0


def _launch_bwd(lib, pr: SigattnProblem, dO, dQ, dK, dV) -> None:
    """The backward, with workspaces from torch's caching allocator.  A
    small dense grid that splits (sigattn_bwd_split_workspace_bytes > 0)
    takes the range-split recompute backward, measured faster than the
    two-pass one wherever it applies (D = 128 non-causal, GPU time:
    B=2 L=1024 H=8 76.3 -> 63.3 us, B=1 L=4096 H=2 232 -> 150 us).  Otherwise
    the head dims in TWO_PASS_HEAD_DIMS take sigattn_bwd_ws with the two-pass
    workspace (bwd_workspace_bytes), and the rest sigattn_bwd_split without
    one, i.e. the recompute kernels.  A workspace that cannot be allocated
    falls back to the kernels that need none."""
    def run(stream):
        split = int(lib.sigattn_bwd_split_workspace_bytes(ctypes.byref(pr)))
        if split > 0 or pr.D not in TWO_PASS_HEAD_DIMS:
            ws, nbytes = _bwd_workspace(split, dQ.device)
            _raise(lib.sigattn_bwd_split(ctypes.byref(pr), _ptr(dO), _ptr(dQ), _ptr(dK), _ptr(dV), _ptr(ws),
                                         nbytes, stream), "sigattn_bwd_split")
            return
        ws, nbytes = _bwd_workspace(bwd_workspace_bytes(lib, pr, dQ.device), dQ.device)
        _raise(lib.sigattn_bwd_ws(ctypes.byref(pr), _ptr(dO), _ptr(dQ), _ptr(dK), _ptr(dV), _ptr(ws), nbytes,
                                  stream), "sigattn_bwd_ws")

    _on_device(dQ.device, run)


def _raise(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed: {strerror(rc)} (status {rc})")


def forward(Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k, causal) -> torch.Tensor:
    """O = sigmoid(QKᵀ·scale + bias + score_mod)·V via sigattn_fwd."""
    lib = load_library()
    Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k = _prepare(
        Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k)
    out = torch.empty_like(Q)
    if out.numel() == 0:
        return out
    pr = _problem(Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k, causal)
    _launch_fwd(lib, pr, out)
    return out


def forward_eager(Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k, causal):
    """forward() for the eager autograd paths.  Also returns the launched
    problem when it points at exactly the tensors given (none needed a copy
    or conversion), which the caller saves for the backward; backward_eager
    then launches on it without validating and describing the problem a
    second time.  Otherwise the problem is None."""
    lib = load_library()
    given = (Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k)
    canon = _prepare(*given)
    out = torch.empty_like(canon[0])
    if out.numel() == 0:
        return out, None
    pr = _problem(*canon, causal)
    _launch_fwd(lib, pr, out)
    return out, (pr if all(a is b for a, b in zip(given, canon)) else None)


def _problem_points_at(pr: SigattnProblem, Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k) -> bool:
    """True when every pointer of `pr` is the address of the matching tensor.
    Saved-tensor hooks (torch.autograd.graph.save_on_cpu, non-reentrant
    checkpointing) hand the backward new tensors at new addresses, and the
    forward's buffers may since have been freed and reused."""
    pairs = ((pr.q, Q), (pr.k, K), (pr.v, V), (pr.bias, bias), (pr.scale, sm_scale), (pr.score_mod, score_mod),
             (pr.seq_lens_q, seq_lens_q), (pr.seq_lens_k, seq_lens_k))
    return all((p or None) == _ptr(t) for p, t in pairs) and all(
        t is None or t.is_contiguous() for t in (Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k))


def backward_eager(pr, Q, K, V, dO, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k, causal):
    """backward() on the problem forward_eager returned, when that problem
    still points at exactly the saved tensors given here (which then keep
    every pointer in it alive); backward() itself otherwise -- no problem, or
    saved tensors that a saved-tensor hook moved."""
    if pr is None or not _problem_points_at(pr, Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k):
        return backward(Q, K, V, dO, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k, causal)
    lib = load_library()
    dO = _as(dO, Q.dtype, Q.device)
    if dO.shape != Q.shape:
        raise RuntimeError(f"dO shape {tuple(dO.shape)} != Q shape {tuple(Q.shape)}")
    dQ, dK, dV = torch.empty_like(Q), torch.empty_like(K), torch.empty_like(V)
    if dQ.numel() == 0 and dK.numel() == 0:
        return dQ, dK, dV
    _launch_bwd(lib, pr, dO, dQ, dK, dV)
    return dQ, dK, dV


def backward(Q, K, V, dO, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k, causal):
    """(dQ, dK, dV) via sigattn_bwd_ws: the two-pass backward (dK/dV kernel
    storing dS, then dQ from dS) where it applies, else the recompute backward
    (dQ kernel, then dK/dV kernel)."""
    lib = load_library()
    Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k = _prepare(
        Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k)
    dO = _as(dO, Q.dtype, Q.device)
    if dO.shape != Q.shape:
        raise RuntimeError(f"dO shape {tuple(dO.shape)} != Q shape {tuple(Q.shape)}")
    dQ, dK, dV = torch.empty_like(Q), torch.empty_like(K), torch.empty_like(V)
    if dQ.numel() == 0 and dK.numel() == 0:
        return dQ, dK, dV
    pr = _problem(Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k, causal)
    _launch_bwd(lib, pr, dO, dQ, dK, dV)
    return dQ, dK, dV


def _prepare_packed(cu_seqlens_q, cu_seqlens_k, dev):
    cu_q = cu_seqlens_q.to(device=dev, dtype=torch.int32).contiguous()
    cu_k = cu_seqlens_k.to(device=dev, dtype=torch.int32).contiguous()
    if cu_q.shape != cu_k.shape or cu_q.dim() != 1 or cu_q.numel() < 1:
        raise RuntimeError(f"cu_seqlens_q {tuple(cu_q.shape)} and cu_seqlens_k {tuple(cu_k.shape)} "
                           "must both be [B + 1]")
    return cu_q, cu_k


def _packed_dims(Q, K, cu_q, cu_k, max_seqlen_q, max_seqlen_k):
    # An axis with no rows has no valid positions whatever max_seqlen says.
    Tq = int(max_seqlen_q) if Q.shape[0] > 0 else 0
    Tk = int(max_seqlen_k) if K.shape[0] > 0 else 0
    return cu_q, cu_k, Tq, Tk


def forward_packed(Q, K, V, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, bias, score_mod,
                   sm_scale, causal) -> torch.Tensor:
    """Forward for packed [rows, H, D] tensors via sigattn_fwd (cu_seqlens set)."""
    lib = load_library()
    Q, K, V, bias, score_mod, sm_scale, _, _ = _prepare(Q, K, V, bias, score_mod, sm_scale, None, None)
    cu_q, cu_k = _prepare_packed(cu_seqlens_q, cu_seqlens_k, Q.device)
    if cu_q.numel() == 1:
        return torch.zeros_like(Q)  # no sequences: every packed row is outside them
    out = torch.empty_like(Q)
    if out.numel() == 0:
        return out
    pr = _problem(Q, K, V, bias, score_mod, sm_scale, None, None, causal,
                  packed=_packed_dims(Q, K, cu_q, cu_k, max_seqlen_q, max_seqlen_k))
    _launch_fwd(lib, pr, out)
    return out


def backward_packed(Q, K, V, dO, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, bias, score_mod,
                    sm_scale, causal):
    """(dQ, dK, dV) for packed [rows, H, D] tensors via sigattn_bwd_ws."""
    lib = load_library()
    Q, K, V, bias, score_mod, sm_scale, _, _ = _prepare(Q, K, V, bias, score_mod, sm_scale, None, None)
    cu_q, cu_k = _prepare_packed(cu_seqlens_q, cu_seqlens_k, Q.device)
    dO = _as(dO, Q.dtype, Q.device)
    if dO.shape != Q.shape:
        raise RuntimeError(f"dO shape {tuple(dO.shape)} != Q shape {tuple(Q.shape)}")
    if cu_q.numel() == 1:
        return torch.zeros_like(Q), torch.zeros_like(K), torch.zeros_like(V)
    dQ, dK, dV = torch.empty_like(Q), torch.empty_like(K), torch.empty_like(V)
    if dQ.numel() == 0 and dK.numel() == 0:
        return dQ, dK, dV
    pr = _problem(Q, K, V, bias, score_mod, sm_scale, None, None, causal,
                  packed=_packed_dims(Q, K, cu_q, cu_k, max_seqlen_q, max_seqlen_k))
    _launch_bwd(lib, pr, dO, dQ, dK, dV)
    return dQ, dK, dV


_CONSTANTS: dict = {}
_CONSTANTS_MAX = 256


def device_constant(shape, value, dtype: torch.dtype, device) -> torch.Tensor:
    """A device tensor of `shape` filled with `value`, for the per-call bias /
    scale / default-length tensors of the public APIs.  Eagerly the tensor is
    made once per (shape, value, dtype, device) by a blocking host-to-device
    copy (complete before first use on any stream), kept for the life of the
    process and reused, so a call launches no fill kernels; under torch.compile it is an ordinary
    torch.full in the graph, and under CUDA-graph capture a captured fill.
    Callers never write to it."""
    dev = torch.device(device)
    if (torch.compiler.is_compiling() or dev.type != "cuda"
            or torch._C._cuda_isCurrentStreamCapturing()):
        return torch.full(shape, value, dtype=dtype, device=dev)
    if dev.index is None:
        dev = torch.device("cuda", torch._C._cuda_getDevice())
    key = (tuple(shape), float(value), dtype, dev)
    t = _CONSTANTS.get(key)
    if t is None:
        if len(_CONSTANTS) >= _CONSTANTS_MAX:
            # Cached tensors are never freed: a kernel still queued on any
            # stream may read one.  Past the cap, a per-call tensor filled on
            # the current stream (freed by torch's allocator in that stream's
            # order) takes its place.
            return torch.full(shape, value, dtype=dtype, device=dev)
        t = torch.full(shape, value, dtype=dtype).to(dev)
        _CONSTANTS[key] = t
    return t
