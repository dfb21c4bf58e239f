"""TEST INFRASTRUCTURE ONLY — CPU oracle for fused sigmoid attention.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker.  The product path (triton_sigmoid) never
imports it.

A numpy restatement (float64 by default) of the reference's kernel semantics,
MSDLLCpapers/triton-sigmoid:
  forward  — _fwd_dense_kernel, src/triton_sigmoid/sigmoid_triton_dense.py:23-154,
             _fwd_padded_kernel, src/triton_sigmoid/sigmoid_triton_padded.py:24-171:
      S = (Q·Kᵀ)·scale + bias[b]                 (:123, :126)
      S += score_mod[b, key]                     (:129-133)
      mask: key < Lk, query < Lq, causal key <= query (:136-143; padded :92, :127)
      P = sigmoid(S), masked P = 0               (:143-146)
      P rounded to the I/O dtype before P·V      (:149)
      padded query rows of O are 0               (padded :93, :171)
  backward — _bwd_dense_dq_kernel / _bwd_dense_dkdv_kernel (:162-307, :315-467)
             and the padded variants (sigmoid_triton_padded.py:179-339, :342-509):
      dP = dO·Vᵀ; dS = P(1-P)dP; masked dS = 0    (:289-296)
      dQ = round(dS)·K·scale                     (:299-302)
      dV = round(P)ᵀ·dO; dK = round(dS)ᵀ·Q·scale  (:443, :456-459)
      padded rows of dQ / dK / dV are 0.
The default biases are those of the reference's public APIs:
-log(T) (sigmoid_triton_dense.py:840-841) and -log(seq_lens_k)
(sigmoid_triton_padded.py:995-996), both without an epsilon.

Pinning (tests/test_oracle.py): closed forms (q=k=0, q=k=v=1 with causal row
counts, T=1 backward), pure-Python brute-force loops on tiny shapes, central
finite differences of `forward` against `backward`, torch.autograd in float64,
invariants (causality, padding-noise invariance, linearity in V, split-KV
additivity, constant score_mod == bias shift), and the committed golden
fixtures under tests/golden/.
"""

from __future__ import annotations

import math
from typing import Optional

import numpy as np

__all__ = [
    "round_to",
    "lengths",
    "valid_mask",
    "default_bias",
    "scores",
    "forward",
    "backward",
    "sigmoid",
]


def sigmoid(x: np.ndarray) -> np.ndarray:
    """Numerically stable logistic function (exact limits at ±inf)."""
    x = np.asarray(x, dtype=np.float64)
    out = np.empty_like(x)
    pos = x >= 0
    out[pos] = 1.0 / (1.0 + np.exp(-x[pos]))
    ex = np.exp(x[~pos])
    out[~pos] = ex / (1.0 + ex)
    return out


def round_to(x: np.ndarray, dtype: Optional[str]) -> np.ndarray:
    """Rounds to 'f16', 'bf16' or 'f32' (round-to-nearest-even) and returns float64.

    None returns x unchanged (no intermediate rounding)."""
    x = np.asarray(x, dtype=np.float64)
    if dtype is None:
        return x
    if dtype == "f32":
        return x.astype(np.float32).astype(np.float64)
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float64)
    if dtype == "bf16":
        f = np.ascontiguousarray(x.astype(np.float32))
        u = f.view(np.uint32).astype(np.uint64)
        rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
        nan = np.isnan(f)
        out = (rounded & 0xFFFFFFFF).astype(np.uint32).view(np.float32).astype(np.float64)
        out[nan] = np.nan
        return out
    raise ValueError(f"unknown dtype {dtype!r}")


def lengths(T: int, B: int, seq_lens: Optional[np.ndarray]) -> np.ndarray:
    """Valid lengths per batch element, clamped to [0, T] (None = T)."""
    if seq_lens is None:
        return np.full((B,), T, dtype=np.int64)
    return np.clip(np.asarray(seq_lens, dtype=np.int64), 0, T)


def valid_mask(B, Tq, Tk, seq_lens_q=None, seq_lens_k=None, causal=False) -> np.ndarray:
    """[B, 1, Tq, Tk] bool: query < Lq, key < Lk and (causal) key <= query."""
    Lq = lengths(Tq, B, seq_lens_q)
    Lk = lengths(Tk, B, seq_lens_k)
    qi = np.arange(Tq)[None, :, None]
    kj = np.arange(Tk)[None, None, :]
    m = (qi < Lq[:, None, None]) & (kj < Lk[:, None, None])
    if causal:
        m = m & (kj <= qi)
    return m[:, None, :, :]


def default_bias(B: int, T: int, seq_lens_k: Optional[np.ndarray] = None) -> np.ndarray:
    """Reference API default bias: -log(T) dense, -log(seq_lens_k) padded (no eps)."""
    if seq_lens_k is None:
        return np.full((B,), -math.log(T), dtype=np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        return -np.log(np.asarray(seq_lens_k, dtype=np.float64))


def scores(q, k, scale, bias, score_mod=None) -> np.ndarray:
    """S[b, h, i, j] = (q[b,i,h]·k[b,j,h])·scale + bias[b] (+ score_mod[b, j])."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    s = np.einsum("bihd,bjhd->bhij", q, k) * scale
    s = s + np.asarray(bias, dtype=np.float64)[:, None, None, None]
    if score_mod is not None:
        s = s + np.asarray(score_mod, dtype=np.float64)[:, None, None, :]
    return s


def _probabilities(q, k, scale, bias, score_mod, seq_lens_q, seq_lens_k, causal):
    B, Tq = q.shape[0], q.shape[1]
    Tk = k.shape[1]
    m = valid_mask(B, Tq, Tk, seq_lens_q, seq_lens_k, causal)
    s = scores(q, k, scale, bias, score_mod)
    with np.errstate(invalid="ignore", over="ignore"):
        p = np.where(m, sigmoid(np.where(m, s, 0.0)), 0.0)
    return p, m


def forward(q, k, v, *, scale, bias, score_mod=None, seq_lens_q=None, seq_lens_k=None,
            causal=False, io_dtype: Optional[str] = None) -> np.ndarray:
    """O[B, Tq, H, D] in float64.  `io_dtype` ('f16'/'bf16'/'f32') rounds P
    the way the kernels do before P·V; None keeps P exact."""
    B, Tq = q.shape[0], q.shape[1]
    p, _ = _probabilities(q, k, scale, bias, score_mod, seq_lens_q, seq_lens_k, causal)
    p = round_to(p, io_dtype)
    o = np.einsum("bhij,bjhd->bihd", p, np.asarray(v, dtype=np.float64))
    Lq = lengths(Tq, B, seq_lens_q)
    o[np.arange(Tq)[None, :] >= Lq[:, None]] = 0.0
    return o


def backward(q, k, v, dout, *, scale, bias, score_mod=None, seq_lens_q=None, seq_lens_k=None,
             causal=False, io_dtype: Optional[str] = None):
    """(dQ, dK, dV) in float64 for the loss sum(O * dout)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    dout = np.asarray(dout, dtype=np.float64)
    B, Tq = q.shape[0], q.shape[1]
    Tk = k.shape[1]
    p, m = _probabilities(q, k, scale, bias, score_mod, seq_lens_q, seq_lens_k, causal)
    dp = np.einsum("bihd,bjhd->bhij", dout, v)
    ds = np.where(m, p * (1.0 - p) * dp, 0.0)
    pr = round_to(p, io_dtype)
    dsr = round_to(ds, io_dtype)
    dv = np.einsum("bhij,bihd->bjhd", pr, dout)
    dq = np.einsum("bhij,bjhd->bihd", dsr, k) * scale
    dk = np.einsum("bhij,bihd->bjhd", dsr, q) * scale
    Lq = lengths(Tq, B, seq_lens_q)
    Lk = lengths(Tk, B, seq_lens_k)
    dq[np.arange(Tq)[None, :] >= Lq[:, None]] = 0.0
    kpad = np.arange(Tk)[None, :] >= Lk[:, None]
    dk[kpad] = 0.0
    dv[kpad] = 0.0
    return dq, dk, dv
