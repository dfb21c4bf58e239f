"""Helpers shared by the GPU parity tests."""

from __future__ import annotations

import numpy as np
import torch

from oracle import sigmoid_oracle as so

IO = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}
# Relative rounding step of one element of each I/O dtype (bound on the final
# store's rounding plus fp32-vs-fp64 accumulation differences).
ULP = {torch.float32: 2.0 ** -20, torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}


def randn(shape, dtype, device, gen, std=1.0):
    """Seeded N(0, std²) on the CPU generator, then moved (identical on every machine)."""
    return (torch.randn(shape, generator=gen, dtype=torch.float32) * std).to(dtype).to(device)


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().double().cpu().numpy()


def oracle_fwd_bwd(q, k, v, dout, *, scale, bias, score_mod=None, seq_lens_q=None,
                   seq_lens_k=None, causal=False, with_bwd=True):
    """float64 oracle on the exact (already rounded) device inputs."""
    dtype = q.dtype
    kw = dict(scale=scale, bias=np.asarray(bias, dtype=np.float64),
              score_mod=None if score_mod is None else to_np(score_mod),
              seq_lens_q=None if seq_lens_q is None else seq_lens_q.cpu().numpy(),
              seq_lens_k=None if seq_lens_k is None else seq_lens_k.cpu().numpy(),
              causal=causal, io_dtype=IO[dtype])
    o = so.forward(to_np(q), to_np(k), to_np(v), **kw)
    if not with_bwd:
        return o, None
    return o, so.backward(to_np(q), to_np(k), to_np(v), to_np(dout), **kw)


def assert_close_to_oracle(got: torch.Tensor, want: np.ndarray, dtype, name: str, factor: float = 2.0):
    """max|got - want| <= factor * ulp(dtype) * max|want| + tiny."""
    g = to_np(got)
    assert np.all(np.isfinite(g)), f"{name}: non-finite values"
    scale = float(np.abs(want).max()) if want.size else 0.0
    bound = factor * ULP[dtype] * scale + 1e-6
    err = float(np.abs(g - want).max()) if want.size else 0.0
    assert err <= bound, f"{name}: max abs err {err:.3e} > bound {bound:.3e} (max|ref| {scale:.3e})"
    return err
