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



def criterion_errors(q, k, v, do, ours_fn, eager_kw, q_valid=None, k_valid=None):
    """The reference tests' error pair (tests/test_sigmoid_dense.py:77-166,
    tests/test_sigmoid_padded.py:76-186): max-abs error of our kernel and of
    the mixed-precision eager path (upcast=False, reorder_ops=True), both
    against the fp32 eager path (upcast=True), for O, dQ, dK, dV.

    Both run on the inputs' device.  The fp32 path goes through autograd in
    fp32; the mixed-precision path is oracle/eager.py's mixed_fwd_bwd, whose
    bf16 / fp16 products all take contiguous operands (autograd through the
    eager einsums would hand torch's batched products transposed views, which
    this pool's GPUs must not be given in bf16).
    q_valid [B, Tq] / k_valid [B, Tk] (bool) restrict errors to valid rows.
    Returns {name: (err_ours, err_mixed)}."""
    from oracle.eager import mixed_fwd_bwd, sigmoid_attention_eager
    dev = q.device
    qm = None if q_valid is None else q_valid.to(dev)[:, :, None, None]
    km = None if k_valid is None else k_valid.to(dev)[:, :, None, None]

    def run(fn, tensors):
        leaves = [t.detach().clone().requires_grad_(True) for t in tensors[:3]]
        o = fn(*leaves)
        o.backward(tensors[3].to(o.dtype))
        return [o.detach()] + [t.grad for t in leaves]

    ours = run(ours_fn, (q, k, v, do))
    ref = run(lambda a, b, c: sigmoid_attention_eager(a, b, c, upcast=True, **eager_kw), (q, k, v, do))
    mixed = mixed_fwd_bwd(q, k, v, do, **eager_kw)
    out = {}
    for i, name in enumerate(("O", "dQ", "dK", "dV")):
        mask = qm if name in ("O", "dQ") else km
        r = ref[i].float()
        e = (ours[i].float() - r)
        em = (mixed[i].to(dev).float() - r)
        if mask is not None:
            e, em = e * mask, em * mask
        out[name] = (e.abs().max().item(), em.abs().max().item())
    return out


def assert_reference_criterion(errs, tol):
    """fwd: err <= 2 err_mixed + tol and err < tol; bwd: 3x (the reference's
    tests/test_sigmoid_dense.py:111-114,154-166)."""
    for name, (e, em) in errs.items():
        f = 2.0 if name == "O" else 3.0
        assert e <= f * em + tol, (name, e, em, tol)
        assert e < tol, (name, e, tol)
