"""Accuracy of the device sigmoid against the exact logistic function.

Every query sees exactly one key (padded API, seq_lens_k = 1) whose value row
is all ones, with q = [x, 0, ...], k = [1, 0, ...], scale 1 and bias 0, so
O[i, :] = sigmoid(x_i).  x sweeps [-30, 30].

The device computes sigmoid(x) = 1 / (1 + 2^(-x log2 e)) with the hardware
exp2 and reciprocal (the reference's accurate mode is tl.sigmoid,
src/triton_sigmoid/kernel_utils.py:236-237).  Rounding the exponent
-x log2 e to fp32 changes 2^(...) by a relative |x| 2^-24 (twice that where
the scale is folded into one FMA), which moves sigmoid by (1 - sigmoid) times
as much; exp2, the add and the reciprocal add a few ulps.  Bound used here,
relative to sigmoid(x):
    fp32 I/O:        2^-24 * (2 (1 - sigmoid(x)) (|x| + 2) + 8)
    bf16 / fp16 I/O: the above plus one ulp of the I/O type (P is rounded to
                     the I/O dtype before P·V, as the reference kernels do),
                     and for fp16 an absolute 2^-24 where P underflows.
At x = -30 the fp32 bound is 5.1e-6 relative (43 fp32 ulps); for |x| <= 1
it is below 1.3e-6.
"""

import math

import numpy as np
import pytest
import torch

import triton_sigmoid as ts

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL_ULP = {torch.float32: 0.0, torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}
# fp16 P underflows below 2^-24 (its subnormal spacing): absolute slack there.
ABS = {torch.float32: 0.0, torch.bfloat16: 0.0, torch.float16: 2.0 ** -24}


def _exact_sigmoid(x: np.ndarray) -> np.ndarray:
    out = np.empty_like(x)
    pos = x >= 0
    out[pos] = 1.0 / (1.0 + np.exp(-x[pos]))
    e = np.exp(x[~pos])
    out[~pos] = e / (1.0 + e)
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [64, 128])
def test_device_sigmoid_error_bound(dtype, D):
    Tq, Tk = 4096, 64
    xs = np.concatenate([np.linspace(-30.0, 30.0, Tq - 8), [0.0, 1e-3, -1e-3, 0.5, -16.0, 16.0, -30.0, 30.0]])
    xq = torch.tensor(xs, dtype=torch.float32).to(dtype)  # the exact inputs the kernel sees
    q = torch.zeros((1, Tq, 1, D), dtype=dtype)
    q[0, :, 0, 0] = xq
    g = torch.Generator().manual_seed(0)
    k = torch.randn((1, Tk, 1, D), generator=g).to(dtype)
    v = torch.randn((1, Tk, 1, D), generator=g).to(dtype)
    k[0, 0, 0] = 0
    k[0, 0, 0, 0] = 1
    v[0, 0, 0] = 1
    sk = torch.tensor([1], dtype=torch.int32, device=DEV)
    o = ts.sigmoid_attention_padded(q.to(DEV), k.to(DEV), v.to(DEV), seq_lens_k=sk, scale=1.0, sigmoid_bias=0.0)
    got = o[0, :, 0].double().cpu().numpy()
    assert np.all(got == got[:, :1]), "every column of a row must hold the same sigmoid"
    x = xq.double().numpy()
    want = _exact_sigmoid(x)
    rel = np.maximum(np.abs(got[:, 0] - want) - ABS[dtype], 0.0) / want
    bound = 2.0 ** -24 * (2.0 * (1.0 - want) * (np.abs(x) + 2.0) + 8.0) + REL_ULP[dtype]
    worst = int(np.argmax(rel / bound))
    assert np.all(rel <= bound), (f"x={x[worst]:.6g}: sigmoid {got[worst, 0]:.9g} vs exact {want[worst]:.9g}, "
                                  f"relative error {rel[worst]:.3e} > bound {bound[worst]:.3e}")
    if dtype == torch.float32:
        print(f"\n[sigmoid] fp32 D={D}: max relative error {rel.max():.3e} "
              f"({rel.max() / 2.0 ** -23:.1f} ulp), at x={x[int(np.argmax(rel))]:.4g}; "
              f"|x|<=1: {rel[np.abs(x) <= 1].max():.3e}")
