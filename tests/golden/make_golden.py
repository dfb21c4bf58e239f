"""Writes the golden fixtures tests/golden/*.npz from the float64 oracle.

Inputs are drawn from a seeded numpy generator and rounded to the case's I/O
dtype, so a device tensor built from them holds exactly the same values.
Expected outputs are the oracle's forward and backward (float64, with P and dS
rounded to the I/O dtype as the kernels do).  The bias and scale are stored as
the fp32 values the public API passes to the kernels.

Run from the repository root:  python tests/golden/make_golden.py
"""

import math
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import sigmoid_oracle as so  # noqa: E402

OUT = Path(__file__).resolve().parent

CASES = {
    "dense_causal_bf16_d64": dict(B=1, Tq=33, Tk=33, H=2, D=64, io="bf16", causal=True, padded=False, sm=False),
    "padded_cross_bf16_d128": dict(B=2, Tq=20, Tk=45, H=1, D=128, io="bf16", causal=False, padded=True, sm=True),
    "padded_causal_f16_d64": dict(B=2, Tq=40, Tk=40, H=2, D=64, io="f16", causal=True, padded=True, sm=False),
    "dense_f16_d16": dict(B=2, Tq=50, Tk=50, H=1, D=16, io="f16", causal=False, padded=False, sm=False),
    "dense_f32_d32": dict(B=1, Tq=24, Tk=24, H=3, D=32, io="f32", causal=True, padded=False, sm=True),
}


def make(name, c, seed):
    rng = np.random.default_rng(seed)
    B, Tq, Tk, H, D = c["B"], c["Tq"], c["Tk"], c["H"], c["D"]
    q, k, v, do = (so.round_to(rng.standard_normal(s), c["io"])
                   for s in [(B, Tq, H, D), (B, Tk, H, D), (B, Tk, H, D), (B, Tq, H, D)])
    sq = sk = None
    if c["padded"]:
        sq = rng.integers(Tq // 3, Tq + 1, size=B)
        sk = rng.integers(Tk // 3, Tk + 1, size=B)
        sq[0], sk[0] = Tq, Tk
        bias = (-np.log(sk.astype(np.float32))).astype(np.float32).astype(np.float64)
    else:
        bias = np.full(B, np.float32(-math.log(Tk)), dtype=np.float64)
    sm = so.round_to(rng.standard_normal((B, Tk)), "f32") if c["sm"] else None
    scale = float(np.float32(1.0 / math.sqrt(D)))
    kw = dict(scale=scale, bias=bias, score_mod=sm, seq_lens_q=sq, seq_lens_k=sk, causal=c["causal"],
              io_dtype=c["io"])
    o = so.forward(q, k, v, **kw)
    dq, dk, dv = so.backward(q, k, v, do, **kw)
    arrays = dict(q=q, k=k, v=v, dout=do, bias=bias, scale=np.array(scale), causal=np.array(c["causal"]),
                  io=np.array(c["io"]), out=o, dq=dq, dk=dk, dv=dv)
    if sq is not None:
        arrays.update(seq_lens_q=sq.astype(np.int32), seq_lens_k=sk.astype(np.int32))
    if sm is not None:
        arrays["score_mod"] = sm
    np.savez_compressed(OUT / f"{name}.npz", **arrays)


if __name__ == "__main__":
    for i, (name, c) in enumerate(sorted(CASES.items())):
        make(name, c, seed=1000 + i)
        print("wrote", name)
