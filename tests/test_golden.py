"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the float64 oracle): the oracle still reproduces them (CPU), and the HIP
kernels match them through the registered ops (GPU)."""

from pathlib import Path

import numpy as np
import pytest
import torch

import triton_sigmoid  # noqa: F401  (registers torch.ops.myops.*)
from helpers import ULP, assert_close_to_oracle
from oracle import sigmoid_oracle as so

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = sorted(p.stem for p in GOLDEN.glob("*.npz"))
TORCH_DTYPE = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _kw(g):
    return dict(scale=float(g["scale"]), bias=g["bias"], score_mod=g.get("score_mod"),
                seq_lens_q=g.get("seq_lens_q"), seq_lens_k=g.get("seq_lens_k"),
                causal=bool(g["causal"]), io_dtype=str(g["io"]))


def test_fixtures_present():
    assert len(CASES) >= 5


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_golden(name):
    g = _load(name)
    kw = _kw(g)
    np.testing.assert_array_equal(so.forward(g["q"], g["k"], g["v"], **kw), g["out"])
    for got, key in zip(so.backward(g["q"], g["k"], g["v"], g["dout"], **kw), ("dq", "dk", "dv")):
        np.testing.assert_array_equal(got, g[key])


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_kernels_match_golden(name):
    g = _load(name)
    dt = TORCH_DTYPE[str(g["io"])]
    dev = "cuda"
    q, k, v = (torch.tensor(g[n]).to(dt).to(dev).requires_grad_(True) for n in ("q", "k", "v"))
    do = torch.tensor(g["dout"]).to(dt).to(dev)
    bias = torch.tensor(g["bias"], dtype=torch.float32, device=dev)
    scale = torch.tensor(float(g["scale"]), dtype=torch.float32, device=dev)
    sm = torch.tensor(g["score_mod"], dtype=torch.float32, device=dev) if "score_mod" in g else None
    causal = bool(g["causal"])
    if "seq_lens_q" in g:
        sq = torch.tensor(g["seq_lens_q"], device=dev)
        sk = torch.tensor(g["seq_lens_k"], device=dev)
        o = torch.ops.myops.sigmoid_attn_padded_fwd(q, k, v, sk, sq, bias, sm, scale, causal)
    else:
        o = torch.ops.myops.sigmoid_attention_fwd(q, k, v, bias, sm, scale, causal)
    o.backward(do)
    assert_close_to_oracle(o, g["out"], dt, "O")
    assert_close_to_oracle(q.grad, g["dq"], dt, "dQ")
    assert_close_to_oracle(k.grad, g["dk"], dt, "dK")
    assert_close_to_oracle(v.grad, g["dv"], dt, "dV")
