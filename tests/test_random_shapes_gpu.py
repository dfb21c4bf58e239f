"""Seeded random configurations of the three public APIs against the float64
oracle: every head dim and dtype, odd sequence lengths, cross-attention,
causal, score_mod, explicit scale and bias, several batches and heads, in
combinations the fixed grids of the other tests do not reach.

Each case draws its configuration from one seeded generator (the same cases
on every machine), runs forward + backward through sigmoid_attention,
sigmoid_attention_padded or sigmoid_attention_varlen, and checks O, dQ, dK and
dV against oracle/sigmoid_oracle.py on the rounded device inputs, padding
rows and their score_mod entries filled with NaN where the layout has them
(they must never be read).  The semantics checked are the reference's
(sigmoid_triton_dense.py:23-154,162-467, sigmoid_triton_padded.py:24-509)."""

import math

import numpy as np
import pytest
import torch

import triton_sigmoid as ts
from helpers import assert_close_to_oracle, oracle_fwd_bwd, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float16, torch.bfloat16, torch.float32]
NCASES = 48


def _configs(n=NCASES, seed=20261202):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        api = ("dense", "padded", "varlen")[i % 3]
        dtype = DTYPES[int(rng.integers(3))]
        D = (16, 32, 64, 128)[int(rng.integers(4))]
        B, H = int(rng.integers(1, 5)), int(rng.integers(1, 5))
        Tq = int(rng.integers(1, 600))
        Tk = Tq if api == "dense" or rng.random() < 0.4 else int(rng.integers(1, 600))
        cfg = dict(api=api, dtype=dtype, D=D, B=B, H=H, Tq=Tq, Tk=Tk,
                   causal=bool(rng.random() < 0.5), score_mod=bool(rng.random() < 0.4),
                   bias=None if rng.random() < 0.5 else round(float(rng.uniform(-6.0, 1.0)), 3),
                   scale=None if rng.random() < 0.5 else round(float(rng.uniform(0.02, 0.3)), 4),
                   seed=int(rng.integers(1 << 30)))
        out.append(cfg)
    return out


def _id(c):
    dt = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}[c["dtype"]]
    flags = ("c" if c["causal"] else "") + ("m" if c["score_mod"] else "") + \
            ("b" if c["bias"] is not None else "") + ("s" if c["scale"] is not None else "")
    return f"{c['api']}-{dt}-D{c['D']}-B{c['B']}H{c['H']}-{c['Tq']}x{c['Tk']}-{flags or 'plain'}"


def _zero_past(t, lens):
    t = t.detach().clone()
    for b in range(t.shape[0]):
        t[b, int(lens[b]):] = 0
    return t


def _pack(x, lens):
    return torch.cat([x[b, :int(lens[b])] for b in range(x.shape[0])], 0)


@pytest.mark.parametrize("cfg", _configs(), ids=_id)
def test_random_configuration_matches_oracle(cfg):
    api, dtype, D, B, H, Tq, Tk = (cfg[k] for k in ("api", "dtype", "D", "B", "H", "Tq", "Tk"))
    causal = cfg["causal"]
    g = torch.Generator().manual_seed(cfg["seed"])
    q = randn((B, Tq, H, D), dtype, DEV, g)
    k = randn((B, Tk, H, D), dtype, DEV, g)
    v = randn((B, Tk, H, D), dtype, DEV, g)
    do = randn((B, Tq, H, D), dtype, DEV, g)
    sm = randn((B, Tk), dtype, DEV, g, 2.0) if cfg["score_mod"] else None
    if api == "dense":
        sq = torch.full((B,), Tq, dtype=torch.int32)
        sk = torch.full((B,), Tk, dtype=torch.int32)
    else:
        # Lengths from 1 to the full extent; one sequence of a batch is full.
        sq = torch.randint(1, Tq + 1, (B,), generator=g, dtype=torch.int32)
        sk = sq.clone() if Tq == Tk else torch.randint(1, Tk + 1, (B,), generator=g, dtype=torch.int32)
        j = int(torch.randint(B, (1,), generator=g))
        sq[j], sk[j] = Tq, Tk
    kw = dict(is_causal=causal, scale=cfg["scale"], sigmoid_bias=cfg["bias"])

    if api == "dense":
        leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
        o = ts.sigmoid_attention(*leaves, score_mod=sm, **kw)
        o.backward(do)
        got = [o.detach()] + [t.grad for t in leaves]
    elif api == "padded":
        qn, kn, vn, don = (t.clone() for t in (q, k, v, do))
        smn = None if sm is None else sm.clone()
        for b in range(B):  # padding rows hold NaN: they must never be read
            qn[b, int(sq[b]):] = float("nan")
            don[b, int(sq[b]):] = float("nan")
            kn[b, int(sk[b]):] = float("nan")
            vn[b, int(sk[b]):] = float("nan")
            if smn is not None:
                smn[b, int(sk[b]):] = float("nan")
        leaves = [t.requires_grad_(True) for t in (qn, kn, vn)]
        o = ts.sigmoid_attention_padded(*leaves, seq_lens_k=sk.to(DEV), seq_lens_q=sq.to(DEV), score_mod=smn, **kw)
        o.backward(don)
        got = [o.detach()] + [t.grad for t in leaves]
        for name, t, lens in zip(("O", "dQ", "dK", "dV"), got, (sq, sq, sk, sk)):
            for b in range(B):
                assert torch.all(t[b, int(lens[b]):] == 0), f"{name}: padding rows of batch {b} not zero"
    else:
        cu = lambda lens: torch.cat([torch.zeros(1, dtype=torch.int64),  # noqa: E731
                                     torch.cumsum(lens.long(), 0)]).to(torch.int32).to(DEV)
        leaves = [_pack(t, s).requires_grad_(True) for t, s in ((q, sq), (k, sk), (v, sk))]
        smp = None if sm is None else _pack(sm[..., None, None], sk)[:, 0, 0]
        o = ts.sigmoid_attention_varlen(*leaves, cu(sq), cu(sk), score_mod=smp, **kw)
        o.backward(_pack(do, sq))
        got = [o.detach()] + [t.grad for t in leaves]

    scale = np.float32(cfg["scale"] if cfg["scale"] is not None else 1.0 / math.sqrt(D))
    if cfg["bias"] is not None:
        bias = np.full(B, np.float32(cfg["bias"]), dtype=np.float64)
    elif api == "dense":
        bias = np.full(B, -math.log(Tk), dtype=np.float32).astype(np.float64)
    else:
        bias = (-torch.log(sk.float())).double().numpy()
    lens = {} if api == "dense" else dict(seq_lens_q=sq, seq_lens_k=sk)
    want_o, (dq, dk, dv) = oracle_fwd_bwd(
        _zero_past(q, sq), _zero_past(k, sk), _zero_past(v, sk), _zero_past(do, sq), scale=scale, bias=bias,
        score_mod=None if sm is None else _zero_past(sm, sk), causal=causal, **lens)
    want = [want_o, dq, dk, dv]
    if api == "varlen":
        sel = lambda a, s: np.concatenate([a[b, :int(s[b])] for b in range(B)], 0)  # noqa: E731
        want = [sel(w, s) for w, s in zip(want, (sq, sq, sk, sk))]
    for name, a, w in zip(("O", "dQ", "dK", "dV"), got, want):
        assert tuple(a.shape) == w.shape, name
        assert_close_to_oracle(a, w, dtype, name)
