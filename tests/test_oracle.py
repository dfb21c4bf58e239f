"""Pins the CPU oracle (oracle/sigmoid_oracle.py, oracle/eager.py) without a GPU.

Each check is chosen so that a plausible mistake in the oracle fails it:
  * closed forms catch a wrong bias sign, scale placement or causal row count;
  * pure-Python loops catch transposed operands / wrong einsum indices;
  * finite differences and float64 autograd catch a wrong backward formula;
  * invariants catch mask leaks (causality, padding noise, split-KV);
  * torch's own bf16/fp16 casts pin the rounding emulation.
"""

import math

import numpy as np
import pytest
import torch

from oracle import sigmoid_oracle as so
from oracle.eager import fwd_bwd_fp32, sigmoid_attention_eager


def _rand(rng, *shape):
    return rng.standard_normal(shape)


def _sig(x):
    return 1.0 / (1.0 + math.exp(-x))


# ---------------------------------------------------------------- rounding --

@pytest.mark.parametrize("dtype,tdtype", [("bf16", torch.bfloat16), ("f16", torch.float16)])
def test_round_to_matches_torch_casts(dtype, tdtype):
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(4000) * 10.0 ** rng.integers(-6, 4, 4000),
                        [0.0, -0.0, 1.0, 0.5, 1 / 3, 65504.0, 1e-8]])
    want = torch.tensor(x, dtype=torch.float32).to(tdtype).double().numpy()
    got = so.round_to(x, dtype)
    np.testing.assert_array_equal(got, want)


# ------------------------------------------------------------ closed forms --

@pytest.mark.parametrize("causal", [False, True])
def test_zero_qk_gives_bias_weighted_value_sums(causal):
    # q = k = 0 -> S = bias, so O[i] = sigmoid(bias) * sum of visible v rows.
    rng = np.random.default_rng(1)
    B, T, H, D = 2, 9, 2, 4
    q = np.zeros((B, T, H, D))
    v = _rand(rng, B, T, H, D)
    bias = np.array([-math.log(T), 0.7])
    o = so.forward(q, q, v, scale=0.3, bias=bias, causal=causal)
    for b in range(B):
        for i in range(T):
            n = i + 1 if causal else T
            want = _sig(bias[b]) * v[b, :n].sum(axis=0)
            np.testing.assert_allclose(o[b, i], want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_all_ones_gives_visible_count_times_sigmoid(causal):
    # q = k = v = 1 -> S = D*scale + bias for every pair, O = n_visible * sigmoid(S).
    B, T, H, D = 1, 7, 1, 5
    ones = np.ones((B, T, H, D))
    scale, bias = 0.25, -math.log(T)
    o = so.forward(ones, ones, ones, scale=scale, bias=np.array([bias]), causal=causal)
    p = _sig(D * scale + bias)
    for i in range(T):
        n = i + 1 if causal else T
        np.testing.assert_allclose(o[0, i, 0], np.full(D, n * p), rtol=1e-12)


def test_padded_all_ones_counts_valid_keys_only():
    B, Tq, Tk, H, D = 2, 6, 8, 1, 3
    q = np.ones((B, Tq, H, D))
    k = np.ones((B, Tk, H, D))
    sq, sk = np.array([4, 6]), np.array([5, 2])
    bias = so.default_bias(B, Tk, sk)
    o = so.forward(q, k, k, scale=1.0, bias=bias, seq_lens_q=sq, seq_lens_k=sk)
    for b in range(B):
        for i in range(Tq):
            want = 0.0 if i >= sq[b] else sk[b] * _sig(D + bias[b])
            np.testing.assert_allclose(o[b, i, 0], np.full(D, want), rtol=1e-12)


def test_single_token_backward_closed_form():
    rng = np.random.default_rng(2)
    D = 3
    q, k, v, do = (_rand(rng, 1, 1, 1, D) for _ in range(4))
    scale, bias = 0.8, -0.3
    dq, dk, dv = so.backward(q, k, v, do, scale=scale, bias=np.array([bias]))
    s = scale * float(q.ravel() @ k.ravel()) + bias
    p = _sig(s)
    g = p * (1 - p) * float(do.ravel() @ v.ravel())
    np.testing.assert_allclose(dv.ravel(), p * do.ravel(), rtol=1e-12)
    np.testing.assert_allclose(dq.ravel(), g * scale * k.ravel(), rtol=1e-12)
    np.testing.assert_allclose(dk.ravel(), g * scale * q.ravel(), rtol=1e-12)


def test_default_bias_matches_reference_api():
    np.testing.assert_allclose(so.default_bias(3, 100), np.full(3, -math.log(100)))
    np.testing.assert_allclose(so.default_bias(2, 9, np.array([4, 9])), -np.log([4.0, 9.0]))


# ------------------------------------------------------------- brute force --

def _forward_loops(q, k, v, scale, bias, sm, sq, sk, causal, io):
    B, Tq, H, D = q.shape
    Tk = k.shape[1]
    o = np.zeros((B, Tq, H, D))
    for b in range(B):
        Lq = min(max(int(sq[b]), 0), Tq) if sq is not None else Tq
        Lk = min(max(int(sk[b]), 0), Tk) if sk is not None else Tk
        for h in range(H):
            for i in range(Lq):
                for j in range(Lk):
                    if causal and j > i:
                        continue
                    s = sum(q[b, i, h, d] * k[b, j, h, d] for d in range(D)) * scale + bias[b]
                    if sm is not None:
                        s += sm[b, j]
                    p = float(so.round_to(np.array([_sig(s)]), io)[0])
                    for d in range(D):
                        o[b, i, h, d] += p * v[b, j, h, d]
    return o


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("padded", [False, True])
@pytest.mark.parametrize("io", [None, "bf16"])
def test_forward_matches_loops(causal, padded, io):
    rng = np.random.default_rng(3)
    B, Tq, Tk, H, D = 2, 5, 7 if padded else 5, 2, 3
    q, k, v = _rand(rng, B, Tq, H, D), _rand(rng, B, Tk, H, D), _rand(rng, B, Tk, H, D)
    sm = _rand(rng, B, Tk)
    sq = np.array([3, 5]) if padded else None
    sk = np.array([7, 4]) if padded else None
    bias = np.array([-0.5, 0.25])
    want = _forward_loops(q, k, v, 0.6, bias, sm, sq, sk, causal, io)
    got = so.forward(q, k, v, scale=0.6, bias=bias, score_mod=sm, seq_lens_q=sq, seq_lens_k=sk,
                     causal=causal, io_dtype=io)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------ backward pins --

@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("padded", [False, True])
def test_backward_matches_finite_differences(causal, padded):
    rng = np.random.default_rng(4)
    B, Tq, Tk, H, D = 2, 4, 5 if padded else 4, 1, 3
    q, k, v = _rand(rng, B, Tq, H, D), _rand(rng, B, Tk, H, D), _rand(rng, B, Tk, H, D)
    do = _rand(rng, B, Tq, H, D)
    sm = _rand(rng, B, Tk)
    kw = dict(scale=0.7, bias=np.array([0.1, -0.4]), score_mod=sm, causal=causal,
              seq_lens_q=np.array([3, 4]) if padded else None,
              seq_lens_k=np.array([5, 2]) if padded else None)
    dq, dk, dv = so.backward(q, k, v, do, **kw)

    def loss(qq, kk, vv):
        return float((so.forward(qq, kk, vv, **kw) * do).sum())

    eps = 1e-6
    for name, x, g in (("q", q, dq), ("k", k, dk), ("v", v, dv)):
        num = np.zeros_like(x)
        it = np.nditer(x, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            args_p = {"q": (xp, k, v), "k": (q, xp, v), "v": (q, k, xp)}[name]
            args_m = {"q": (xm, k, v), "k": (q, xm, v), "v": (q, k, xm)}[name]
            num[idx] = (loss(*args_p) - loss(*args_m)) / (2 * eps)
        np.testing.assert_allclose(g, num, rtol=1e-6, atol=1e-8, err_msg=name)


@pytest.mark.parametrize("causal", [False, True])
def test_backward_matches_float64_autograd(causal):
    rng = np.random.default_rng(5)
    B, T, H, D = 2, 6, 2, 4
    arrs = [_rand(rng, B, T, H, D) for _ in range(4)]
    sm = _rand(rng, B, T)
    q, k, v, do = (torch.tensor(a, requires_grad=i < 3) for i, a in enumerate(arrs))
    o = sigmoid_attention_eager(q, k, v, scale=0.4, sigmoid_bias=-0.2, upcast=False,
                                causal=causal, score_mod=torch.tensor(sm))
    o.backward(do)
    kw = dict(scale=0.4, bias=np.full(B, -0.2), score_mod=sm, causal=causal)
    np.testing.assert_allclose(so.forward(*arrs[:3], **kw), o.detach().numpy(), rtol=1e-12, atol=1e-13)
    dq, dk, dv = so.backward(*arrs, **kw)
    np.testing.assert_allclose(dq, q.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dk, k.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dv, v.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_eager_padded_matches_oracle():
    rng = np.random.default_rng(6)
    B, Tq, Tk, H, D = 2, 5, 6, 2, 4
    q, k, v = _rand(rng, B, Tq, H, D), _rand(rng, B, Tk, H, D), _rand(rng, B, Tk, H, D)
    sq, sk = np.array([5, 2]), np.array([3, 6])
    o = sigmoid_attention_eager(torch.tensor(q), torch.tensor(k), torch.tensor(v),
                                seq_lens_k=torch.tensor(sk), seq_lens_q=torch.tensor(sq),
                                scale=0.5, upcast=False, causal=True)
    # The eager reference keeps its epsilon and computes the bias in fp32.
    bias = (-torch.log(torch.tensor(sk).float() + 1e-6)).double().numpy()
    want = so.forward(q, k, v, scale=0.5, bias=bias, seq_lens_q=sq, seq_lens_k=sk, causal=True)
    np.testing.assert_allclose(o.numpy(), want, rtol=1e-12, atol=1e-13)


# ---------------------------------------------------------------- invariants --

def test_causality_future_keys_do_not_change_past():
    rng = np.random.default_rng(7)
    B, T, H, D = 1, 10, 2, 4
    q, k, v = (_rand(rng, B, T, H, D) for _ in range(3))
    kw = dict(scale=0.5, bias=np.array([-1.0]), causal=True)
    o1 = so.forward(q, k, v, **kw)
    k2, v2 = k.copy(), v.copy()
    k2[:, 6:] = _rand(rng, B, 4, H, D)
    v2[:, 6:] = _rand(rng, B, 4, H, D)
    o2 = so.forward(q, k2, v2, **kw)
    np.testing.assert_array_equal(o1[:, :6], o2[:, :6])
    assert not np.allclose(o1[:, 6:], o2[:, 6:])


def test_padding_noise_does_not_leak():
    rng = np.random.default_rng(8)
    B, T, H, D = 2, 8, 1, 3
    q, k, v, do = (_rand(rng, B, T, H, D) for _ in range(4))
    sq, sk = np.array([5, 8]), np.array([6, 3])
    kw = dict(scale=0.5, bias=so.default_bias(B, T, sk), seq_lens_q=sq, seq_lens_k=sk, causal=False)
    base = so.forward(q, k, v, **kw), *so.backward(q, k, v, do, **kw)
    q2, k2, v2, do2 = q.copy(), k.copy(), v.copy(), do.copy()
    for b in range(B):
        q2[b, sq[b]:] = 1e3
        do2[b, sq[b]:] = -1e3
        k2[b, sk[b]:] = 1e3
        v2[b, sk[b]:] = -1e3
    noisy = so.forward(q2, k2, v2, **kw), *so.backward(q2, k2, v2, do2, **kw)
    for a, b_ in zip(base, noisy):
        np.testing.assert_allclose(a, b_, rtol=1e-12, atol=1e-12)
    for b in range(B):
        assert np.all(base[0][b, sq[b]:] == 0) and np.all(base[1][b, sq[b]:] == 0)
        assert np.all(base[2][b, sk[b]:] == 0) and np.all(base[3][b, sk[b]:] == 0)


def test_linearity_in_v_and_split_kv_additivity():
    rng = np.random.default_rng(9)
    B, T, H, D = 1, 8, 2, 4
    q, k, v, v2 = (_rand(rng, B, T, H, D) for _ in range(4))
    kw = dict(scale=0.5, bias=np.array([-0.7]))
    np.testing.assert_allclose(so.forward(q, k, 2 * v + v2, **kw),
                               2 * so.forward(q, k, v, **kw) + so.forward(q, k, v2, **kw), atol=1e-12)
    # No row normalisation: attention over [K1; K2] is the sum of the two halves.
    o = so.forward(q, k, v, **kw)
    o1 = so.forward(q, k[:, :3], v[:, :3], **kw)
    o2 = so.forward(q, k[:, 3:], v[:, 3:], **kw)
    np.testing.assert_allclose(o, o1 + o2, atol=1e-12)


def test_constant_score_mod_equals_bias_shift():
    rng = np.random.default_rng(10)
    B, T, H, D = 2, 6, 1, 4
    q, k, v = (_rand(rng, B, T, H, D) for _ in range(3))
    bias = np.array([0.2, -0.9])
    a = so.forward(q, k, v, scale=0.5, bias=bias, score_mod=np.full((B, T), 1.5))
    b = so.forward(q, k, v, scale=0.5, bias=bias + 1.5)
    np.testing.assert_allclose(a, b, atol=1e-12)
    z = so.forward(q, k, v, scale=0.5, bias=bias, score_mod=np.zeros((B, T)))
    np.testing.assert_array_equal(z, so.forward(q, k, v, scale=0.5, bias=bias))


def test_negative_and_oversized_seq_lens_are_clamped():
    rng = np.random.default_rng(11)
    B, T, H, D = 2, 5, 1, 2
    q, k, v = (_rand(rng, B, T, H, D) for _ in range(3))
    o = so.forward(q, k, v, scale=1.0, bias=np.zeros(B), seq_lens_q=np.array([-3, 99]),
                   seq_lens_k=np.array([99, -1]))
    assert np.all(o[0] == 0)           # no valid queries
    assert np.all(o[1] == 0)           # no valid keys
    assert np.all(np.isfinite(o))


# ------------------------------------------- fp32 eager checker (upcast) --
# oracle/eager.py's upcast=True branch and fwd_bwd_fp32 decide the full-size
# GPU tests (BASELINE configs c2-c5 within 2e-2) and the "ref" side of every
# reference-criterion test, so they are pinned here against the float64
# oracle, which the closed forms, loops, finite differences and autograd
# above pin in turn.  A dropped bias, a scale on the wrong operand, a
# triu offset off by one or a key mask applied before the sigmoid each move
# the fp32 result by far more than fp32 rounding.

def _fp32_case(rng, B, Tq, Tk, H, D):
    return [torch.tensor(_rand(rng, B, t, H, D), dtype=torch.float32) for t in (Tq, Tk, Tk, Tq)]


def _fp32_bound(want, n_terms):
    # fp32 accumulation of n_terms products: relative error well under
    # n_terms * 2^-24 of the largest magnitude.
    return 8.0 * n_terms * 2.0 ** -24 * float(np.abs(want).max()) + 1e-7


@pytest.mark.parametrize("case", ["dense", "causal", "padded_cross", "padded_causal", "score_mod", "explicit_bias"])
def test_eager_fp32_matches_oracle(case):
    rng = np.random.default_rng(40 + len(case))
    B, H, D = 2, 3, 16
    Tq, Tk = (9, 13) if case == "padded_cross" else (11, 11)
    q, k, v, do = _fp32_case(rng, B, Tq, Tk, H, D)
    kw = dict(causal=case in ("causal", "padded_causal", "score_mod"))
    sq = sk = sm = None
    if case.startswith("padded"):
        sq = torch.tensor([Tq - 3, Tq], dtype=torch.int32)
        sk = torch.tensor([Tk, Tk - 5], dtype=torch.int32)
        kw.update(seq_lens_q=sq, seq_lens_k=sk)
    if case == "score_mod":
        sm = torch.tensor(_rand(rng, B, Tk), dtype=torch.float32)
        kw["score_mod"] = sm
    scale = 0.37 if case == "explicit_bias" else None
    if case == "explicit_bias":
        kw.update(scale=scale, sigmoid_bias=-1.25)
    # The bias the eager path uses: explicit, else -log(len + 1e-6) in fp32
    # (padded) or in float64 (dense), as sigmoid_reference.py:73-80 does.
    if case == "explicit_bias":
        bias = np.full(B, -1.25)
    elif sk is not None:
        bias = (-torch.log(sk.float() + 1e-6)).double().numpy()
    else:
        bias = np.full(B, -math.log(Tk + 1e-6))
    okw = dict(scale=np.float32(scale if scale is not None else 1.0 / math.sqrt(D)), bias=bias,
               score_mod=None if sm is None else sm.double().numpy(),
               seq_lens_q=None if sq is None else sq.numpy(), seq_lens_k=None if sk is None else sk.numpy(),
               causal=kw["causal"])
    qn, kn, vn, dn = (t.double().numpy() for t in (q, k, v, do))
    want_o = so.forward(qn, kn, vn, **okw)
    want_g = so.backward(qn, kn, vn, dn, **okw)

    o = sigmoid_attention_eager(q, k, v, upcast=True, **kw)
    assert o.dtype == torch.float32
    np.testing.assert_allclose(o.double().numpy(), want_o, rtol=0, atol=_fp32_bound(want_o, D + Tk))
    o2, dq, dk, dv = fwd_bwd_fp32(q, k, v, do, **kw)
    np.testing.assert_array_equal(o2.numpy(), o.numpy())
    for name, got, want in zip(("dQ", "dK", "dV"), (dq, dk, dv), want_g):
        np.testing.assert_allclose(got.double().numpy(), want, rtol=0,
                                   atol=_fp32_bound(want, D + Tq + Tk), err_msg=name)


@pytest.mark.parametrize("causal", [False, True])
def test_eager_fp32_at_c1_matches_oracle(causal):
    """BASELINE.json configs[0] (CPU plumbing): fp32 B=2 L=256 H=4 D=64,
    q/k/v/dO ~ N(0,1) from a seed, scale 1/sqrt(D), default bias, fwd+bwd."""
    B, L, H, D = 2, 256, 4, 64
    g = torch.Generator().manual_seed(0)
    q, k, v, do = (torch.randn((B, L, H, D), generator=g) for _ in range(4))
    o, dq, dk, dv = fwd_bwd_fp32(q, k, v, do, causal=causal)
    okw = dict(scale=np.float32(1.0 / math.sqrt(D)), bias=np.full(B, -math.log(L + 1e-6)), causal=causal)
    qn, kn, vn, dn = (t.double().numpy() for t in (q, k, v, do))
    want_o = so.forward(qn, kn, vn, **okw)
    want_g = so.backward(qn, kn, vn, dn, **okw)
    for name, got, want in zip(("O", "dQ", "dK", "dV"), (o, dq, dk, dv), (want_o, *want_g)):
        err = float(np.abs(got.double().numpy() - want).max())
        # fp32 sums of a few hundred terms: ~1e-6 of the largest magnitude.
        assert err <= 4e-6 * float(np.abs(want).max()) + 1e-6, (name, err)


# -------------------------- mixed-precision eager path, written out (GPU use) --

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.float64])
@pytest.mark.parametrize("case", ["dense", "causal", "padded", "score_mod", "padded_causal_sm"])
def test_mixed_fwd_bwd_matches_autograd(dtype, case):
    """oracle/eager.py's mixed_fwd_bwd (contiguous matmuls, backward by hand)
    against autograd through sigmoid_attention_eager(upcast=False,
    reorder_ops=True), the reference's mixed-precision path: same values up
    to the summation order of the products (bit for bit on this CPU)."""
    from oracle.eager import mixed_fwd_bwd
    g = torch.Generator().manual_seed(hash(case) % 1000)
    B, Lq, H, D = 2, 40, 3, 32
    Lk = 56 if case == "padded" else 40
    q, k, v = ((torch.randn(B, t, H, D, generator=g) * 0.5).to(dtype) for t in (Lq, Lk, Lk))
    do = torch.randn(B, Lq, H, D, generator=g).to(dtype)
    kw = dict(causal=case in ("causal", "padded_causal_sm"))
    if case.startswith("padded"):
        kw.update(seq_lens_q=torch.tensor([Lq - 5, Lq], dtype=torch.int32),
                  seq_lens_k=torch.tensor([Lk, Lk - 9], dtype=torch.int32))
    if case in ("score_mod", "padded_causal_sm"):
        kw["score_mod"] = torch.randn(B, Lk, generator=g).to(dtype)
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
    o = sigmoid_attention_eager(*leaves, upcast=False, reorder_ops=True, **kw)
    o.backward(do)
    want = [o.detach()] + [t.grad for t in leaves]
    got = mixed_fwd_bwd(q, k, v, do, **kw)
    ulp = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2.0 ** -24,
           torch.float64: 2.0 ** -53}[dtype]
    for name, a, b in zip(("O", "dQ", "dK", "dV"), got, want):
        assert a.dtype == b.dtype and a.shape == b.shape, name
        err = (a.double() - b.double()).abs().max().item()
        assert err <= ulp * b.double().abs().max().item(), (name, err)
    if dtype == torch.float64:
        # In float64 the path is exact math: the float64 oracle, with the
        # eager bias -log(L + 1e-6) (padded: computed in fp32, as there).
        sq, sk = kw.get("seq_lens_q"), kw.get("seq_lens_k")
        bias = ((-torch.log(sk.float() + 1e-6)).double().numpy() if sk is not None
                else np.full(B, -math.log(Lk + 1e-6)))
        okw = dict(scale=1.0 / math.sqrt(D), bias=bias, causal=kw["causal"],
                   score_mod=None if "score_mod" not in kw else kw["score_mod"].numpy(),
                   seq_lens_q=None if sq is None else sq.numpy(), seq_lens_k=None if sk is None else sk.numpy())
        arrs = [t.numpy() for t in (q, k, v, do)]
        for name, a, b in zip(("O", "dQ", "dK", "dV"), got,
                              (so.forward(*arrs[:3], **okw), *so.backward(*arrs, **okw))):
            np.testing.assert_allclose(a.numpy(), b, rtol=1e-12, atol=1e-13, err_msg=name)
