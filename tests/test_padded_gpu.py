"""GPU parity tests for the padded path (sigmoid_attention_padded ->
myops::sigmoid_attn_padded_fwd/bwd -> libsigattn.so).  Mirrors the reference's
tests/test_sigmoid_padded.py."""

import ctypes
import math

import numpy as np
import pytest
import torch

import triton_sigmoid as ts
from triton_sigmoid import _capi
from conftest import get_tolerance
from helpers import (assert_close_to_oracle, assert_reference_criterion, criterion_errors,
                     oracle_fwd_bwd, randn, to_np)

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float16, torch.bfloat16, torch.float32]


def _case(B, Tq, Tk, H, D, dtype, seed, std=1.0, noise=True, lo=0.5):
    g = torch.Generator().manual_seed(seed)
    q = randn((B, Tq, H, D), dtype, DEV, g, std)
    k = randn((B, Tk, H, D), dtype, DEV, g, std)
    v = randn((B, Tk, H, D), dtype, DEV, g, std)
    do = randn((B, Tq, H, D), dtype, DEV, g, 1.0)
    sq = torch.randint(int(lo * Tq), Tq + 1, (B,), generator=g, dtype=torch.int32)
    sk = sq.clone() if Tq == Tk else torch.randint(int(lo * Tk), Tk + 1, (B,), generator=g, dtype=torch.int32)
    if noise:  # padding rows hold NaN: they must never be read
        for b in range(B):
            q[b, sq[b]:] = float("nan")
            do[b, sq[b]:] = float("nan")
            k[b, sk[b]:] = float("nan")
            v[b, sk[b]:] = float("nan")
    return q, k, v, do, sq.to(DEV), sk.to(DEV)


def _clean(t, lens):
    t = t.detach().clone()
    for b in range(t.shape[0]):
        t[b, int(lens[b]):] = 0
    return t


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("Tq,Tk", [(128, 128), (200, 77), (77, 300), (513, 513)])
@pytest.mark.parametrize("causal", [False, True])
def test_padded_matches_oracle(dtype, D, Tq, Tk, causal):
    B, H = 3, 2
    q, k, v, do, sq, sk = _case(B, Tq, Tk, H, D, dtype, seed=Tq + Tk + D)
    for t in (q, k, v):
        t.requires_grad_(True)
    o = ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk, seq_lens_q=sq, is_causal=causal)
    o.backward(do)
    bias = (-torch.log(sk.float())).double().cpu().numpy()
    qc, kc, vc, doc = _clean(q, sq), _clean(k, sk), _clean(v, sk), _clean(do, sq)
    want_o, (dq, dk, dv) = oracle_fwd_bwd(qc, kc, vc, doc, scale=np.float32(1 / math.sqrt(D)), bias=bias,
                                          seq_lens_q=sq, seq_lens_k=sk, causal=causal)
    assert_close_to_oracle(o, want_o, dtype, "O")
    assert_close_to_oracle(q.grad, dq, dtype, "dQ")
    assert_close_to_oracle(k.grad, dk, dtype, "dK")
    assert_close_to_oracle(v.grad, dv, dtype, "dV")
    # padded rows are exact zeros
    for b in range(B):
        assert torch.all(o[b, sq[b]:] == 0) and torch.all(q.grad[b, sq[b]:] == 0)
        assert torch.all(k.grad[b, sk[b]:] == 0) and torch.all(v.grad[b, sk[b]:] == 0)


def _padded_vs_oracle(q, k, v, do, sq, sk, causal, dtype):
    """Runs sigmoid_attention_padded forward + backward and checks O and the
    gradients against the oracle on the inputs with padding rows zeroed."""
    D = q.shape[-1]
    for t in (q, k, v):
        t.requires_grad_(True)
    o = ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk, seq_lens_q=sq, is_causal=causal)
    o.backward(do)
    Lq = sq if sq is not None else torch.full((q.shape[0],), q.shape[1], dtype=torch.int32)
    bias = (-torch.log(sk.float())).double().cpu().numpy()
    qc, kc, vc, doc = _clean(q, Lq), _clean(k, sk), _clean(v, sk), _clean(do, Lq)
    want_o, (dq, dk, dv) = oracle_fwd_bwd(qc, kc, vc, doc, scale=np.float32(1 / math.sqrt(D)), bias=bias,
                                          seq_lens_q=sq, seq_lens_k=sk, causal=causal)
    assert_close_to_oracle(o, want_o, dtype, "O")
    assert_close_to_oracle(q.grad, dq, dtype, "dQ")
    assert_close_to_oracle(k.grad, dk, dtype, "dK")
    assert_close_to_oracle(v.grad, dv, dtype, "dV")


@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_padded_extreme_length_variation(D, causal):
    """Key lengths from 16 to the full T in one batch, queries unpadded (the
    reference's tests/test_sigmoid_padded.py:752-773 checks NaN only)."""
    B, T, H = 4, 256, 3
    dtype = torch.float16
    q, k, v, do, _, _ = _case(B, T, T, H, D, dtype, seed=D + int(causal), noise=False)
    sk = torch.tensor([16, 64, 128, T], dtype=torch.int32, device=DEV)
    for b in range(B):  # padding keys hold NaN: they must never be read
        k[b, int(sk[b]):] = float("nan")
        v[b, int(sk[b]):] = float("nan")
    _padded_vs_oracle(q, k, v, do, None, sk, causal, dtype)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("Tq,Tk", [(32, 512), (512, 32), (1, 2048), (2048, 1)])
def test_cross_attention_extreme_length_ratio(D, Tq, Tk):
    """Very different query and key lengths, both padded (the reference's
    tests/test_sigmoid_padded.py:776-798 checks NaN only).  Tq = 1 against
    2048 keys takes the split-KV decode kernel."""
    B, H = 2, 2
    dtype = torch.bfloat16
    q, k, v, do, sq, sk = _case(B, Tq, Tk, H, D, dtype, seed=Tq + Tk + D)
    _padded_vs_oracle(q, k, v, do, sq, sk, False, dtype)


@pytest.mark.parametrize("causal", [False, True])
def test_padded_many_batches_odd_key_blocks(causal):
    """B > 64 takes the kernels' plain grid order, where the D = 128 dK/dV
    kernel runs key blocks j and nblk-1-j in one workgroup; T = 300 gives an
    odd number (3) of 128-key blocks, so one workgroup has a single block.
    Lengths include 0 and the full T."""
    B, T, H, D = 70, 300, 1, 128
    dtype = torch.bfloat16
    q, k, v, do, sq, sk = _case(B, T, T, H, D, dtype, seed=70 + int(causal), noise=False, lo=0.0)
    sq[0], sq[1] = 0, T
    sk.copy_(sq)
    for b in range(B):  # padding rows hold NaN: they must never be read
        for t in (q, k, v, do):
            t[b, int(sq[b]):] = float("nan")
    for t in (q, k, v):
        t.requires_grad_(True)
    o = ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk, seq_lens_q=sq, is_causal=causal)
    o.backward(do)
    bias = (-torch.log(sk.float())).double().cpu().numpy()
    qc, kc, vc, doc = _clean(q, sq), _clean(k, sk), _clean(v, sk), _clean(do, sq)
    want_o, (dq, dk, dv) = oracle_fwd_bwd(qc, kc, vc, doc, scale=np.float32(1 / math.sqrt(D)), bias=bias,
                                          seq_lens_q=sq, seq_lens_k=sk, causal=causal)
    assert_close_to_oracle(o, want_o, dtype, "O")
    assert_close_to_oracle(q.grad, dq, dtype, "dQ")
    assert_close_to_oracle(k.grad, dk, dtype, "dK")
    assert_close_to_oracle(v.grad, dv, dtype, "dV")
    for b in range(B):
        assert torch.all(k.grad[b, sk[b]:] == 0) and torch.all(v.grad[b, sk[b]:] == 0)


@pytest.mark.parametrize("D,B,H", [(64, 48, 2), (128, 64, 3)])
def test_causal_padded_dealing_rounds(D, B, H):
    """Causal ragged batches deal their items heaviest level first over the
    GPU's compute units, every odd round of workgroup ids placed at launch
    in reverse (WorkOrder::dealt; D = 64, where a CU holds two or three
    workgroups; the D = 128 kernels hold one and keep the plain order).
    These shapes give the kernels about 290-580 valid items: a full first
    round, a reversed odd round and partial last rounds, with padding items
    past them.  Every valid row is
    held to the reference's criterion (fp32 and mixed eager paths, as in
    test_padded_reference_criterion), and the packed layout, a different
    caller of the same work order, must match the padded one bit for bit."""
    T = 400
    dtype = torch.float16
    tol = get_tolerance(dtype)
    q, k, v, do, sq, sk = _case(B, T, T, H, D, dtype, seed=1000 + D, std=0.5, noise=False, lo=0.5)
    q_valid = torch.arange(T)[None, :] < sq.cpu()[:, None]
    fn = lambda a, b, c: ts.sigmoid_attention_padded(a, b, c, seq_lens_k=sk, seq_lens_q=sq, is_causal=True)
    errs = criterion_errors(q, k, v, do, fn, dict(seq_lens_k=sk, seq_lens_q=sq, causal=True),
                            q_valid=q_valid, k_valid=q_valid)
    assert_reference_criterion(errs, tol)

    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
    o = fn(*leaves)
    o.backward(do)
    lens = sq.cpu().tolist()
    rows = lambda t: torch.cat([t[b, :lens[b]] for b in range(B)])
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32, device=DEV)
    pk = [rows(t).detach().clone().requires_grad_(True) for t in (q, k, v)]
    op = ts.sigmoid_attention_varlen(*pk, cu, cu, max_seqlen_q=T, max_seqlen_k=T, is_causal=True)
    op.backward(rows(do))
    assert torch.equal(op, rows(o.detach()))
    for name, a, b_ in zip(("dQ", "dK", "dV"), pk, leaves):
        assert torch.equal(a.grad, rows(b_.grad)), name
    for b in range(B):  # padded key rows get exactly zero gradients
        assert torch.all(leaves[1].grad[b, lens[b]:] == 0) and torch.all(leaves[2].grad[b, lens[b]:] == 0)


# The reference's test_op grid (tests/test_sigmoid_padded.py:48-186): B, H in
# {(1, 2), (4, 8)}, (Tq, Tk) pairs, D in {64, 128}, causal (skipped for
# Tq > Tk, as there), fp16 / bf16 / fp32, seq_lens ~ U[0.8 T, T], N(0, 0.5²)
# inputs; errors on valid rows only.
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,H", [(1, 2), (4, 8)])
@pytest.mark.parametrize("Tq,Tk", [(128, 128), (256, 512), (512, 256), (1024, 1024), (4096, 4096)])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_padded_reference_criterion(dtype, B, H, Tq, Tk, D, causal):
    if causal and Tq > Tk:
        pytest.skip("causal needs Tq <= Tk (the reference skips it too)")
    tol = get_tolerance(dtype)
    q, k, v, do, sq, sk = _case(B, Tq, Tk, H, D, dtype, seed=Tq + 3 * Tk + D + B, std=0.5, noise=False, lo=0.8)
    q_valid = torch.arange(Tq)[None, :] < sq.cpu()[:, None]
    k_valid = torch.arange(Tk)[None, :] < sk.cpu()[:, None]
    errs = criterion_errors(
        q, k, v, do,
        lambda a, b, c: ts.sigmoid_attention_padded(a, b, c, seq_lens_k=sk, seq_lens_q=sq, is_causal=causal),
        dict(seq_lens_k=sk, seq_lens_q=sq, causal=causal), q_valid=q_valid, k_valid=k_valid)
    assert_reference_criterion(errs, tol)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("Tq,Tk", [(128, 128), (200, 77), (77, 300)])
@pytest.mark.parametrize("causal", [False, True])
def test_padded_score_mod_matches_oracle(dtype, D, Tq, Tk, causal):
    """score_mod [B, Tk] on the padded path, forward and backward against the
    float64 oracle at every head dim and dtype (the reference checks one fp16
    D = 64 case, tests/test_sigmoid_padded.py:387-477).  The score_mod entries
    of padding keys hold NaN: like the padding rows of Q/K/V they must never
    be read."""
    B, H = 3, 2
    q, k, v, do, sq, sk = _case(B, Tq, Tk, H, D, dtype, seed=7 * Tq + Tk + D + int(causal))
    g = torch.Generator().manual_seed(Tq + 5 * D)
    sm = (torch.randn((B, Tk), generator=g) * 2.0).to(dtype).to(DEV)
    sm_noisy = sm.clone()
    for b in range(B):
        sm_noisy[b, int(sk[b]):] = float("nan")
    for t in (q, k, v):
        t.requires_grad_(True)
    o = ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk, seq_lens_q=sq, is_causal=causal, score_mod=sm_noisy)
    o.backward(do)
    bias = (-torch.log(sk.float())).double().cpu().numpy()
    qc, kc, vc, doc = _clean(q, sq), _clean(k, sk), _clean(v, sk), _clean(do, sq)
    want_o, (dq, dk, dv) = oracle_fwd_bwd(qc, kc, vc, doc, scale=np.float32(1 / math.sqrt(D)), bias=bias,
                                          score_mod=_clean(sm, sk), seq_lens_q=sq, seq_lens_k=sk, causal=causal)
    assert_close_to_oracle(o, want_o, dtype, "O")
    assert_close_to_oracle(q.grad, dq, dtype, "dQ")
    assert_close_to_oracle(k.grad, dk, dtype, "dK")
    assert_close_to_oracle(v.grad, dv, dtype, "dV")
    for b in range(B):
        assert torch.all(o[b, sq[b]:] == 0) and torch.all(q.grad[b, sq[b]:] == 0)
        assert torch.all(k.grad[b, sk[b]:] == 0) and torch.all(v.grad[b, sk[b]:] == 0)


@pytest.mark.parametrize("dtype", DTYPES)
def test_padded_score_mod_reference_criterion(dtype):
    """The reference's test_score_mod_padded (tests/test_sigmoid_padded.py:387-477):
    B=2 L=128 H=4 D=64, N(0, 0.5²) inputs, score_mod ~ N(0, 1) in the input
    dtype, seq_lens_k = [100, 110] and no seq_lens_q; errors against the fp32
    eager path within 2x (forward) / 3x (backward) the mixed-precision eager
    path's plus the tolerance, the gradients of padding keys excluded.  Its
    absolute bounds (O, dQ and dK below the tolerance, dV below twice it) are
    checked in fp16, the dtype the reference runs this test in: one bf16
    rounding step of the dV entries in [2, 4) this case produces is 2^-6,
    above twice the bf16 tolerance, for any kernel that stores bf16."""
    B, L, H, D = 2, 128, 4, 64
    tol = get_tolerance(dtype)
    g = torch.Generator().manual_seed(387)
    q, k, v = (randn((B, L, H, D), dtype, DEV, g, 0.5) for _ in range(3))
    do = randn((B, L, H, D), dtype, DEV, g)
    sm = randn((B, L), dtype, DEV, g)
    sk = torch.tensor([100, 110], dtype=torch.int32, device=DEV)
    k_valid = torch.arange(L)[None, :] < sk.cpu()[:, None]
    errs = criterion_errors(
        q, k, v, do,
        lambda a, b, c: ts.sigmoid_attention_padded(a, b, c, seq_lens_k=sk, score_mod=sm),
        dict(seq_lens_k=sk, score_mod=sm), k_valid=k_valid)
    for name, (e, em) in errs.items():
        assert e <= (2.0 if name == "O" else 3.0) * em + tol, (name, e, em, tol)
        if dtype == torch.float16:
            assert e < (2.0 * tol if name == "dV" else tol), (name, e, tol)
    out_none = ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk, score_mod=None)
    assert out_none.shape == (B, L, H, D)


def test_padding_noise_invariance():
    B, T, H, D = 2, 300, 2, 64
    q, k, v, do, sq, sk = _case(B, T, T, H, D, torch.bfloat16, seed=3, noise=False)
    a = ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk, seq_lens_q=sq, is_causal=True)
    q2, k2, v2 = q.clone(), k.clone(), v.clone()
    for b in range(B):
        q2[b, sq[b]:] = 1e4
        k2[b, sk[b]:] = float("inf")
        v2[b, sk[b]:] = float("nan")
    b_ = ts.sigmoid_attention_padded(q2, k2, v2, seq_lens_k=sk, seq_lens_q=sq, is_causal=True)
    assert torch.equal(a, b_)


def test_full_lengths_match_dense():
    B, T, H, D = 2, 384, 4, 128
    g = torch.Generator().manual_seed(1)
    q, k, v = (randn((B, T, H, D), torch.bfloat16, DEV, g) for _ in range(3))
    for causal in (False, True):
        # Same explicit bias: the same kernel runs, so results are bitwise equal.
        a = ts.sigmoid_attention(q, k, v, is_causal=causal, sigmoid_bias=-4.5)
        b = ts.sigmoid_attention_padded(q, k, v, is_causal=causal, sigmoid_bias=-4.5)
        assert torch.equal(a, b)
        # Default biases: -log(T) in fp64 (dense) vs -log(seq_lens) in fp32
        # (padded) may differ by one fp32 ulp (tests/test_sigmoid_padded.py:723-749
        # compares these within 2*tol).
        a = ts.sigmoid_attention(q, k, v, is_causal=causal)
        b = ts.sigmoid_attention_padded(q, k, v, is_causal=causal)
        torch.testing.assert_close(a, b, atol=2 * 7e-3, rtol=0)


def test_zero_and_out_of_range_seq_lens():
    B, T, H, D = 3, 128, 2, 64
    q, k, v, do, _, _ = _case(B, T, T, H, D, torch.float16, seed=4, noise=False)
    sq = torch.tensor([0, -5, 500], dtype=torch.int32, device=DEV)
    sk = torch.tensor([64, 0, 1000], dtype=torch.int64, device=DEV)
    for t in (q, k, v):
        t.requires_grad_(True)
    o = ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk, seq_lens_q=sq, sigmoid_bias=-1.0)
    o.backward(do)
    assert torch.isfinite(o).all() and torch.isfinite(q.grad).all()
    assert torch.all(o[0] == 0) and torch.all(o[1] == 0)
    full = ts.sigmoid_attention_padded(q[2:], k[2:], v[2:], sigmoid_bias=-1.0)
    assert torch.equal(o[2:], full)


def test_cross_attention_short_queries():
    B, Tq, Tk, H, D = 2, 32, 512, 2, 64
    q, k, v, do, sq, sk = _case(B, Tq, Tk, H, D, torch.float16, seed=5, noise=False)
    o = ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk, seq_lens_q=sq)
    want, _ = oracle_fwd_bwd(q, k, v, do, scale=np.float32(1 / 8), bias=(-torch.log(sk.float())).double().cpu().numpy(),
                             seq_lens_q=sq, seq_lens_k=sk, with_bwd=False)
    assert_close_to_oracle(o, want, torch.float16, "O")


def test_padded_forward_deterministic():
    q, k, v, do, sq, sk = _case(2, 700, 700, 4, 128, torch.bfloat16, seed=6, noise=False)
    a = ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk, seq_lens_q=sq, is_causal=True)
    b = ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk, seq_lens_q=sq, is_causal=True)
    assert torch.equal(a, b)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_head_major_layout_equals_contiguous(D, causal):
    """Tensors whose rows do not hold every head back to back (a head-major
    [B, H, T, D] buffer viewed as [B, T, H, D]) go through the C ABI with
    their own strides: padding row blocks then take the per-head zero-row
    path instead of the contiguous span.  Every output and gradient equals
    the contiguous layout's (public API) bit for bit, padding rows zero."""
    import ctypes

    from triton_sigmoid import _capi

    B, T, H, dtype = 3, 520, 2, torch.bfloat16
    q, k, v, do, sq, sk = _case(B, T, T, H, D, dtype, seed=60 + D, noise=False)
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
    o = ts.sigmoid_attention_padded(*leaves, seq_lens_k=sk, seq_lens_q=sq, is_causal=causal)
    o.backward(do)
    want = [o.detach()] + [t.grad for t in leaves]

    def head_major(t):  # same values, strides (H*T*D, D, T*D, 1)
        return t.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)

    hq, hk, hv, hdo = (head_major(t) for t in (q, k, v, do))
    assert hq.stride(1) == D and hq.stride(2) == T * D
    outs = [head_major(torch.full_like(t, float("nan"))) for t in (q, q, k, k)]  # O, dQ, dK, dV
    bias = -torch.log(sk.float())
    scale = torch.full((), 1 / math.sqrt(D), dtype=torch.float32, device=DEV)
    lib = _capi.load_library()
    pr = _capi._problem(hq, hk, hv, bias, None, scale, sq, sk, causal)
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.sigattn_fwd_ws(ctypes.byref(pr), outs[0].data_ptr(), None, 0, stream) == 0
    # The public API's backward policy (two-pass, range split or recompute
    # kernels), so both layouts run the same kernels.
    _capi._launch_bwd(lib, pr, hdo, outs[1], outs[2], outs[3])
    torch.cuda.synchronize()
    for name, got, ref, lens in zip(("O", "dQ", "dK", "dV"), outs, want, (sq, sq, sk, sk)):
        assert torch.equal(got, ref), f"{name} differs from the contiguous layout"
        for b in range(B):
            assert torch.all(got[b, int(lens[b]):] == 0), f"{name}: padding rows of batch {b} not zero"


@pytest.mark.parametrize("layout", ["padded", "packed"])
def test_concurrent_backward_equals_the_two_kernels(layout):
    """A ragged non-causal D = 64 problem of 2048 query blocks (eight per CU of
    the MI355X) runs its recompute backward's dQ and dK/dV kernels on two
    streams; its dQ, dK and dV equal those of the two kernels run alone, one
    after the other on one stream (sigattn_bwd_dq, sigattn_bwd_dkdv), bit for
    bit, with the padding rows zero."""
    B, T, H, D, dtype = 2, 4096, 32, 64, torch.float16
    q, k, v, do, sq, sk = _case(B, T, T, H, D, dtype, seed=91, noise=False)
    sq = sk = torch.tensor([4096, 2731], dtype=torch.int32)
    lib = _capi.load_library()
    bias = -torch.log(sk.float()).to(DEV)
    scale = torch.full((), 1 / math.sqrt(D), dtype=torch.float32, device=DEV)
    if layout == "packed":
        lens = sq.tolist()
        q, k, v, do = (torch.cat([t[b, :n] for b, n in enumerate(lens)], 0).contiguous() for t in (q, k, v, do))
        cu = torch.tensor([0, lens[0], lens[0] + lens[1]], dtype=torch.int32, device=DEV)
        pr = _capi._problem(q, k, v, bias, None, scale, None, None, False, packed=(cu, cu, T, T))
    else:
        pr = _capi._problem(q, k, v, bias, None, scale, sq.to(DEV), sk.to(DEV), False)
    stream = torch.cuda.current_stream().cuda_stream
    one = [torch.full_like(t, float("nan")) for t in (q, k, v)]
    two = [torch.full_like(t, float("nan")) for t in (q, k, v)]
    assert lib.sigattn_bwd(ctypes.byref(pr), do.data_ptr(), *(t.data_ptr() for t in one), stream) == 0
    assert lib.sigattn_bwd_dq(ctypes.byref(pr), do.data_ptr(), two[0].data_ptr(), stream) == 0
    assert lib.sigattn_bwd_dkdv(ctypes.byref(pr), do.data_ptr(), two[1].data_ptr(), two[2].data_ptr(), stream) == 0
    torch.cuda.synchronize()
    for name, a, b in zip(("dQ", "dK", "dV"), one, two):
        assert torch.isfinite(a).all(), name
        assert torch.equal(a, b), name
    if layout == "padded":
        for t in one:
            assert torch.all(t[1, 2731:] == 0)
