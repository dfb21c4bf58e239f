"""GPU parity tests for the packed variable-length path (sigmoid_attention_varlen
-> myops::sigmoid_attn_varlen_fwd/bwd -> libsigattn.so with cu_seqlens set).

The packed layout has no counterpart in the reference's operator API; its
semantics are the padded operator's (sigmoid_triton_padded.py:853-1010) on the
same sequences.  The kernels start their tiles at each sequence's first row in
both layouts, so every valid output row must be bitwise equal to the padded
path's, and the padded path is itself held to the float64 oracle."""

import ctypes
import math

import numpy as np
import pytest
import torch

import triton_sigmoid as ts
from helpers import assert_close_to_oracle, oracle_fwd_bwd, randn
from triton_sigmoid import _capi

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lengths(B, T, lo, g):
    return torch.randint(int(lo * T), T + 1, (B,), generator=g, dtype=torch.int32)


def _pack(x, lens):
    """[B, T, H, D] -> [sum(lens), H, D] (valid rows only)."""
    return torch.cat([x[b, :int(lens[b])] for b in range(x.shape[0])], 0)


def _cu(lens):
    return torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(lens.long(), 0)]).to(torch.int32)


def _case(B, Tq, Tk, H, D, dtype, seed, lo=0.3, same=True):
    g = torch.Generator().manual_seed(seed)
    q = randn((B, Tq, H, D), dtype, DEV, g)
    k = randn((B, Tk, H, D), dtype, DEV, g)
    v = randn((B, Tk, H, D), dtype, DEV, g)
    do = randn((B, Tq, H, D), dtype, DEV, g)
    sq = _lengths(B, Tq, lo, g)
    sk = sq.clone() if (same and Tq == Tk) else _lengths(B, Tk, lo, g)
    return q, k, v, do, sq, sk


def _run_padded(q, k, v, do, sq, sk, causal, score_mod=None):
    q, k, v = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk.to(DEV), seq_lens_q=sq.to(DEV), is_causal=causal,
                                    score_mod=score_mod)
    o.backward(do)
    return o.detach(), q.grad, k.grad, v.grad


def _run_varlen(q, k, v, do, sq, sk, causal, score_mod=None, max_given=True):
    qp, kp, vp = (_pack(t, s).requires_grad_(True) for t, s in ((q, sq), (k, sk), (v, sk)))
    dop = _pack(do, sq)
    smp = None if score_mod is None else _pack(score_mod[..., None, None], sk)[:, 0, 0]
    kw = dict(max_seqlen_q=int(sq.max()), max_seqlen_k=int(sk.max())) if max_given else {}
    o = ts.sigmoid_attention_varlen(qp, kp, vp, _cu(sq).to(DEV), _cu(sk).to(DEV), is_causal=causal,
                                    score_mod=smp, **kw)
    o.backward(dop)
    return o.detach(), qp.grad, kp.grad, vp.grad


def _assert_equal_packed(padded, packed, sq, sk, what):
    for name, P, V, lens in zip(("O", "dQ", "dK", "dV"), padded, packed, (sq, sq, sk, sk)):
        want = _pack(P, lens)
        assert V.shape == want.shape, (what, name)
        assert torch.equal(V, want), f"{what} {name}: max diff {(V.float() - want.float()).abs().max().item()}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("Tq,Tk", [(128, 128), (513, 513), (200, 77), (77, 300)])
@pytest.mark.parametrize("causal", [False, True])
def test_varlen_equals_padded_bitwise(dtype, D, Tq, Tk, causal):
    B, H = 3, 2
    q, k, v, do, sq, sk = _case(B, Tq, Tk, H, D, dtype, seed=Tq * 7 + Tk + D)
    _assert_equal_packed(_run_padded(q, k, v, do, sq, sk, causal),
                         _run_varlen(q, k, v, do, sq, sk, causal), sq, sk, f"{dtype} D={D}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
def test_varlen_matches_oracle(dtype, causal):
    B, T, H, D = 4, 300, 2, 64
    q, k, v, do, sq, sk = _case(B, T, T, H, D, dtype, seed=11)
    o, dq, dk, dv = _run_varlen(q, k, v, do, sq, sk, causal, max_given=False)
    # The oracle sees the padded form with zeroed padding.
    mask = lambda t, s: torch.stack([torch.where(torch.arange(T, device=DEV)[:, None, None] < s[b], t[b], 0)
                                     for b in range(B)])
    bias = (-torch.log(sk.float())).double().numpy()
    want_o, (want_dq, want_dk, want_dv) = oracle_fwd_bwd(
        mask(q, sq), mask(k, sk), mask(v, sk), mask(do, sq), scale=np.float32(1 / math.sqrt(D)), bias=bias,
        seq_lens_q=sq, seq_lens_k=sk, causal=causal)
    sel = lambda a, s: np.concatenate([a[b, :int(s[b])] for b in range(B)], 0)
    assert_close_to_oracle(o, sel(want_o, sq), dtype, "O")
    assert_close_to_oracle(dq, sel(want_dq, sq), dtype, "dQ")
    assert_close_to_oracle(dk, sel(want_dk, sk), dtype, "dK")
    assert_close_to_oracle(dv, sel(want_dv, sk), dtype, "dV")


@pytest.mark.parametrize("D", [64, 128])
def test_varlen_score_mod_equals_padded(D):
    B, T, H = 3, 400, 2
    q, k, v, do, sq, sk = _case(B, T, T, H, D, torch.bfloat16, seed=3)
    g = torch.Generator().manual_seed(4)
    sm = torch.randn((B, T), generator=g).to(DEV)
    _assert_equal_packed(_run_padded(q, k, v, do, sq, sk, True, score_mod=sm),
                         _run_varlen(q, k, v, do, sq, sk, True, score_mod=sm), sq, sk, "score_mod")


def test_varlen_many_sequences_and_zero_lengths():
    """B > 64 (grid in plain order) and empty sequences in the middle."""
    B, T, H, D = 80, 96, 2, 64
    q, k, v, do, sq, sk = _case(B, T, T, H, D, torch.float16, seed=5, lo=0.0)
    sq[::7] = 0
    sk.copy_(sq)
    _assert_equal_packed(_run_padded(q, k, v, do, sq, sk, True),
                         _run_varlen(q, k, v, do, sq, sk, True), sq, sk, "B=80")


def _packed_c_abi(q, k, v, do, cu, T, causal, fill, two_pass=False, halves=False):
    """sigattn_fwd and sigattn_bwd on packed rows through the C ABI, with
    every output pre-filled with `fill`; two_pass: sigattn_bwd_ws with the
    whole dS workspace; halves: sigattn_bwd_dkdv, then sigattn_bwd_dq."""
    lib = _capi.load_library()
    B = cu.numel() - 1
    lens = (cu[1:] - cu[:-1]).clamp(min=1).float()
    bias = -torch.log(lens).to(DEV)
    scale = torch.tensor(1 / math.sqrt(q.shape[-1]), dtype=torch.float32, device=DEV)
    pr = _capi._problem(q, k, v, bias, None, scale, None, None, causal, packed=(cu, cu, T, T))
    out, dq, dk, dv = (torch.full_like(q, fill) for _ in range(4))
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.sigattn_fwd(ctypes.byref(pr), out.data_ptr(), stream) == 0
    if two_pass:
        nbytes = lib.sigattn_bwd_workspace_bytes(ctypes.byref(pr))
        assert nbytes > 0
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        assert lib.sigattn_bwd_ws(ctypes.byref(pr), do.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                  ws.data_ptr(), nbytes, stream) == 0
    elif halves:
        assert lib.sigattn_bwd_dkdv(ctypes.byref(pr), do.data_ptr(), dk.data_ptr(), dv.data_ptr(), stream) == 0
        assert lib.sigattn_bwd_dq(ctypes.byref(pr), do.data_ptr(), dq.data_ptr(), stream) == 0
    else:
        assert lib.sigattn_bwd(ctypes.byref(pr), do.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                               stream) == 0
    torch.cuda.synchronize()
    assert B >= 0
    return out, dq, dk, dv


@pytest.mark.parametrize("D,dtype", [(128, torch.bfloat16), (64, torch.float16), (32, torch.bfloat16),
                                     (16, torch.float16), (32, torch.float32)])
@pytest.mark.parametrize("cu_rows,T,outside", [
    # non-decreasing cu: rows before cu[0] and past cu[B], and rows 550..610
    # past the longest sequence T = 300 of the 361-row sequence 2
    ([40, 250, 250, 611], 300, [(0, 40), (550, 611), (611, 700)]),
    # decreasing cu (sequence 1 is empty): rows 100..299 and 400.. outside
    ([300, 400, 0, 100], 100, [(100, 300), (400, 700)]),
], ids=["sorted", "unsorted"])
def test_packed_rows_outside_sequences_are_zero(D, dtype, cu_rows, T, outside):
    """Through the C ABI, outputs pre-filled with NaN: the rows no sequence
    covers come back as zeros in O, dQ, dK and dV, the rows of the sequences
    are finite and equal to a run whose outputs started as zeros."""
    H, rows = 2, 700
    g = torch.Generator().manual_seed(9)
    q, k, v, do = (randn((rows, H, D), dtype, DEV, g) for _ in range(4))
    cu = torch.tensor(cu_rows, dtype=torch.int32, device=DEV)
    got = _packed_c_abi(q, k, v, do, cu, T, True, float("nan"))
    ref = _packed_c_abi(q, k, v, do, cu, T, True, 0.0)
    mask = torch.zeros(rows, dtype=torch.bool, device=DEV)
    for a, b in outside:
        mask[a:b] = True
    for name, t, r in zip(("O", "dQ", "dK", "dV"), got, ref):
        assert torch.all(t[mask] == 0), f"{name}: rows outside every sequence are not zero"
        assert torch.all(torch.isfinite(t[~mask])), f"{name}: a sequence row is not finite"
        assert torch.equal(t, r), f"{name}: differs from the run on zero-filled outputs"


@pytest.mark.parametrize("how", ["two_pass", "halves"])
def test_packed_gap_rows_other_backward_paths(how):
    """The gap rows are zeroed on the backward's other routes too: the
    two-pass backward (its first dQ-from-dS launch zeroes the dQ, dK and dV
    gaps) and the halves called one by one (dK/dV alone zeroes its own by a
    launch of its own)."""
    H, D, rows, T = 2, 128, 700, 300
    g = torch.Generator().manual_seed(10)
    q, k, v, do = (randn((rows, H, D), torch.bfloat16, DEV, g) for _ in range(4))
    cu = torch.tensor([40, 250, 250, 611], dtype=torch.int32, device=DEV)
    kw = {how: True}
    got = _packed_c_abi(q, k, v, do, cu, T, True, float("nan"), **kw)
    ref = _packed_c_abi(q, k, v, do, cu, T, True, 0.0, **kw)
    mask = torch.zeros(rows, dtype=torch.bool, device=DEV)
    for a, b in [(0, 40), (550, 611), (611, 700)]:
        mask[a:b] = True
    for name, t, r in zip(("O", "dQ", "dK", "dV"), got, ref):
        assert torch.all(t[mask] == 0), f"{name}: rows outside every sequence are not zero"
        assert torch.all(torch.isfinite(t[~mask])), f"{name}: a sequence row is not finite"
        assert torch.equal(t, r), f"{name}: differs from the run on zero-filled outputs"


def test_packed_api_rows_outside_sequences_are_zero():
    """The public API (C++ and Python nodes alike go through the C ABI):
    cu_seqlens covering rows 0..599 of 640, and B = 0 (no sequence at all)."""
    H, D, rows = 2, 64, 640
    g = torch.Generator().manual_seed(12)
    q, k, v, do = (randn((rows, H, D), torch.bfloat16, DEV, g).requires_grad_(True) for _ in range(4))
    cu = torch.tensor([0, 250, 600], dtype=torch.int32, device=DEV)
    o = ts.sigmoid_attention_varlen(q, k, v, cu, cu, 350, 350, is_causal=True)
    o.backward(do.detach())
    for name, t in (("O", o), ("dQ", q.grad), ("dK", k.grad), ("dV", v.grad)):
        assert torch.all(t[600:] == 0), name
        assert torch.all(torch.isfinite(t[:600])), name
    none = torch.zeros(1, dtype=torch.int32, device=DEV)
    leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v)]
    o = ts.sigmoid_attention_varlen(*leaves, none, none, 0, 0)
    o.backward(do.detach())
    for name, t in zip(("O", "dQ", "dK", "dV"), [o] + [t.grad for t in leaves]):
        assert torch.all(t == 0), f"B = 0: {name} is not all zeros"


def test_varlen_empty_batch_and_validation():
    H, D = 2, 64
    q = torch.zeros((0, H, D), dtype=torch.bfloat16, device=DEV)
    cu = torch.zeros(1, dtype=torch.int32, device=DEV)
    assert ts.sigmoid_attention_varlen(q, q, q, cu, cu).shape == (0, H, D)
    x = torch.zeros((10, H, D), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="3D tensors"):
        ts.sigmoid_attention_varlen(x[None], x[None], x[None], cu, cu)
    with pytest.raises(ValueError, match="same shape"):
        ts.sigmoid_attention_varlen(x, x, x, torch.tensor([0, 10], device=DEV),
                                    torch.tensor([0, 5, 10], device=DEV))
    with pytest.raises(ValueError, match="score_mod must have shape"):
        ts.sigmoid_attention_varlen(x, x, x, cu, cu, score_mod=torch.zeros(3, device=DEV))


def test_varlen_under_torch_compile():
    B, T, H, D = 3, 256, 4, 64
    q, k, v, do, sq, sk = _case(B, T, T, H, D, torch.bfloat16, seed=21)
    qp, kp, vp = _pack(q, sq), _pack(k, sk), _pack(v, sk)
    cq, ck = _cu(sq).to(DEV), _cu(sk).to(DEV)
    mq, mk = int(sq.max()), int(sk.max())
    torch._dynamo.reset()
    fn = lambda a, b, c, **kw: ts.sigmoid_attention_varlen(a, b, c, cq, ck, mq, mk, is_causal=True, **kw)
    compiled = torch.compile(fn, fullgraph=True)
    le = [t.clone().requires_grad_(True) for t in (qp, kp, vp)]
    lc = [t.clone().requires_grad_(True) for t in (qp, kp, vp)]
    oe, oc = fn(*le), compiled(*lc)
    # Compiled, the default bias -log(len) comes from Inductor's own kernel and
    # may differ from eager ATen by an fp32 ulp (as for the padded op).
    tol = 2 * 7e-3
    torch.testing.assert_close(oe, oc, atol=tol, rtol=0)
    dop = _pack(do, sq)
    oe.backward(dop)
    oc.backward(dop)
    for a, b in zip(le, lc):
        torch.testing.assert_close(a.grad, b.grad, atol=tol, rtol=0)
    # With an explicit bias both run identical kernels: bitwise equal.
    assert torch.equal(compiled(qp, kp, vp, sigmoid_bias=-3.0), fn(qp, kp, vp, sigmoid_bias=-3.0))


def test_varlen_c5_shape_equals_padded():
    """BASELINE configs[4] (bf16 B=4 Lmax=8192 H=12 D=64, non-causal) packed."""
    B, T, H, D = 4, 8192, 12, 64
    q, k, v, do, sq, sk = _case(B, T, T, H, D, torch.bfloat16, seed=1, lo=0.125)
    _assert_equal_packed(_run_padded(q, k, v, do, sq, sk, False),
                         _run_varlen(q, k, v, do, sq, sk, False), sq, sk, "c5 shape")
