"""GPU parity tests for the split-KV forward (decode shapes: Tq <= 32 queries
against Tk >= 256 keys, non-causal), which sigmoid_attention_padded and
sigmoid_attention_varlen take automatically.  The reference has no separate
decode path: its padded forward (sigmoid_triton_padded.py:24-171) computes
these shapes with one program per 16..128-query block, so the semantics, and
the float64 oracle they are checked against, are the padded forward's."""

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


def _case(B, Tq, Tk, H, D, dtype, seed, full=False):
    g = torch.Generator().manual_seed(seed)
    q = randn((B, Tq, H, D), dtype, DEV, g)
    k = randn((B, Tk, H, D), dtype, DEV, g)
    v = randn((B, Tk, H, D), dtype, DEV, g)
    sk = torch.full((B,), Tk, dtype=torch.int32) if full else torch.randint(1, Tk + 1, (B,), generator=g,
                                                                             dtype=torch.int32)
    sq = torch.full((B,), Tq, dtype=torch.int32) if full else torch.randint(0, Tq + 1, (B,), generator=g,
                                                                             dtype=torch.int32)
    for b in range(B):  # padding holds NaN: it must never be read
        k[b, sk[b]:] = float("nan")
        v[b, sk[b]:] = float("nan")
        q[b, sq[b]:] = float("nan")
    return q, k, v, sq, sk


def _clean(t, lens):
    t = t.detach().clone()
    for b in range(t.shape[0]):
        t[b, int(lens[b]):] = 0
    return t




@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("Tq,Tk", [(1, 256), (1, 4099), (5, 1000), (32, 20000), (17, 300)])
def test_decode_matches_oracle(dtype, D, Tq, Tk):
    # D = 16 and 32, and fp32, have no split-KV kernel: one MFMA forward
    # workgroup per 128 queries.
    B, H = 3, 4
    q, k, v, sq, sk = _case(B, Tq, Tk, H, D, dtype, seed=Tq * 1000 + Tk + D)
    o = ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk.to(DEV), seq_lens_q=sq.to(DEV))
    bias = (-torch.log(sk.float())).double().numpy()
    want, _ = oracle_fwd_bwd(_clean(q, sq), _clean(k, sk), _clean(v, sk), None,
                             scale=np.float32(1 / math.sqrt(D)), bias=bias, seq_lens_q=sq, seq_lens_k=sk,
                             with_bwd=False)
    assert_close_to_oracle(o, want, dtype, "O")
    for b in range(B):
        assert torch.all(o[b, sq[b]:] == 0)


@pytest.mark.parametrize("D", [64, 128])
def test_decode_score_mod_matches_oracle(D):
    B, Tq, Tk, H = 2, 3, 3000, 2
    q, k, v, sq, sk = _case(B, Tq, Tk, H, D, torch.bfloat16, seed=7)
    g = torch.Generator().manual_seed(8)
    sm = torch.randn((B, Tk), generator=g).to(DEV)
    o = ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk.to(DEV), seq_lens_q=sq.to(DEV), score_mod=sm,
                                    sigmoid_bias=-4.0)
    want, _ = oracle_fwd_bwd(_clean(q, sq), _clean(k, sk), _clean(v, sk), None,
                             scale=np.float32(1 / math.sqrt(D)), bias=np.full(B, -4.0), score_mod=sm,
                             seq_lens_q=sq, seq_lens_k=sk, with_bwd=False)
    assert_close_to_oracle(o, want, torch.bfloat16, "O")


@pytest.mark.parametrize("D", [64, 128])
def test_split_and_single_chunk_agree(D):
    """With a workspace the keys are cut into chunks; without one each
    (batch, head) is one chunk.  Both are deterministic and agree up to the
    fp32 summation order (a few bf16 ulps at most)."""
    lib = _capi.load_library()
    B, Tq, Tk, H = 2, 4, 9000, 2
    q, k, v, sq, sk = _case(B, Tq, Tk, H, D, torch.bfloat16, seed=D, full=True)
    bias = torch.full((B,), -math.log(Tk), device=DEV)
    scale = torch.tensor(1 / math.sqrt(D), device=DEV)
    sq_d, sk_d = sq.to(DEV), sk.to(DEV)   # the problem holds raw pointers: keep them alive
    pr = _capi._problem(q, k, v, bias, None, scale, sq_d, sk_d, False)
    nbytes = lib.sigattn_fwd_workspace_bytes(ctypes.byref(pr))
    assert nbytes > 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for w in (ws, ws, None):
        o = torch.full_like(q, float("nan"))
        rc = lib.sigattn_fwd_ws(ctypes.byref(pr), o.data_ptr(), None if w is None else w.data_ptr(),
                                0 if w is None else nbytes, stream)
        assert rc == 0
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    torch.testing.assert_close(outs[0], outs[2], atol=2 ** -7 * outs[2].abs().max().item(), rtol=0)
    want, _ = oracle_fwd_bwd(q, k, v, None, scale=np.float32(1 / math.sqrt(D)),
                             bias=np.full(B, -math.log(Tk), dtype=np.float32).astype(np.float64),
                             seq_lens_q=sq, seq_lens_k=sk, with_bwd=False)
    assert_close_to_oracle(outs[0], want, torch.bfloat16, "split")
    assert_close_to_oracle(outs[2], want, torch.bfloat16, "single chunk")


def test_decode_packed_sequences():
    """Packed layout: one query per sequence against its own cache."""
    B, H, D = 6, 4, 128
    g = torch.Generator().manual_seed(12)
    lens_k = torch.randint(200, 5000, (B,), generator=g)
    cu_k = torch.cat([torch.zeros(1, dtype=torch.int64), lens_k.cumsum(0)]).to(torch.int32)
    cu_q = torch.arange(B + 1, dtype=torch.int32)
    q = randn((B, H, D), torch.bfloat16, DEV, g)
    k = randn((int(cu_k[-1]), H, D), torch.bfloat16, DEV, g)
    v = randn((int(cu_k[-1]), H, D), torch.bfloat16, DEV, g)
    o = ts.sigmoid_attention_varlen(q, k, v, cu_q.to(DEV), cu_k.to(DEV), 1, int(lens_k.max()))
    for b in range(B):
        ks, ke = int(cu_k[b]), int(cu_k[b + 1])
        want, _ = oracle_fwd_bwd(q[b:b + 1, None], k[None, ks:ke], v[None, ks:ke], None,
                                 scale=np.float32(1 / math.sqrt(D)),
                                 bias=(-torch.log(torch.tensor([float(ke - ks)]))).double().numpy(),
                                 with_bwd=False)
        assert_close_to_oracle(o[b:b + 1, None], want, torch.bfloat16, f"seq {b}")


def test_decode_backward_through_autograd():
    """Decode-shaped problems keep the standard backward kernels."""
    B, Tq, Tk, H, D = 2, 4, 1500, 2, 64
    q, k, v, sq, sk = _case(B, Tq, Tk, H, D, torch.float16, seed=5, full=True)
    g = torch.Generator().manual_seed(6)
    do = randn((B, Tq, H, D), torch.float16, DEV, g)
    for t in (q, k, v):
        t.requires_grad_(True)
    o = ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk.to(DEV), seq_lens_q=sq.to(DEV))
    o.backward(do)
    want_o, (dq, dk, dv) = oracle_fwd_bwd(q, k, v, do, scale=np.float32(1 / math.sqrt(D)),
                                          bias=(-torch.log(sk.float())).double().numpy(),
                                          seq_lens_q=sq, seq_lens_k=sk)
    assert_close_to_oracle(o, want_o, torch.float16, "O")
    assert_close_to_oracle(q.grad, dq, torch.float16, "dQ")
    assert_close_to_oracle(k.grad, dk, torch.float16, "dK")
    assert_close_to_oracle(v.grad, dv, torch.float16, "dV")


def test_decode_long_cache_sum_of_halves():
    """Size-independent check at a long cache (B=1, H=8, Tk=131072): O over
    the whole cache equals O over its two halves summed (same bias), within
    the bf16 rounding of the three outputs."""
    B, Tq, Tk, H, D = 1, 1, 131072, 8, 128
    q, k, v, sq, sk = _case(B, Tq, Tk, H, D, torch.bfloat16, seed=99, full=True)
    f = lambda kk, vv: ts.sigmoid_attention_padded(q, kk, vv, sigmoid_bias=-math.log(Tk)).float()
    whole = f(k, v)
    h1, h2 = f(k[:, :Tk // 2], v[:, :Tk // 2]), f(k[:, Tk // 2:], v[:, Tk // 2:])
    mag = max(t.abs().max().item() for t in (whole, h1, h2))
    torch.testing.assert_close(whole, h1 + h2, atol=3 * 2 ** -8 * mag, rtol=0)
