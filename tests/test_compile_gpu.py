"""torch.compile on the GPU: compiled == eager for both APIs, forward and
backward (mirrors the reference's tests/test_torch_compile.py), plus the
padded BASELINE configurations (c4 eager, c5 through torch.compile) at full
size against an fp32 eager reference (max-abs <= 2e-2)."""

import pytest
import torch

import triton_sigmoid as ts
from helpers import randn
from oracle.eager import sigmoid_attention_eager

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _qkv(B, T, H, D, dtype, seed, Tk=None):
    g = torch.Generator().manual_seed(seed)
    Tk = Tk or T
    return (randn((B, T, H, D), dtype, DEV, g), randn((B, Tk, H, D), dtype, DEV, g),
            randn((B, Tk, H, D), dtype, DEV, g), randn((B, T, H, D), dtype, DEV, g))


@pytest.mark.parametrize("D,dtype", [(64, torch.float16), (128, torch.bfloat16)])
@pytest.mark.parametrize("causal", [False, True])
def test_compiled_dense_matches_eager(causal, D, dtype):
    """D = 128 takes the two-pass backward (dS workspace allocated inside the
    compiled op), D = 64 the recompute backward."""
    torch._dynamo.reset()
    q, k, v, do = _qkv(2, 256, 4, D, dtype, 1)
    f = torch.compile(ts.sigmoid_attention, fullgraph=True)
    leaves_e = [t.clone().requires_grad_(True) for t in (q, k, v)]
    leaves_c = [t.clone().requires_grad_(True) for t in (q, k, v)]
    oe = ts.sigmoid_attention(*leaves_e, is_causal=causal)
    oc = f(*leaves_c, is_causal=causal)
    assert torch.equal(oe, oc)
    oe.backward(do)
    oc.backward(do)
    for a, b in zip(leaves_e, leaves_c):
        assert torch.equal(a.grad, b.grad)


def test_compiled_dense_score_mod_and_recompile_new_shapes():
    torch._dynamo.reset()
    f = torch.compile(ts.sigmoid_attention)
    for B, T in [(1, 128), (2, 192), (3, 320)]:
        q, k, v, _ = _qkv(B, T, 2, 128, torch.bfloat16, B + T)
        sm = torch.randn(B, T, device=DEV)
        assert torch.equal(f(q, k, v, score_mod=sm), ts.sigmoid_attention(q, k, v, score_mod=sm))


@pytest.mark.parametrize("causal", [False, True])
def test_compiled_padded_matches_eager(causal):
    torch._dynamo.reset()
    q, k, v, do = _qkv(3, 200, 2, 64, torch.bfloat16, 2)
    sl = torch.tensor([200, 150, 77], dtype=torch.int32, device=DEV)
    f = torch.compile(ts.sigmoid_attention_padded, fullgraph=True)
    le = [t.clone().requires_grad_(True) for t in (q, k, v)]
    lc = [t.clone().requires_grad_(True) for t in (q, k, v)]
    oe = ts.sigmoid_attention_padded(*le, seq_lens_k=sl, seq_lens_q=sl, is_causal=causal)
    oc = f(*lc, seq_lens_k=sl, seq_lens_q=sl, is_causal=causal)
    # The default bias -log(seq_lens_k) is computed by Inductor's own kernel
    # when compiled, which may differ from eager ATen by an fp32 ulp; the
    # reference's tests/test_torch_compile.py also compares within tolerance.
    tol = 2 * 7e-3
    torch.testing.assert_close(oe, oc, atol=tol, rtol=0)
    oe.backward(do)
    oc.backward(do)
    for a, b in zip(le, lc):
        torch.testing.assert_close(a.grad, b.grad, atol=tol, rtol=0)
    # With an explicit bias both paths run identical kernels: bitwise equal.
    oe = ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sl, seq_lens_q=sl, is_causal=causal,
                                     sigmoid_bias=-3.0)
    oc = f(q, k, v, seq_lens_k=sl, seq_lens_q=sl, is_causal=causal, sigmoid_bias=-3.0)
    assert torch.equal(oe, oc)


def test_compiled_padded_cross_attention_and_new_lmax():
    torch._dynamo.reset()
    f = torch.compile(ts.sigmoid_attention_padded)
    for Tq, Tk in [(32, 512), (64, 256), (96, 1024)]:
        q, k, v, _ = _qkv(2, Tq, 2, 64, torch.float16, Tq, Tk=Tk)
        sk = torch.tensor([Tk, Tk // 2], dtype=torch.int32, device=DEV)
        assert torch.equal(f(q, k, v, seq_lens_k=sk), ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk))


def _padded_case(B, L, H, D, dtype, lo, seed):
    g = torch.Generator().manual_seed(seed)
    sl = torch.randint(lo, L + 1, (B,), generator=g, dtype=torch.int32)
    q, k, v, do = (randn((B, L, H, D), dtype, DEV, g) for _ in range(4))
    for b in range(B):  # padding filled with fresh N(0,1) noise
        for t in (q, k, v, do):
            t[b, sl[b]:] = torch.randn_like(t[b, sl[b]:])
    return q, k, v, do, sl.to(DEV)


def _check_padded_against_fp32(fn, q, k, v, do, sl, causal):
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
    o = fn(*leaves, seq_lens_k=sl, seq_lens_q=sl, is_causal=causal)
    o.backward(do)
    for b in range(q.shape[0]):
        n = int(sl[b])
        qq, kk, vv = (t[b:b + 1, :n].detach().float().requires_grad_(True) for t in (q, k, v))
        ro = sigmoid_attention_eager(qq, kk, vv, sigmoid_bias=-float(torch.log(torch.tensor(float(n)))),
                                     upcast=True, causal=causal)
        ro.backward(do[b:b + 1, :n].float())
        for name, got, want in (("O", o[b:b + 1, :n], ro), ("dQ", leaves[0].grad[b:b + 1, :n], qq.grad),
                                ("dK", leaves[1].grad[b:b + 1, :n], kk.grad),
                                ("dV", leaves[2].grad[b:b + 1, :n], vv.grad)):
            err = (got.float() - want).abs().max().item()
            assert err <= 2e-2, (b, name, err)
        for t in (o, leaves[0].grad, leaves[1].grad, leaves[2].grad):
            assert torch.all(t[b, n:] == 0)


def test_c4_padded_fp16_causal_within_2e2():
    q, k, v, do, sl = _padded_case(8, 2048, 8, 64, torch.float16, 512, seed=4)
    _check_padded_against_fp32(ts.sigmoid_attention_padded, q, k, v, do, sl, causal=True)


def test_c5_padded_bf16_long_context_compiled_within_2e2():
    torch._dynamo.reset()
    q, k, v, do, sl = _padded_case(4, 8192, 12, 64, torch.bfloat16, 1024, seed=5)
    f = torch.compile(ts.sigmoid_attention_padded, fullgraph=True)
    _check_padded_against_fp32(f, q, k, v, do, sl, causal=False)
