"""GPU tests of the C++ autograd node of the eager public APIs
(_sigattn_autograd, csrc/torch_autograd.cpp).  It launches the same kernels
with the same workspace policy as the Python nodes (torch.autograd.Function
in sigmoid_dense.py / sigmoid_padded.py / sigmoid_varlen.py, selected by
SIGATTN_EAGER_BINDING=python), so outputs and gradients must be bitwise
equal to theirs; the Python nodes are checked against the oracle by the
other GPU tests.  The reference's eager path is the Python autograd of
src/triton_sigmoid/sigmoid_triton_dense.py:696-753 and
sigmoid_triton_padded.py:780-846."""

import math

import pytest
import torch

import triton_sigmoid as ts
from helpers import randn
from triton_sigmoid import _capi

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(fn, inputs, do, binding, monkeypatch):
    if binding == "python":
        monkeypatch.setenv("SIGATTN_EAGER_BINDING", "python")
    else:
        monkeypatch.delenv("SIGATTN_EAGER_BINDING", raising=False)
    leaves = [t.detach().clone().requires_grad_(True) for t in inputs]
    o = fn(*leaves)
    node = type(o.grad_fn).__name__
    o.backward(do)
    torch.cuda.synchronize()
    return [o.detach()] + [t.grad for t in leaves], node


def _case(B, Tq, Tk, H, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = randn((B, Tq, H, D), dtype, DEV, g)
    k = randn((B, Tk, H, D), dtype, DEV, g)
    v = randn((B, Tk, H, D), dtype, DEV, g)
    do = randn((B, Tq, H, D), dtype, DEV, g)
    return q, k, v, do


def _assert_same(cpp, py, what):
    (a, node_a), (b, node_b) = cpp, py
    assert node_a == "CppFunction", f"{what}: the C++ node did not run ({node_a})"
    assert node_b.endswith("EagerBackward"), f"{what}: the Python node did not run ({node_b})"
    for name, x, y in zip(("O", "dQ", "dK", "dV"), a, b):
        assert torch.equal(x, y), f"{what}: {name} differs between the C++ and Python nodes"


DENSE = [  # (B, T, H, D, dtype, causal)
    (2, 1024, 8, 64, torch.float16, False),   # c2: too few keys for the range split
    (1, 2048, 4, 64, torch.float16, False),   # range split forward and backward
    (2, 1024, 8, 64, torch.float16, True),
    (2, 384, 4, 128, torch.bfloat16, False),  # two-pass backward
    (1, 2048, 2, 128, torch.bfloat16, False), # range split forward and dQ
    (1, 300, 3, 128, torch.bfloat16, True),
    (2, 77, 2, 32, torch.float32, False),     # fp32 MFMA kernels
    (1, 16, 2, 64, torch.bfloat16, False),    # decode-sized queries
]


@pytest.mark.parametrize("case", DENSE, ids=lambda c: f"B{c[0]}T{c[1]}H{c[2]}D{c[3]}{str(c[4])[6:]}{'c' if c[5] else ''}")
def test_dense_matches_python_node(case, monkeypatch):
    B, T, H, D, dtype, causal = case
    q, k, v, do = _case(B, T, T, H, D, dtype, seed=T + D)
    fn = lambda q, k, v: ts.sigmoid_attention(q, k, v, is_causal=causal)  # noqa: E731
    _assert_same(_run(fn, (q, k, v), do, "cpp", monkeypatch), _run(fn, (q, k, v), do, "python", monkeypatch),
                 str(case))


def test_dense_score_mod_and_bias_match_python_node(monkeypatch):
    B, T, H, D = 2, 520, 2, 64
    q, k, v, do = _case(B, T, T, H, D, torch.bfloat16, seed=5)
    sm = randn((B, T), torch.float32, DEV, torch.Generator().manual_seed(6), std=2.0)
    fn = lambda q, k, v: ts.sigmoid_attention(q, k, v, sigmoid_bias=-2.5, scale=0.2, score_mod=sm)  # noqa: E731
    _assert_same(_run(fn, (q, k, v), do, "cpp", monkeypatch), _run(fn, (q, k, v), do, "python", monkeypatch),
                 "score_mod")


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("D", [64, 128])
def test_padded_matches_python_node(D, causal, monkeypatch):
    B, Tq, Tk, H = 3, 300, 420, 2
    q, k, v, do = _case(B, Tq, Tk, H, D, torch.float16, seed=D + causal)
    sq = torch.tensor([300, 17, 250], dtype=torch.int64, device=DEV)
    sk = torch.tensor([420, 33, 1], dtype=torch.int32, device=DEV)
    fn = lambda q, k, v: ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk, seq_lens_q=sq,  # noqa: E731
                                                     is_causal=causal)
    _assert_same(_run(fn, (q, k, v), do, "cpp", monkeypatch), _run(fn, (q, k, v), do, "python", monkeypatch),
                 f"padded D={D} causal={causal}")


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("D", [64, 128])
def test_varlen_matches_python_node(D, causal, monkeypatch):
    """Packed sequences ([rows, H, D] with cu_seqlens, given as int32 and
    int64), one of a single key."""
    lens_q, lens_k = [300, 17, 250], [420, 33, 1]
    cu_q = torch.tensor([0, 300, 317, 567], dtype=torch.int32, device=DEV)
    cu_k = torch.tensor([0, 420, 453, 454], dtype=torch.int64, device=DEV)
    g = torch.Generator().manual_seed(D + causal)
    H, dtype = 2, torch.bfloat16
    q = randn((567, H, D), dtype, DEV, g)
    k = randn((454, H, D), dtype, DEV, g)
    v = randn((454, H, D), dtype, DEV, g)
    do = randn((567, H, D), dtype, DEV, g)
    fn = lambda q, k, v: ts.sigmoid_attention_varlen(q, k, v, cu_q, cu_k, max(lens_q), max(lens_k),  # noqa: E731
                                                     is_causal=causal)
    _assert_same(_run(fn, (q, k, v), do, "cpp", monkeypatch), _run(fn, (q, k, v), do, "python", monkeypatch),
                 f"varlen D={D} causal={causal}")


@pytest.mark.parametrize("mb", ["2048", "0", "600", "100"])
def test_workspace_limits_match_python_node(mb, monkeypatch):
    """The two-pass policy under several workspace limits at B=4 L=4096 H=16
    causal (67.6 MB of dS per head): the whole dS, none, groups of 8 heads
    (600 MB; 256 dQ-from-dS workgroups) and single heads whose 32-workgroup
    grid takes the recompute backward (100 MB).  A different choice would
    change dQ's summation order."""
    monkeypatch.setenv("SIGATTN_BWD_WORKSPACE_MB", mb)
    q, k, v, do = _case(4, 4096, 4096, 16, 128, torch.bfloat16, seed=11)
    fn = lambda q, k, v: ts.sigmoid_attention(q, k, v, is_causal=True)  # noqa: E731
    _assert_same(_run(fn, (q, k, v), do, "cpp", monkeypatch), _run(fn, (q, k, v), do, "python", monkeypatch),
                 f"limit {mb} MB")


def test_non_contiguous_no_grad_and_empty(monkeypatch):
    monkeypatch.delenv("SIGATTN_EAGER_BINDING", raising=False)
    base = torch.randn(2, 4, 200, 64, device=DEV, dtype=torch.float16)
    q = base.transpose(1, 2)  # [B, T, H, D] view, not contiguous
    qc = q.detach().clone().requires_grad_(True)
    qn = q.detach().clone().requires_grad_(True)
    a = ts.sigmoid_attention(qc, qc, qc)
    b = ts.sigmoid_attention(qn.transpose(1, 2).contiguous().transpose(1, 2), qn, qn)
    assert torch.equal(a, b)
    a.sum().backward()
    b.sum().backward()
    assert torch.equal(qc.grad, qn.grad)
    with torch.no_grad():
        o = ts.sigmoid_attention(q, q, q)
    assert o.grad_fn is None and torch.equal(o, a.detach())
    z = torch.empty(2, 0, 4, 64, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    oz = ts.sigmoid_attention(z, z, z)
    assert oz.shape == z.shape
    oz.sum().backward()
    assert z.grad.shape == z.shape


def test_cpp_node_errors_are_runtime_errors(monkeypatch):
    monkeypatch.delenv("SIGATTN_EAGER_BINDING", raising=False)
    q = torch.randn(1, 64, 2, 48, device=DEV, dtype=torch.float16)  # D = 48: no kernel
    with pytest.raises(RuntimeError, match="sigattn_fwd failed"):
        ts.sigmoid_attention(q, q, q)


def test_cpp_node_workspace_oom_falls_back_to_recompute(monkeypatch):
    """With the device memory taken up, the two-pass workspace cannot be
    allocated: the C++ node's backward runs the recompute kernels instead and
    gives exactly their gradients."""
    monkeypatch.delenv("SIGATTN_EAGER_BINDING", raising=False)
    B, T, H, D = 2, 4096, 16, 128  # whole-problem dS: 1.07 GB
    q, k, v, do = _case(B, T, T, H, D, torch.bfloat16, seed=21)
    fn = lambda q, k, v: ts.sigmoid_attention(q, k, v)  # noqa: E731
    monkeypatch.setenv("SIGATTN_BWD_WORKSPACE_MB", "0")
    ref, node = _run(fn, (q, k, v), do, "cpp", monkeypatch)
    assert node == "CppFunction"
    monkeypatch.delenv("SIGATTN_BWD_WORKSPACE_MB")
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    free, _ = torch.cuda.mem_get_info()
    blocker = torch.empty(free - (400 << 20), dtype=torch.uint8, device=DEV)  # leaves 400 MB
    try:
        got, _ = _run(fn, (q, k, v), do, "cpp", monkeypatch)
    finally:
        del blocker
        torch.cuda.empty_cache()
    for name, x, y in zip(("O", "dQ", "dK", "dV"), got, ref):
        assert torch.equal(x, y), f"{name}: OOM fallback differs from the recompute backward"


HOOK_CASES = [  # (B, Tq, Tk, H, D, dtype, causal, padded)
    (2, 384, 384, 4, 128, torch.bfloat16, True, False),   # two-pass backward
    (1, 2048, 2048, 4, 64, torch.float16, False, False),  # range-split recompute backward
    (3, 300, 420, 2, 64, torch.float16, True, True),      # padded
]


@pytest.mark.parametrize("binding", ["cpp", "python"])
@pytest.mark.parametrize("hook", ["save_on_cpu", "checkpoint"])
@pytest.mark.parametrize("case", HOOK_CASES, ids=lambda c: f"D{c[4]}{'p' if c[7] else ''}{'c' if c[6] else ''}")
def test_saved_tensor_hooks_give_plain_gradients(case, hook, binding, monkeypatch):
    """Under saved-tensor hooks the backward receives new Q / K / V tensors at
    new addresses, and the forward's buffers (Q, K, V are computed inside the
    hooked region here) are freed and then overwritten with NaN: the gradients
    must still equal those of a plain backward bit for bit."""
    B, Tq, Tk, H, D, dtype, causal, padded = case
    q, k, v, do = _case(B, Tq, Tk, H, D, dtype, seed=Tq + D)
    if padded:
        sq = torch.tensor([Tq, 17, 250], dtype=torch.int32, device=DEV)
        sk = torch.tensor([Tk, 33, 1], dtype=torch.int32, device=DEV)

    def fn(q, k, v):
        q, k, v = q * 1.0, k * 1.0, v * 1.0  # fresh buffers, referenced only by the saved tensors
        if padded:
            return ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sk, seq_lens_q=sq, is_causal=causal)
        return ts.sigmoid_attention(q, k, v, is_causal=causal)

    want, _ = _run(fn, (q, k, v), do, binding, monkeypatch)
    leaves = [t.detach().clone().requires_grad_(True) for t in (q, k, v)]
    if hook == "save_on_cpu":
        with torch.autograd.graph.save_on_cpu():
            o = fn(*leaves)
    else:
        o = torch.utils.checkpoint.checkpoint(fn, *leaves, use_reentrant=False)
    junk = [torch.full_like(t, float("nan")) for t in (q, k, v, q, k, v)]
    o.backward(do)
    torch.cuda.synchronize()
    del junk
    for name, x, y in zip(("O", "dQ", "dK", "dV"), [o.detach()] + [t.grad for t in leaves], want):
        assert torch.equal(x, y), f"{name} under {hook} ({binding} node) differs from the plain backward"
