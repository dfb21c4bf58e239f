"""CPU tests of the public API and the operator boundary (no GPU needed):
ValueError texts of the reference API, custom-op names and schemas, fake
(meta) kernels, torch.compile tracing without graph breaks, the loud failure
without a GPU, and the exported eager sigmoid_attention_ref against the
float64 oracle."""

import math
import re

import numpy as np
import pytest
import torch

import triton_sigmoid as ts
from oracle import sigmoid_oracle as so


def _t(*shape):
    return torch.randn(*shape)


# --- validation (reference: sigmoid_triton_dense.py:803-823, sigmoid_triton_padded.py:940-981)

@pytest.mark.parametrize("fn", [ts.sigmoid_attention, ts.sigmoid_attention_padded])
def test_rank_error(fn):
    with pytest.raises(ValueError, match="Expected query, key, and value to be 4D tensors"):
        fn(_t(2, 8, 16), _t(2, 8, 2, 16), _t(2, 8, 2, 16))


@pytest.mark.parametrize("fn", [ts.sigmoid_attention, ts.sigmoid_attention_padded])
@pytest.mark.parametrize("shapes,msg", [
    (((2, 8, 2, 16), (3, 8, 2, 16), (2, 8, 2, 16)), "Batch size mismatch: Q=2, K=3, V=2"),
    (((2, 8, 2, 16), (2, 8, 4, 16), (2, 8, 2, 16)), "Number of heads mismatch: Q=2, K=4, V=2"),
    (((2, 8, 2, 16), (2, 8, 2, 32), (2, 8, 2, 16)), "Head dimension mismatch: Q=16, K=32, V=16"),
])
def test_shape_mismatch_errors(fn, shapes, msg):
    with pytest.raises(ValueError, match=re.escape(msg)):
        fn(*(_t(*s) for s in shapes))


def test_dense_requires_same_lengths():
    with pytest.raises(ValueError, match="Dense attention requires same sequence length for Q, K, V, got 8, 16, 16"):
        ts.sigmoid_attention(_t(2, 8, 2, 16), _t(2, 16, 2, 16), _t(2, 16, 2, 16))


def test_padded_requires_same_key_value_lengths():
    with pytest.raises(ValueError, match="Key and value sequence lengths must match, got K=16, V=8"):
        ts.sigmoid_attention_padded(_t(2, 8, 2, 16), _t(2, 16, 2, 16), _t(2, 8, 2, 16))


@pytest.mark.parametrize("fn", [ts.sigmoid_attention, ts.sigmoid_attention_padded])
def test_score_mod_shape_error(fn):
    with pytest.raises(ValueError, match=r"score_mod must have shape \(2, 8\)"):
        fn(_t(2, 8, 2, 16), _t(2, 8, 2, 16), _t(2, 8, 2, 16), score_mod=torch.zeros(2, 7))


def test_seq_lens_shape_errors():
    q = _t(2, 8, 2, 16)
    with pytest.raises(ValueError, match=r"seq_lens_k must have shape \(2,\)"):
        ts.sigmoid_attention_padded(q, q, q, seq_lens_k=torch.tensor([1, 2, 3]))
    with pytest.raises(ValueError, match=r"seq_lens_q must have shape \(2,\)"):
        ts.sigmoid_attention_padded(q, q, q, seq_lens_q=torch.tensor([[1, 2]]))


# --- no fallback: the kernels need a gfx950 GPU

@pytest.mark.parametrize("fn", [ts.sigmoid_attention, ts.sigmoid_attention_padded])
def test_cpu_tensors_fail_loudly(fn):
    q = _t(1, 8, 2, 16)
    with pytest.raises(RuntimeError, match="gfx950"):
        fn(q, q, q)


def test_varlen_cpu_tensors_fail_loudly():
    q = torch.randn(12, 2, 16)
    cu = torch.tensor([0, 5, 12], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="gfx950"):
        ts.sigmoid_attention_varlen(q, q, q, cu, cu)


# --- packed (THD) API validation

def test_varlen_validation_errors():
    q = torch.randn(12, 2, 16)
    cu = torch.tensor([0, 5, 12], dtype=torch.int32)
    with pytest.raises(ValueError, match="3D tensors"):
        ts.sigmoid_attention_varlen(q[None], q[None], q[None], cu, cu)
    with pytest.raises(ValueError, match="Number of heads mismatch"):
        ts.sigmoid_attention_varlen(q, torch.randn(12, 3, 16), torch.randn(12, 3, 16), cu, cu)
    with pytest.raises(ValueError, match="Head dimension mismatch"):
        ts.sigmoid_attention_varlen(q, torch.randn(12, 2, 32), torch.randn(12, 2, 32), cu, cu)
    with pytest.raises(ValueError, match="Key and value token counts must match"):
        ts.sigmoid_attention_varlen(q, q, torch.randn(11, 2, 16), cu, cu)
    with pytest.raises(ValueError, match=r"cu_seqlens_q must have shape \(B \+ 1,\)"):
        ts.sigmoid_attention_varlen(q, q, q, cu[None], cu)
    with pytest.raises(ValueError, match="same shape"):
        ts.sigmoid_attention_varlen(q, q, q, cu, torch.tensor([0, 12], dtype=torch.int32))
    with pytest.raises(ValueError, match=r"score_mod must have shape \(12,\)"):
        ts.sigmoid_attention_varlen(q, q, q, cu, cu, score_mod=torch.zeros(2, 12))
    with pytest.raises(ValueError, match="non-negative"):
        ts.sigmoid_attention_varlen(q, q, q, cu, cu, max_seqlen_q=-1, max_seqlen_k=7)


# --- operator boundary: names and schemas of the reference's ops

@pytest.mark.parametrize("name,schema_args", [
    ("sigmoid_attention_fwd", ["Q", "K", "V", "bias", "score_mod", "sm_scale", "is_causal"]),
    ("sigmoid_attention_bwd", ["Q", "K", "V", "dO", "bias", "score_mod", "sm_scale", "is_causal"]),
    ("sigmoid_attn_padded_fwd", ["Q", "K", "V", "seq_lens_k", "seq_lens_q", "bias", "score_mod",
                                 "sm_scale", "is_causal"]),
    ("sigmoid_attn_padded_bwd", ["Q", "K", "V", "dO", "seq_lens_k", "seq_lens_q", "bias", "score_mod",
                                 "sm_scale", "is_causal"]),
    ("sigmoid_attn_varlen_fwd", ["Q", "K", "V", "cu_seqlens_k", "cu_seqlens_q", "max_seqlen_k", "max_seqlen_q",
                                 "bias", "score_mod", "sm_scale", "is_causal"]),
    ("sigmoid_attn_varlen_bwd", ["Q", "K", "V", "dO", "cu_seqlens_k", "cu_seqlens_q", "max_seqlen_k",
                                 "max_seqlen_q", "bias", "score_mod", "sm_scale", "is_causal"]),
])
def test_ops_registered_with_reference_schemas(name, schema_args):
    op = getattr(torch.ops.myops, name).default
    args = [a.name for a in op._schema.arguments]
    assert args == schema_args
    types = {a.name: str(a.type) for a in op._schema.arguments}
    assert types["score_mod"] == "Optional[Tensor]"
    assert types["is_causal"] == "bool"
    n_out = 3 if name.endswith("bwd") else 1
    assert len(op._schema.returns) == n_out


def test_fake_tensor_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        q = torch.empty(2, 32, 4, 64, dtype=torch.bfloat16)
        k = torch.empty(2, 48, 4, 64, dtype=torch.bfloat16)
        sl = torch.empty(2, dtype=torch.int32)
        bias = torch.empty(2)
        sc = torch.empty(())
        o = torch.ops.myops.sigmoid_attn_padded_fwd(q, k, k, sl, sl, bias, None, sc, False)
        assert o.shape == q.shape and o.dtype == q.dtype
        dq, dk, dv = torch.ops.myops.sigmoid_attn_padded_bwd(q, k, k, q, sl, sl, bias, None, sc, True)
        assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == k.shape
        o = torch.ops.myops.sigmoid_attention_fwd(q, q, q, bias, None, sc, True)
        assert o.shape == q.shape
        qp, kp = torch.empty(50, 4, 64, dtype=torch.bfloat16), torch.empty(70, 4, 64, dtype=torch.bfloat16)
        cu = torch.empty(3, dtype=torch.int32)
        o = torch.ops.myops.sigmoid_attn_varlen_fwd(qp, kp, kp, cu, cu, 40, 30, bias, None, sc, True)
        assert o.shape == qp.shape and o.dtype == qp.dtype
        dq, dk, dv = torch.ops.myops.sigmoid_attn_varlen_bwd(qp, kp, kp, qp, cu, cu, 40, 30, bias, None, sc, False)
        assert dq.shape == qp.shape and dk.shape == kp.shape and dv.shape == kp.shape


def _trace_only_backend(graphs):
    def backend(gm, example_inputs):
        graphs.append(gm)
        def run(*args):
            raise RuntimeError("trace-only backend")
        return run
    return backend


@pytest.mark.parametrize("padded", [False, True])
def test_torch_compile_fullgraph_traces_one_op(padded):
    """The custom op is one opaque node: dynamo traces the API with fullgraph=True
    (no graph breaks) on CPU; execution is left to the GPU tests."""
    torch._dynamo.reset()
    graphs = []
    fn = ts.sigmoid_attention_padded if padded else ts.sigmoid_attention
    compiled = torch.compile(fn, backend=_trace_only_backend(graphs), fullgraph=True)
    q = _t(2, 16, 2, 32)
    with pytest.raises(RuntimeError, match="trace-only backend"):
        if padded:
            compiled(q, q, q, torch.tensor([10, 16], dtype=torch.int32), None, True)
        else:
            compiled(q, q, q, True)
    assert len(graphs) == 1
    targets = [str(n.target) for n in graphs[0].graph.nodes if n.op == "call_function"]
    wanted = "myops.sigmoid_attn_padded_fwd" if padded else "myops.sigmoid_attention_fwd"
    assert any(wanted in t for t in targets), targets


# --- exported eager reference == float64 oracle

@pytest.mark.parametrize("causal", [False, True])
def test_exported_reference_matches_oracle(causal):
    rng = np.random.default_rng(0)
    B, Tq, Tk, H, D = 2, 9, 11, 2, 8
    q, k, v = (rng.standard_normal(s) for s in [(B, Tq, H, D), (B, Tk, H, D), (B, Tk, H, D)])
    sm = rng.standard_normal((B, Tk))
    sq, sk = np.array([9, 4]), np.array([7, 11])
    out = ts.sigmoid_attention_ref(torch.tensor(q), torch.tensor(k), torch.tensor(v),
                                   seq_lens_k=torch.tensor(sk), seq_lens_q=torch.tensor(sq),
                                   scale=0.3, sigmoid_bias=-1.25, upcast=False, causal=causal,
                                   score_mod=torch.tensor(sm))
    want = so.forward(q, k, v, scale=0.3, bias=np.full(B, -1.25), score_mod=sm,
                      seq_lens_q=sq, seq_lens_k=sk, causal=causal)
    np.testing.assert_allclose(out.numpy(), want, rtol=1e-12, atol=1e-13)


def test_exported_reference_default_bias_has_epsilon():
    q = torch.zeros(1, 4, 1, 2, dtype=torch.float64)
    v = torch.ones(1, 4, 1, 2, dtype=torch.float64)
    out = ts.sigmoid_attention_ref(q, q, v, upcast=False)
    want = 4 / (1 + math.exp(math.log(4 + 1e-6)))
    assert abs(out[0, 0, 0, 0].item() - want) < 1e-12
