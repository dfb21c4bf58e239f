"""A whole forward + backward step captured in a HIP graph (torch.cuda.graph)
and replayed: every replay must reproduce the eager step bit for bit.  The
step allocates (outputs, gradients, the two-pass backward's dS workspace,
the range split's partials, the default bias and scale tensors) and launches
the library's kernels on the capturing stream; none of it may be a host-side
shortcut that a replay skips."""

import pytest
import torch

import triton_sigmoid as ts
from helpers import randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(kind):
    g = torch.Generator().manual_seed(11)
    if kind == "dense_d128_causal":
        B, T, H, D, dtype = 2, 320, 4, 128, torch.bfloat16
        q, k, v, do = (randn((B, T, H, D), dtype, DEV, g) for _ in range(4))
        return (q, k, v, do), lambda q, k, v: ts.sigmoid_attention(q, k, v, is_causal=True)
    if kind == "dense_d64_range_split":
        # A small dense non-causal grid: forward, dQ and dK/dV range-split,
        # their arrival counters cleared by a captured kernel each replay.
        B, T, H, D, dtype = 1, 2100, 2, 64, torch.float16
        q, k, v, do = (randn((B, T, H, D), dtype, DEV, g) for _ in range(4))
        return (q, k, v, do), lambda q, k, v: ts.sigmoid_attention(q, k, v)
    if kind == "dense_d64_one_launch_bwd":
        # c2's causal shape: the backward's two kernels as one launch.
        B, T, H, D, dtype = 2, 1024, 8, 64, torch.float16
        q, k, v, do = (randn((B, T, H, D), dtype, DEV, g) for _ in range(4))
        return (q, k, v, do), lambda q, k, v: ts.sigmoid_attention(q, k, v, is_causal=True)
    if kind == "fp32_d128":
        B, T, H, D, dtype = 1, 300, 2, 128, torch.float32
        q, k, v, do = (randn((B, T, H, D), dtype, DEV, g) for _ in range(4))
        return (q, k, v, do), lambda q, k, v: ts.sigmoid_attention(q, k, v, is_causal=True)
    if kind == "packed_d64_gaps":
        # Rows 510-570 lie past max_seqlen 300 of the 361-row sequence and
        # rows 571-639 past cu[B]: the launches' leading workgroups zero them.
        rows, H, D, dtype = 640, 2, 64, torch.float16
        q, k, v, do = (randn((rows, H, D), dtype, DEV, g) for _ in range(4))
        cu = torch.tensor([0, 210, 210, 571], dtype=torch.int32, device=DEV)
        return (q, k, v, do), lambda q, k, v: ts.sigmoid_attention_varlen(q, k, v, cu, cu, 300, 300,
                                                                           is_causal=True)
    if kind == "padded_d64_concurrent_bwd":
        # Large enough (B·H·T/128 = 2048 query blocks, eight per CU) for the
        # eager backward to run its two kernels on two streams; under capture
        # the library keeps them on the capturing stream.
        B, T, H, D, dtype = 2, 4096, 32, 64, torch.float16
        q, k, v, do = (randn((B, T, H, D), dtype, DEV, g) for _ in range(4))
        sl = torch.tensor([4096, 2500], dtype=torch.int32, device=DEV)
        return (q, k, v, do), lambda q, k, v: ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sl, seq_lens_q=sl)
    B, T, H, D, dtype = 3, 200, 2, 64, torch.float16
    q, k, v, do = (randn((B, T, H, D), dtype, DEV, g) for _ in range(4))
    sl = torch.tensor([200, 77, 130], dtype=torch.int32, device=DEV)
    return (q, k, v, do), lambda q, k, v: ts.sigmoid_attention_padded(q, k, v, seq_lens_k=sl, seq_lens_q=sl)


@pytest.mark.parametrize("kind", ["dense_d128_causal", "dense_d64_range_split", "padded_d64",
                                  "dense_d64_one_launch_bwd", "fp32_d128", "packed_d64_gaps",
                                  "padded_d64_concurrent_bwd"])
def test_graph_replays_match_eager(kind):
    (q, k, v, do), attn = _case(kind)
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]

    def step():
        for t in leaves:
            t.grad = None
        o = attn(*leaves)
        o.backward(do)
        return o

    o_ref = step().detach().clone()
    grads_ref = [t.grad.clone() for t in leaves]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    for t in leaves:
        t.grad = None
    with torch.cuda.graph(graph):
        o_static = attn(*leaves)
        o_static.backward(do)
    grads_static = [t.grad for t in leaves]

    for rep in range(3):
        # eager work and synchronisation between replays; the static outputs
        # are overwritten so a replay that skips a kernel shows
        scratch = (q.float() * 2.0).sum()
        for t in (o_static, *grads_static):
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(scratch)
        assert torch.equal(o_static, o_ref), f"replay {rep}: output differs"
        for name, a, b in zip("qkv", grads_static, grads_ref):
            assert torch.equal(a, b), f"replay {rep}: d{name} differs"
