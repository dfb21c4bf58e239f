"""sigattn_fwd_noalloc: the split-KV forward with its partials in the
library's fixed device scratch instead of a caller workspace.  Checked
against sigattn_fwd_ws (the same kernels with a workspace from torch's
allocator) bit for bit, and against the float64 oracle, on two calls in a
row whose second problem is smaller, plus a problem that does not split."""

import ctypes
import math

import numpy as np
import pytest
import torch

from helpers import assert_close_to_oracle, oracle_fwd_bwd, randn
from triton_sigmoid import _capi

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(B, Tq, Tk, H, D, dtype, seed, lens_k=None):
    g = torch.Generator().manual_seed(seed)
    q = randn((B, Tq, H, D), dtype, DEV, g)
    k = randn((B, Tk, H, D), dtype, DEV, g)
    v = randn((B, Tk, H, D), dtype, DEV, g)
    sk = torch.tensor(lens_k if lens_k is not None else [Tk] * B, dtype=torch.int32, device=DEV)
    sq = torch.full((B,), Tq, dtype=torch.int32, device=DEV)
    bias = -torch.log(sk.float())
    scale = torch.full((), 1.0 / math.sqrt(D), dtype=torch.float32, device=DEV)
    pr = _capi._problem(q, k, v, bias, None, scale, sq, sk, False)
    # The problem holds raw pointers: every tensor it points to stays alive
    # with the returned tuple.
    return q, k, v, sq, sk, bias, scale, pr


def _with_workspace(lib, pr, out):
    nbytes = int(lib.sigattn_fwd_workspace_bytes(ctypes.byref(pr)))
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.sigattn_fwd_ws(ctypes.byref(pr), out.data_ptr(), ws.data_ptr() if nbytes else None, nbytes, stream)
    assert rc == 0, _capi.strerror(rc)
    return nbytes


def test_noalloc_first_call_under_graph_capture():
    """The first sigattn_fwd_noalloc call of the process on this device comes
    while torch.cuda.graph captures (so the scratch address is looked up under
    capture), on a split-KV shape; every replay, with eager work and
    synchronisation between replays and the output overwritten with NaN first,
    equals the eager sigattn_fwd_ws result bit for bit.  It runs first in
    this file, whose tests are the only callers of sigattn_fwd_noalloc."""
    lib = _capi.load_library()
    q, k, v, sq, sk, bias, scale, pr = _case(2, 4, 8192, 8, 128, torch.bfloat16, seed=99, lens_k=[8192, 3000])
    want = torch.empty_like(q)
    assert _with_workspace(lib, pr, want) > 0  # the problem splits
    torch.cuda.synchronize()
    got = torch.full_like(q, float("nan"))
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(graph, stream=side):
        rc = lib.sigattn_fwd_noalloc(ctypes.byref(pr), got.data_ptr(), side.cuda_stream)
    assert rc == 0, _capi.strerror(rc)
    for rep in range(3):
        busy = (q.float() * 2.0).sum()
        got.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(busy)
        assert torch.equal(got, want), f"replay {rep} differs from sigattn_fwd_ws"


def test_noalloc_matches_workspace_entry_point_on_two_calls():
    lib = _capi.load_library()
    stream = torch.cuda.current_stream().cuda_stream
    cases = [
        # (B, Tq, Tk, H, D, dtype, lens_k): the second call is smaller.
        (2, 4, 8192, 8, 128, torch.bfloat16, [8192, 5000]),
        (1, 1, 2048, 4, 64, torch.float16, [1700]),
    ]
    for i, (B, Tq, Tk, H, D, dtype, lens) in enumerate(cases):
        print(f"[no-alloc] call {i}: B={B} Tq={Tq} Tk={Tk} H={H} D={D} {dtype}", flush=True)
        q, k, v, sq, sk, bias, scale, pr = _case(B, Tq, Tk, H, D, dtype, seed=100 + i, lens_k=lens)
        want = torch.empty_like(q)
        nbytes = _with_workspace(lib, pr, want)
        assert 0 < nbytes <= (16 << 20), nbytes  # the problem splits, within the fixed scratch
        got = torch.full_like(q, float("nan"))
        rc = lib.sigattn_fwd_noalloc(ctypes.byref(pr), got.data_ptr(), stream)
        assert rc == 0, _capi.strerror(rc)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {i}: differs from sigattn_fwd_ws"
        o, _ = oracle_fwd_bwd(q, k, v, q, scale=np.float32(1 / math.sqrt(D)), bias=bias.double().cpu().numpy(),
                              seq_lens_q=sq, seq_lens_k=sk, with_bwd=False)
        assert_close_to_oracle(got, o, dtype, f"O (call {i})")


def test_noalloc_runs_range_split_problems_unsplit():
    """A small dense non-causal grid that sigattn_fwd_ws range-splits runs
    unsplit here: sigattn_fwd's bits."""
    lib = _capi.load_library()
    stream = torch.cuda.current_stream().cuda_stream
    g = torch.Generator().manual_seed(9)
    q, k, v = (torch.randn((1, 1536, 2, 64), generator=g).to("cuda", torch.float16) for _ in range(3))
    bias = torch.full((1,), -math.log(1536), dtype=torch.float32, device="cuda")
    scale = torch.full((), 0.125, dtype=torch.float32, device="cuda")
    pr = _capi._problem(q, k, v, bias, None, scale, None, None, False)
    assert lib.sigattn_fwd_workspace_bytes(ctypes.byref(pr)) > 0
    want, got = torch.empty_like(q), torch.empty_like(q)
    assert lib.sigattn_fwd(ctypes.byref(pr), want.data_ptr(), stream) == 0
    assert lib.sigattn_fwd_noalloc(ctypes.byref(pr), got.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_noalloc_runs_unsplit_problems_like_sigattn_fwd():
    lib = _capi.load_library()
    stream = torch.cuda.current_stream().cuda_stream
    q, k, v, sq, sk, bias, scale, pr = _case(2, 200, 200, 2, 128, torch.bfloat16, seed=7)
    assert lib.sigattn_fwd_workspace_bytes(ctypes.byref(pr)) == 0
    want, got = torch.empty_like(q), torch.empty_like(q)
    assert lib.sigattn_fwd(ctypes.byref(pr), want.data_ptr(), stream) == 0
    assert lib.sigattn_fwd_noalloc(ctypes.byref(pr), got.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(got, want)
