"""GPU tests of the range split of small dense non-causal grids: when a
problem's (batch, head, row block) items leave at least half of the GPU's
compute units idle, the forward and dQ kernels split each item's key range,
and the dK/dV kernel each item's query range, into two to four chunks of at
least 512 rows, one workgroup each, when the split saves at least 1024 rows
of an item's range at head_dim 64 (512 at head_dim 128); the
last workgroup of an item to finish adds the partials in chunk order and
stores the result (sigattn_fwd_ws / sigattn_bwd_split).  The reference runs
one program per row block, streaming every key, whatever the grid size
(src/triton_sigmoid/sigmoid_triton_dense.py:108-118 and grid :534; backward
:162-307); the results
must match the float64 oracle like the unsplit kernels' and equal them within
fp32 summation order, and repeated calls must be bitwise equal.

Every workspace here starts filled with 0xFF bytes: the counters must be
cleared by the call itself, and a partial read before it was stored would be
NaN."""

import ctypes
import math

import numpy as np
import pytest
import torch

from helpers import ULP, assert_close_to_oracle, oracle_fwd_bwd, randn
from triton_sigmoid import _capi

pytestmark = pytest.mark.gpu
DEV = "cuda"


ERR_WORKSPACE = -10  # SIGATTN_ERR_WORKSPACE


def _case(B, T, H, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return [randn((B, T, H, D), dtype, DEV, g) for _ in range(4)]


def _scalars(B, T, D):
    bias = torch.full((B,), -math.log(T), dtype=torch.float32, device=DEV)
    scale = torch.full((), 1.0 / math.sqrt(D), dtype=torch.float32, device=DEV)
    return bias, scale


def _nan_workspace(nbytes):
    return torch.full((max(nbytes, 16),), 0xFF, dtype=torch.uint8, device=DEV)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _fwd(pr, out, ws=None, nbytes=0):
    lib = _capi.load_library()
    rc = lib.sigattn_fwd_ws(ctypes.byref(pr), out.data_ptr(), None if ws is None else ws.data_ptr(), nbytes,
                            _stream())
    assert rc == 0, _capi.strerror(rc)
    torch.cuda.synchronize()


def _bwd_split(pr, do, dq, dk, dv, ws=None, nbytes=0):
    lib = _capi.load_library()
    rc = lib.sigattn_bwd_split(ctypes.byref(pr), do.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                               None if ws is None else ws.data_ptr(), nbytes, _stream())
    assert rc == 0, _capi.strerror(rc)
    torch.cuda.synchronize()


def _assert_fp32_order(got, ref, dtype, name):
    """Same inputs and kernels; only the fp32 summation order differs: a few
    units in the last place of the largest value."""
    assert torch.isfinite(got).all(), f"{name}: non-finite values (a partial was read before it was stored)"
    err = (got.float() - ref.float()).abs().max().item()
    bound = 2 * ULP[dtype] * ref.float().abs().max().item() + 1e-6
    assert err <= bound, f"{name} split vs unsplit: {err:.3e} > {bound:.3e}"


# (B, T, H, D): every shape splits on a 256-CU device (dense problems have
# Tq = Tk), in two chunks (T = 1024 at D = 128), three (T = 1536, 1700) or
# four (T = 2100).  T = 1700 and 2100 leave a ragged last key tile in the
# last chunk and a ragged last row block.
FWD_SHAPES = [(1, 1536, 2, 64), (2, 1700, 2, 64), (1, 2100, 2, 64), (1, 1024, 2, 128), (1, 1700, 1, 128)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", FWD_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_forward_split_matches_oracle_and_unsplit(shape, dtype):
    B, T, H, D = shape
    print(f"forward split {shape} {dtype}", flush=True)
    q, k, v, do = _case(B, T, H, D, dtype, seed=T + D)
    bias, scale = _scalars(B, T, D)
    pr = _capi._problem(q, k, v, bias, None, scale, None, None, False)
    lib = _capi.load_library()
    nbytes = int(lib.sigattn_fwd_workspace_bytes(ctypes.byref(pr)))
    assert nbytes > 0, "this shape should take the range split"
    ref, got = torch.empty_like(q), torch.empty_like(q)
    _fwd(pr, ref)
    _fwd(pr, got, _nan_workspace(nbytes), nbytes)
    _assert_fp32_order(got, ref, dtype, "O")
    want, _ = oracle_fwd_bwd(q, k, v, do, scale=np.float32(1 / math.sqrt(D)), bias=bias.double().cpu().numpy(),
                             with_bwd=False)
    assert_close_to_oracle(got, want, dtype, "O")


def test_forward_split_with_score_mod():
    """score_mod is indexed by the absolute key: each chunk offsets it by its
    first key."""
    B, T, H, D, dtype = 2, 1536, 2, 64, torch.bfloat16
    q, k, v, do = _case(B, T, H, D, dtype, seed=5)
    g = torch.Generator().manual_seed(6)
    sm = randn((B, T), torch.float32, DEV, g, std=2.0)
    bias, scale = _scalars(B, T, D)
    pr = _capi._problem(q, k, v, bias, sm, scale, None, None, False)
    lib = _capi.load_library()
    nbytes = int(lib.sigattn_fwd_workspace_bytes(ctypes.byref(pr)))
    assert nbytes > 0
    ref, got = torch.empty_like(q), torch.empty_like(q)
    _fwd(pr, ref)
    _fwd(pr, got, _nan_workspace(nbytes), nbytes)
    _assert_fp32_order(got, ref, dtype, "O")
    want, _ = oracle_fwd_bwd(q, k, v, do, scale=np.float32(1 / math.sqrt(D)), bias=bias.double().cpu().numpy(),
                             score_mod=sm, with_bwd=False)
    assert_close_to_oracle(got, want, dtype, "O")


def test_forward_split_repeats_bitwise_and_reuses_its_workspace():
    """Two calls on one workspace give the same bits (the counters are
    cleared by each call); a smaller problem on the same workspace after
    them is still right."""
    dtype = torch.float16
    lib = _capi.load_library()
    q, k, v, do = _case(1, 2048, 4, 64, dtype, seed=11)
    bias, scale = _scalars(1, 2048, 64)
    pr = _capi._problem(q, k, v, bias, None, scale, None, None, False)
    nbytes = int(lib.sigattn_fwd_workspace_bytes(ctypes.byref(pr)))
    assert nbytes > 0
    ws = _nan_workspace(nbytes)
    a, b = torch.empty_like(q), torch.empty_like(q)
    _fwd(pr, a, ws, nbytes)
    _fwd(pr, b, ws, nbytes)
    assert torch.equal(a, b)
    q2, k2, v2, do2 = _case(1, 1700, 2, 64, dtype, seed=12)
    bias2, scale2 = _scalars(1, 1700, 64)
    pr2 = _capi._problem(q2, k2, v2, bias2, None, scale2, None, None, False)
    n2 = int(lib.sigattn_fwd_workspace_bytes(ctypes.byref(pr2)))
    assert 0 < n2 <= nbytes
    ref, got = torch.empty_like(q2), torch.empty_like(q2)
    _fwd(pr2, ref)
    _fwd(pr2, got, ws, n2)
    _assert_fp32_order(got, ref, dtype, "O (second problem)")


# (B, T, H, D): at D = 64 the dQ and dK/dV kernels split, at D = 128 the dQ
# kernel (the dK/dV kernel runs one key block per workgroup).
BWD_SHAPES = [(1, 1536, 2, 64), (2, 1700, 2, 64), (1, 1700, 1, 64), (1, 2100, 1, 64), (1, 1100, 2, 128),
              (1, 2100, 1, 128)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", BWD_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_backward_split_matches_oracle_and_unsplit(shape, dtype):
    B, T, H, D = shape
    print(f"backward split {shape} {dtype}", flush=True)
    q, k, v, do = _case(B, T, H, D, dtype, seed=3 * T + H + D)
    bias, scale = _scalars(B, T, D)
    pr = _capi._problem(q, k, v, bias, None, scale, None, None, False)
    lib = _capi.load_library()
    nbytes = int(lib.sigattn_bwd_split_workspace_bytes(ctypes.byref(pr)))
    assert nbytes > 0, "this shape should take the range split"
    ref = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(k)]
    got = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(k)]
    _bwd_split(pr, do, *ref)  # no workspace: the unsplit recompute backward
    _bwd_split(pr, do, *got, ws=_nan_workspace(nbytes), nbytes=nbytes)
    for name, a, b in zip(("dQ", "dK", "dV"), got, ref):
        _assert_fp32_order(a, b, dtype, name)
    _, grads = oracle_fwd_bwd(q, k, v, do, scale=np.float32(1 / math.sqrt(D)), bias=bias.double().cpu().numpy())
    for name, a, want in zip(("dQ", "dK", "dV"), got, grads):
        assert_close_to_oracle(a, want, dtype, name)


def test_backward_split_repeats_bitwise_with_score_mod():
    B, T, H, D, dtype = 2, 1536, 2, 64, torch.float16
    q, k, v, do = _case(B, T, H, D, dtype, seed=21)
    g = torch.Generator().manual_seed(22)
    sm = randn((B, T), torch.float32, DEV, g, std=2.0)
    bias, scale = _scalars(B, T, D)
    pr = _capi._problem(q, k, v, bias, sm, scale, None, None, False)
    lib = _capi.load_library()
    nbytes = int(lib.sigattn_bwd_split_workspace_bytes(ctypes.byref(pr)))
    assert nbytes > 0
    ws = _nan_workspace(nbytes)
    runs = []
    for _ in range(2):
        out = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(k)]
        _bwd_split(pr, do, *out, ws=ws, nbytes=nbytes)
        runs.append(out)
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    _, grads = oracle_fwd_bwd(q, k, v, do, scale=np.float32(1 / math.sqrt(D)), bias=bias.double().cpu().numpy(),
                              score_mod=sm)
    for name, a, want in zip(("dQ", "dK", "dV"), runs[0], grads):
        assert_close_to_oracle(a, want, dtype, name)


def test_split_at_the_item_count_boundary():
    """128 items (8 heads x 16 row blocks of 2048 keys) are exactly half of
    a 256-CU device's CUs: the forward and both backward kernels split in
    two.  Checked against the unsplit kernels."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("item-count boundaries are stated for a 256-CU device")
    dtype = torch.float16
    q, k, v, do = _case(1, 2048, 8, 64, dtype, seed=71)
    bias, scale = _scalars(1, 2048, 64)
    pr = _capi._problem(q, k, v, bias, None, scale, None, None, False)
    lib = _capi.load_library()
    fb = int(lib.sigattn_fwd_workspace_bytes(ctypes.byref(pr)))
    bb = int(lib.sigattn_bwd_split_workspace_bytes(ctypes.byref(pr)))
    assert fb == 512 + 128 * 2 * 128 * 64 * 4
    assert bb == (512 + 128 * 2 * 128 * 64 * 4) + (512 + 128 * 2 * 2 * 128 * 64 * 4)
    ref, got = torch.empty_like(q), torch.empty_like(q)
    _fwd(pr, ref)
    _fwd(pr, got, _nan_workspace(fb), fb)
    _assert_fp32_order(got, ref, dtype, "O")
    ref = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(k)]
    got = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(k)]
    _bwd_split(pr, do, *ref)
    _bwd_split(pr, do, *got, ws=_nan_workspace(bb), nbytes=bb)
    for name, a, b in zip(("dQ", "dK", "dV"), got, ref):
        _assert_fp32_order(a, b, dtype, name)


def test_backward_split_halves_equal_the_whole():
    """dQ alone (dk, dv NULL) and dK/dV alone (dq NULL) on the same workspace
    give the whole call's bits."""
    q, k, v, do = _case(2, 1700, 2, 64, torch.bfloat16, seed=61)
    bias, scale = _scalars(2, 1700, 64)
    pr = _capi._problem(q, k, v, bias, None, scale, None, None, False)
    lib = _capi.load_library()
    nbytes = int(lib.sigattn_bwd_split_workspace_bytes(ctypes.byref(pr)))
    assert nbytes > 0
    ws = _nan_workspace(nbytes)
    whole = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(k)]
    _bwd_split(pr, do, *whole, ws=ws, nbytes=nbytes)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(k)
    for args in ((dq.data_ptr(), None, None), (None, dk.data_ptr(), dv.data_ptr())):
        rc = lib.sigattn_bwd_split(ctypes.byref(pr), do.data_ptr(), *args, ws.data_ptr(), nbytes, _stream())
        assert rc == 0, _capi.strerror(rc)
    torch.cuda.synchronize()
    for name, a, b in zip(("dQ", "dK", "dV"), (dq, dk, dv), whole):
        assert torch.equal(a, b), f"{name}: half call differs from the whole"


def _random_split_cases(n=12, seed=2024):
    """Seeded shapes that split (B*H*row blocks within half of 256 CUs,
    T >= 2048 at D = 64 and T >= 1024 at D = 128, so two chunks save enough
    rows), across head dims, dtypes and score_mod."""
    import random
    rng = random.Random(seed)
    cases = []
    while len(cases) < n:
        D = rng.choice([64, 128])
        T = rng.randrange(2048 if D == 64 else 1024, 3300)
        H = rng.randrange(1, 5)
        B = rng.randrange(1, 3)
        if B * H * -(-T // 128) > 128:  # the backward kernels' 128-row blocks
            continue
        cases.append((B, T, H, D, rng.choice([torch.float16, torch.bfloat16]), rng.random() < 0.5))
    return cases


@pytest.mark.parametrize("case", _random_split_cases(), ids=lambda c: "B{}T{}H{}D{}{}{}".format(
    c[0], c[1], c[2], c[3], str(c[4])[6:], "sm" if c[5] else ""))
def test_random_split_shapes_equal_unsplit(case):
    """Forward and backward through the split kernels equal the unsplit
    ones within fp32 summation order on seeded random shapes (ragged last
    tiles and row blocks, 2-4 chunks)."""
    B, T, H, D, dtype, with_sm = case
    print(f"random split case {case}", flush=True)
    q, k, v, do = _case(B, T, H, D, dtype, seed=T * 7 + H)
    sm = randn((B, T), torch.float32, DEV, torch.Generator().manual_seed(T), std=2.0) if with_sm else None
    bias, scale = _scalars(B, T, D)
    pr = _capi._problem(q, k, v, bias, sm, scale, None, None, False)
    lib = _capi.load_library()
    fb = int(lib.sigattn_fwd_workspace_bytes(ctypes.byref(pr)))
    bb = int(lib.sigattn_bwd_split_workspace_bytes(ctypes.byref(pr)))
    assert fb > 0 and bb > 0, "this shape should take the range split"
    ref, got = torch.empty_like(q), torch.empty_like(q)
    _fwd(pr, ref)
    _fwd(pr, got, _nan_workspace(fb), fb)
    _assert_fp32_order(got, ref, dtype, "O")
    ref = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(k)]
    got = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(k)]
    _bwd_split(pr, do, *ref)
    _bwd_split(pr, do, *got, ws=_nan_workspace(bb), nbytes=bb)
    for name, a, b in zip(("dQ", "dK", "dV"), got, ref):
        _assert_fp32_order(a, b, dtype, name)


def test_workspace_too_small():
    """sigattn_fwd_ws with a workspace too small for the range split's
    partials (say, one sized for split-KV decode), or misaligned, runs the
    problem unsplit: the result equals sigattn_fwd's bit for bit.
    sigattn_bwd_split, which asks for the split explicitly, rejects it."""
    q, k, v, do = _case(1, 1536, 2, 64, torch.float16, seed=31)
    bias, scale = _scalars(1, 1536, 64)
    pr = _capi._problem(q, k, v, bias, None, scale, None, None, False)
    lib = _capi.load_library()
    fb = int(lib.sigattn_fwd_workspace_bytes(ctypes.byref(pr)))
    bb = int(lib.sigattn_bwd_split_workspace_bytes(ctypes.byref(pr)))
    assert fb > 0 and bb > 0, "this shape should take the range split"
    ws = _nan_workspace(max(fb, bb) + 16)
    ref = torch.empty_like(q)
    assert lib.sigattn_fwd(ctypes.byref(pr), ref.data_ptr(), _stream()) == 0
    for ptr, nbytes in ((ws.data_ptr(), fb - 1), (ws.data_ptr() + 8, fb)):
        o = torch.full_like(q, float("nan"))
        assert lib.sigattn_fwd_ws(ctypes.byref(pr), o.data_ptr(), ptr, nbytes, _stream()) == 0
        torch.cuda.synchronize()
        assert torch.equal(o, ref)
    g = [torch.empty_like(t) for t in (q, k, v)]
    assert lib.sigattn_bwd_split(ctypes.byref(pr), do.data_ptr(), *(t.data_ptr() for t in g), ws.data_ptr(),
                                 bb - 1, _stream()) == ERR_WORKSPACE


@pytest.mark.parametrize("shape", [(4, 1024, 8, 64), (1, 2048, 9, 64), (2, 1024, 8, 64), (1, 1400, 4, 64),
                                   (2, 2048, 8, 64, True)],
                         ids=["half-full", "144-items", "c2", "short", "causal"])
def test_grids_that_do_not_split(shape):
    """More than half the CUs' worth of items (256; 144 = 9 heads x 16 row
    blocks) does not split; at head_dim 64 a split must save 1024 rows of an
    item's range, which 1024 keys in two chunks (c2) or
    1400 keys in two do not (and 1400 make no three chunks of 512); causal
    problems never split.  Such problems need no workspace."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("item-count boundaries are stated for a 256-CU device")
    B, T, H, D = shape[:4]
    causal = len(shape) > 4
    q, k, v, do = _case(B, T, H, D, torch.float16, seed=51)
    bias, scale = _scalars(B, T, D)
    pr = _capi._problem(q, k, v, bias, None, scale, None, None, causal)
    lib = _capi.load_library()
    assert int(lib.sigattn_fwd_workspace_bytes(ctypes.byref(pr))) == 0
    assert int(lib.sigattn_bwd_split_workspace_bytes(ctypes.byref(pr))) == 0


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,T,H,split", [(2, 1024, 8, False), (1, 2048, 8, True)], ids=["c2", "split"])
def test_public_api_small_grids(B, T, H, split, dtype):
    """The public API at B=2 L=1024 H=8 D=64 non-causal (
    whose keys are too few for a split to pay) equals the unsplit C-ABI calls
    bit for bit; at B=1 L=2048 H=8 it takes the split and equals the unsplit
    calls within fp32 summation order (the split kernels themselves are
    pinned to the oracle above)."""
    import triton_sigmoid as ts
    D = 64
    q, k, v, do = _case(B, T, H, D, dtype, seed=41)
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
    o = ts.sigmoid_attention(*leaves)
    o.backward(do)
    bias, scale = _scalars(B, T, D)
    pr = _capi._problem(q, k, v, bias, None, scale, None, None, False)
    lib = _capi.load_library()
    assert (int(lib.sigattn_fwd_workspace_bytes(ctypes.byref(pr))) > 0) == split
    assert (int(lib.sigattn_bwd_split_workspace_bytes(ctypes.byref(pr))) > 0) == split
    ref_o = torch.empty_like(q)
    _fwd(pr, ref_o)
    ref = [torch.empty_like(q), torch.empty_like(k), torch.empty_like(k)]
    _bwd_split(pr, do, *ref)
    for name, got, want in zip(("O", "dQ", "dK", "dV"), [o.detach()] + [t.grad for t in leaves], [ref_o] + ref):
        if split:
            _assert_fp32_order(got, want, dtype, name)
        else:
            assert torch.equal(got, want), f"{name}: the unsplit public API differs from the C ABI"
