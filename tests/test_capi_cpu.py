"""CPU tests of the C ABI (include/sigattn.h, libsigattn.so): symbols, struct
layout, validation and error codes.  No kernel is launched: every call here
returns before any HIP call."""

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest
import torch

from triton_sigmoid import _capi

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "sigattn.h"

pytestmark = pytest.mark.skipif(not _capi.LIB_PATH.exists(), reason="libsigattn.so not built")


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sigattn_\w+)\s*\(", text)))


def _problem(**kw):
    p = _capi.SigattnProblem()
    p.abi_version = _capi.ABI_VERSION
    p.dtype = _capi.BF16
    p.B, p.Tq, p.Tk, p.H, p.D = 2, 16, 16, 2, 64
    p.q_stride_b, p.q_stride_t, p.q_stride_h = 16 * 2 * 64, 2 * 64, 64
    p.k_stride_b, p.k_stride_t, p.k_stride_h = 16 * 2 * 64, 2 * 64, 64
    fake = 1 << 20  # never dereferenced: validation fails or the problem is empty
    p.q = p.k = p.v = fake
    p.bias = p.scale = fake
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_capi.LIB_PATH))
    declared = _declared_functions()
    assert declared == sorted(_capi.SIGNATURES), declared
    for name in declared:
        assert hasattr(lib, name), name


def test_autograd_node_loads_and_binds_to_the_library():
    """The C++ autograd node imports next to the library, binds to the
    library's entry points (every name it asks for is a declared one) and
    exposes attention(); calling it needs a GPU."""
    import importlib

    mod = importlib.import_module("triton_sigmoid._sigattn_autograd")
    assert set(_capi._AUTOGRAD_FNS) <= set(_capi.SIGNATURES)
    assert hasattr(mod, "attention") and hasattr(mod, "bind")
    with pytest.raises(RuntimeError, match="missing sigattn_fwd_ws"):
        mod.bind({"sigattn_strerror": 1, "sigattn_fwd_workspace_bytes": 1}, [128], 512)
    node = _capi.autograd_node()
    assert node is mod


def test_eager_binding_env_selects_the_python_node(monkeypatch):
    monkeypatch.setenv("SIGATTN_EAGER_BINDING", "python")
    assert _capi.autograd_node() is None


def test_abi_version_and_strerror():
    lib = _capi.load_library()
    assert lib.sigattn_abi_version() == _capi.ABI_VERSION
    assert lib.sigattn_strerror(0) == b"success"
    for code in range(-11, 0):
        assert lib.sigattn_strerror(code) not in (b"", b"unknown sigattn status")
    assert lib.sigattn_strerror(-99) == b"unknown sigattn status"


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_struct_layout_matches_header(tmp_path):
    fields = [f[0] for f in _capi.SigattnProblem._fields_]
    src = tmp_path / "layout.c"
    body = "\n".join(f'  printf("{f} %zu\\n", offsetof(sigattn_problem, {f}));' for f in fields)
    src.write_text(
        "#include <stddef.h>\n#include <stdio.h>\n#include \"sigattn.h\"\n"
        "int main(void) {\n" + body + '\n  printf("sizeof %zu\\n", sizeof(sigattn_problem));\n  return 0;\n}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-I", str(HEADER.parent), str(src), "-o", str(exe)], check=True)
    out = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                       check=True).stdout.splitlines())
    for f in fields:
        assert int(out[f]) == getattr(_capi.SigattnProblem, f).offset, f
    assert int(out["sizeof"]) == ctypes.sizeof(_capi.SigattnProblem)


@pytest.mark.parametrize("change,code", [
    (dict(abi_version=99), -7),
    (dict(dtype=7), -2),
    (dict(D=48), -3),
    (dict(D=256), -3),
    (dict(B=-1), -4),
    (dict(Tq=1 << 40), -4),
    (dict(k_stride_t=-5), -5),
    (dict(Tk=8), -6),           # dense (no seq_lens) requires Tq == Tk
    (dict(rows_q=-1, cu_seqlens_q=1 << 20), -4),
    (dict(cu_seqlens_q=1 << 20, seq_lens_q=1 << 20), -9),   # one layout per axis
    (dict(cu_seqlens_k=1 << 20, seq_lens_k=1 << 20), -9),
    (dict(bias=None), -1),
    (dict(scale=None), -1),
    (dict(q=None), -1),
    (dict(v=None), -1),
])
def test_validation_error_codes(change, code):
    lib = _capi.load_library()
    p = _problem(**change)
    assert lib.sigattn_check(ctypes.byref(p)) == code
    assert lib.sigattn_fwd(ctypes.byref(p), 1 << 20, None) == code
    assert lib.sigattn_fwd_noalloc(ctypes.byref(p), 1 << 20, None) == code
    assert lib.sigattn_bwd(ctypes.byref(p), 1 << 20, 1 << 20, 1 << 20, 1 << 20, None) == code


def test_null_problem_and_null_outputs():
    lib = _capi.load_library()
    assert lib.sigattn_check(None) == -1
    assert lib.sigattn_fwd(None, 1 << 20, None) == -1
    p = _problem()
    assert lib.sigattn_check(ctypes.byref(p)) == 0
    assert lib.sigattn_fwd(ctypes.byref(p), None, None) == -1
    assert lib.sigattn_fwd_noalloc(ctypes.byref(p), None, None) == -1
    assert lib.sigattn_bwd(ctypes.byref(p), 1 << 20, None, 1 << 20, 1 << 20, None) == -1
    assert lib.sigattn_bwd(ctypes.byref(p), None, 1 << 20, 1 << 20, 1 << 20, None) == -1
    assert lib.sigattn_bwd_dq(ctypes.byref(p), 1 << 20, None, None) == -1
    assert lib.sigattn_bwd_dkdv(ctypes.byref(p), 1 << 20, 1 << 20, None, None) == -1


def test_cross_attention_allowed_with_seq_lens():
    lib = _capi.load_library()
    p = _problem(Tk=8, seq_lens_k=1 << 20, seq_lens_q=1 << 20)
    assert lib.sigattn_check(ctypes.byref(p)) == 0


def test_packed_layout_allows_different_lengths():
    lib = _capi.load_library()
    p = _problem(Tk=8, cu_seqlens_q=1 << 20, cu_seqlens_k=1 << 20, rows_q=40, rows_k=20)
    assert lib.sigattn_check(ctypes.byref(p)) == 0
    p = _problem(Tk=8, cu_seqlens_q=1 << 20, seq_lens_k=1 << 20, rows_q=40)
    assert lib.sigattn_check(ctypes.byref(p)) == 0


def test_decode_workspace_size_and_errors():
    """Split-KV forward (Tq <= 32, Tk >= 256, non-causal, MFMA dtypes): the
    workspace size follows the plan, and a short or misaligned workspace is
    rejected before any launch."""
    lib = _capi.load_library()
    D = 128
    p = _problem(B=1, H=1, Tq=1, Tk=4096, D=D, seq_lens_q=1 << 20, seq_lens_k=1 << 20,
                 q_stride_b=D, q_stride_t=D, q_stride_h=D, k_stride_b=4096 * D, k_stride_t=D, k_stride_h=D)
    # 1 (batch, head) pair -> 16 chunks of 256 keys; fp32 partials [16, 1, 1, 1, D]
    assert lib.sigattn_fwd_workspace_bytes(ctypes.byref(p)) == 16 * D * 4
    assert lib.sigattn_fwd_ws(ctypes.byref(p), 1 << 20, 1 << 20, 16 * D * 4 - 1, None) == -10
    assert lib.sigattn_fwd_ws(ctypes.byref(p), 1 << 20, (1 << 20) + 4, 16 * D * 4, None) == -10
    # No split: causal, Tq > 32, Tk < 256, fp32 -> no workspace.
    for change in (dict(causal=1), dict(Tq=33), dict(Tk=255), dict(dtype=_capi.F32)):
        q = _problem(B=1, H=1, Tq=1, Tk=4096, D=D, seq_lens_q=1 << 20, seq_lens_k=1 << 20)
        for k, v in change.items():
            setattr(q, k, v)
        assert lib.sigattn_fwd_workspace_bytes(ctypes.byref(q)) == 0, change
    # More (batch, head) pairs -> fewer chunks (about 512 workgroups in all);
    # from 512 pairs on nothing is split; invalid problems -> 0.
    p.B, p.H = 8, 32
    assert lib.sigattn_fwd_workspace_bytes(ctypes.byref(p)) == 2 * 8 * 32 * D * 4
    p.B = 16
    assert lib.sigattn_fwd_workspace_bytes(ctypes.byref(p)) == 0
    p.D = 48
    assert lib.sigattn_fwd_workspace_bytes(ctypes.byref(p)) == 0


def test_two_pass_backward_workspace_size_and_errors():
    """Two-pass backward: 2 KB per 32x32 (query, key) block per batch and
    head, causal problems keeping the lower triangle only; 0 for problems the
    two-pass kernels do not take (fp32, head_dim other than 64 or 128,
    misaligned strides, empty grids).  Bad workspaces are rejected before any
    launch."""
    lib = _capi.load_library()
    D, T = 128, 100  # 4 blocks of 32 rows per axis
    p = _problem(B=3, H=5, Tq=T, Tk=T, D=D, q_stride_b=T * 5 * D, q_stride_t=5 * D, q_stride_h=D,
                 k_stride_b=T * 5 * D, k_stride_t=5 * D, k_stride_h=D)
    assert lib.sigattn_bwd_workspace_bytes(ctypes.byref(p)) == 3 * 5 * 16 * 2048
    p.causal = 1
    assert lib.sigattn_bwd_workspace_bytes(ctypes.byref(p)) == 3 * 5 * 10 * 2048
    p.causal = 0
    p.Tk, p.seq_lens_k, p.seq_lens_q = 33, 1 << 20, 1 << 20  # cross: 4 x 2 blocks
    assert lib.sigattn_bwd_workspace_bytes(ctypes.byref(p)) == 3 * 5 * 8 * 2048
    for change in (dict(dtype=_capi.F32), dict(D=32), dict(q_stride_t=5 * D + 4), dict(Tq=0), dict(B=0),
                   dict(D=48)):
        q = _problem(B=3, H=5, Tq=T, Tk=T, D=D, q_stride_b=T * 5 * D, q_stride_t=5 * D, q_stride_h=D,
                     k_stride_b=T * 5 * D, k_stride_t=5 * D, k_stride_h=D)
        for k, v in change.items():
            setattr(q, k, v)
        assert lib.sigattn_bwd_workspace_bytes(ctypes.byref(q)) == 0, change
    fake, nbytes = 1 << 20, 3 * 5 * 16 * 2048
    p = _problem(B=3, H=5, Tq=T, Tk=T, D=D, q_stride_b=T * 5 * D, q_stride_t=5 * D, q_stride_h=D,
                 k_stride_b=T * 5 * D, k_stride_t=5 * D, k_stride_h=D)
    # misaligned workspace
    assert lib.sigattn_bwd_ws(ctypes.byref(p), fake, fake, fake, fake, fake + 8, nbytes, None) == -10
    # the halves need the whole problem's workspace, and a workspace at all
    assert lib.sigattn_bwd_dkdv_ws(ctypes.byref(p), fake, fake, fake, fake, nbytes - 1, None) == -10
    assert lib.sigattn_bwd_dq_ws(ctypes.byref(p), fake, fake, nbytes - 2048, None) == -10
    assert lib.sigattn_bwd_dq_ws(ctypes.byref(p), fake, None, nbytes, None) == -10
    assert lib.sigattn_bwd_dkdv_ws(ctypes.byref(p), fake, fake, fake, None, nbytes, None) == -10
    # ... and a problem the two-pass kernels take (fp32 has none)
    p.dtype = _capi.F32
    assert lib.sigattn_bwd_dq_ws(ctypes.byref(p), fake, fake, nbytes, None) == -10
    p.dtype = _capi.BF16
    # null outputs are still reported first
    assert lib.sigattn_bwd_ws(ctypes.byref(p), fake, None, fake, fake, fake, nbytes, None) == -1
    assert lib.sigattn_bwd_dkdv_ws(ctypes.byref(p), None, fake, fake, fake, nbytes, None) == -1


def test_python_layer_backward_workspace_policy(monkeypatch):
    """The Python layer passes the whole dS when it fits the limit, else the
    largest whole number of heads, and no workspace (the recompute backward)
    at D != 128 or when one group's dQ-from-dS grid, in workgroups of 256
    query rows, would have fewer workgroups than the GPU has compute units."""
    lib = _capi.load_library()
    dev = torch.device("cuda", 0)
    monkeypatch.setitem(_capi._CU_COUNT, 0, 256)
    B, H, D, T = 2, 16, 128, 8192
    p = _problem(B=B, H=H, Tq=T, Tk=T, D=D, q_stride_b=T * H * D, q_stride_t=H * D, q_stride_h=D,
                 k_stride_b=T * H * D, k_stride_t=H * D, k_stride_h=D)
    full = lib.sigattn_bwd_workspace_bytes(ctypes.byref(p))
    per_head = full // H
    assert per_head == B * 256 * 256 * 2048
    monkeypatch.setenv("SIGATTN_BWD_WORKSPACE_MB", str(full >> 20))
    assert _capi.bwd_workspace_bytes(lib, p, dev) == full
    monkeypatch.setenv("SIGATTN_BWD_WORKSPACE_MB", "2303")   # 8 heads of 2 batches
    assert _capi.bwd_workspace_bytes(lib, p, dev) == 8 * per_head
    monkeypatch.setenv("SIGATTN_BWD_WORKSPACE_MB", "1024")   # 4 heads: 256 workgroups of 256 rows
    assert _capi.bwd_workspace_bytes(lib, p, dev) == 4 * per_head
    monkeypatch.setenv("SIGATTN_BWD_WORKSPACE_MB", "1023")   # 3 heads: 192 workgroups
    assert _capi.bwd_workspace_bytes(lib, p, dev) == 0
    monkeypatch.setenv("SIGATTN_BWD_WORKSPACE_MB", "0")
    assert _capi.bwd_workspace_bytes(lib, p, dev) == 0
    monkeypatch.delenv("SIGATTN_BWD_WORKSPACE_MB")
    p.D, p.q_stride_t, p.k_stride_t = 64, H * 64, H * 64
    assert _capi.bwd_workspace_bytes(lib, p, dev) == 0


def test_empty_problems_return_before_any_launch():
    lib = _capi.load_library()
    for change in (dict(B=0), dict(H=0), dict(B=0, q=None, k=None, v=None, bias=None, scale=None)):
        p = _problem(**change)
        assert lib.sigattn_fwd(ctypes.byref(p), None, None) == 0
        assert lib.sigattn_bwd(ctypes.byref(p), None, None, None, None, None) == 0
    p = _problem(Tq=0, Tk=0)
    assert lib.sigattn_fwd(ctypes.byref(p), None, None) == 0


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not available")
@pytest.mark.parametrize("src", ["fwd.hip", "bwd.hip", "decode.hip", "f32.hip", "generic.hip"])
def test_device_code_has_no_packed_fp32_instructions(src):
    """Every HIP source is built with packed-fp32 selection disabled; check the
    gfx950 assembly of each kernel file."""
    from triton_sigmoid import _build
    cmd = [_build.hipcc(), *_build.compile_flags(), "-S", "--cuda-device-only",
           str(_build.CSRC / src), "-o", "-"]
    asm = subprocess.run(cmd, capture_output=True, text=True, check=True).stdout
    assert "v_mfma" in asm or src == "generic.hip"
    if src == "f32.hip":
        assert "v_mfma_f32_32x32x2_f32" in asm
    assert not re.search(r"v_pk_(fma|mul|add)_f32", asm)
    # The range split's arrival counter (split_combine) is an agent-scope
    # acquire-release atomic: in every kernel that counts, the add sits
    # between the release (L2 write-back) and the acquire (L2 invalidate),
    # and the partials move with agent-coherent (sc1) accesses.
    atomics = 0
    for body in re.split(r"\n(?=_Z\w+:)", asm):
        lines = [ln.strip() for ln in body.splitlines()]
        adds = [i for i, ln in enumerate(lines) if ln.startswith("global_atomic_add ")]
        for i in adds:
            atomics += 1
            assert any(ln.startswith("buffer_wbl2 sc1") for ln in lines[max(0, i - 4):i]), "no release before the add"
            assert any(ln.startswith("buffer_inv sc1") for ln in lines[i + 1:i + 5]), "no acquire after the add"
        if adds:
            assert any(ln.startswith("buffer_store_dwordx4") and ln.endswith("sc1") for ln in lines)
            assert any(ln.startswith("buffer_load_dwordx4") and ln.endswith("sc1") for ln in lines)
    assert (atomics > 0) == (src in ("fwd.hip", "bwd.hip"))


def test_backward_workspace_oom_falls_back_to_recompute(monkeypatch):
    """An out-of-memory error while allocating the two-pass dS workspace
    gives no workspace (the recompute backward runs) instead of failing."""
    def no_memory(*a, **k):
        raise torch.OutOfMemoryError("forced: no device memory for the workspace")
    assert _capi._bwd_workspace(0, torch.device("cpu")) == (None, 0)
    ws, n = _capi._bwd_workspace(64, torch.device("cpu"))
    assert n == 64 and ws.numel() == 64
    monkeypatch.setattr(_capi.torch, "empty", no_memory)
    assert _capi._bwd_workspace(1 << 30, torch.device("cpu")) == (None, 0)


def test_device_constants_are_never_freed(monkeypatch):
    """Cached constants stay alive for the process (a kernel queued on any
    stream may still read one); past the cap, calls get uncached tensors."""
    made = []
    monkeypatch.setattr(_capi, "_CONSTANTS", {})
    monkeypatch.setattr(_capi, "_CONSTANTS_MAX", 3)
    monkeypatch.setattr(torch._C, "_cuda_isCurrentStreamCapturing", lambda: False)
    monkeypatch.setattr(torch._C, "_cuda_getDevice", lambda: 0)

    class _T:
        def __init__(self, v):
            self.v = v

        def to(self, dev):
            made.append(self)
            return self

    real_full = torch.full
    monkeypatch.setattr(_capi.torch, "full",
                        lambda shape, value, dtype=None, device=None: _T(value) if device is None
                        else real_full(shape, value, dtype=dtype))
    first = [_capi.device_constant((2,), float(i), torch.float32, "cuda:0") for i in range(3)]
    assert len(made) == 3 and len(_capi._CONSTANTS) == 3
    again = [_capi.device_constant((2,), float(i), torch.float32, "cuda:0") for i in range(3)]
    assert all(a is b for a, b in zip(first, again))
    extra = _capi.device_constant((2,), 9.0, torch.float32, "cuda:0")
    assert isinstance(extra, torch.Tensor) and len(_capi._CONSTANTS) == 3
    assert all(_capi._CONSTANTS[((2,), float(i), torch.float32, torch.device("cuda", 0))] is first[i]
               for i in range(3))
