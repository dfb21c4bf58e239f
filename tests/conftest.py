"""Shared pytest configuration.

* Puts the repository root (for `oracle`) and `triton-sigmoid_amd/` (for the
  `triton_sigmoid` package) on sys.path.
* Registers the `gpu` marker.  GPU tests need a gfx950 device and the built
  libsigattn.so; in a container without a GPU they are skipped with a reason.
* Tolerances follow the reference's conftest (tests/conftest.py:27-34):
  fp32 1e-5, fp16 1e-3, bf16 7e-3, used with N(0, 0.5²) inputs.
"""

import os
import random
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "triton-sigmoid_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

TOLERANCE = {torch.float32: 1e-5, torch.float16: 1e-3, torch.bfloat16: 7e-3}
IO_DTYPE = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}


def get_tolerance(dtype: torch.dtype) -> float:
    return TOLERANCE[dtype]


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libsigattn.so")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment (gpu tests run on the MI355X box)")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def reset_test_state():
    torch.manual_seed(32)
    np.random.seed(32)
    random.seed(32)
    if torch.cuda.is_available():
        torch.cuda.manual_seed_all(32)
    yield


@pytest.fixture(autouse=True)
def _announce(request):
    # GPU steps print their case name first so a fault names its test.
    if "gpu" in request.node.keywords and os.environ.get("SIGATTN_ANNOUNCE", "1") == "1":
        print(f"\n[case] {request.node.nodeid}", flush=True)
    yield
