import os
import sys
from fractions import Fraction

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "kestrel-llm_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

# The reference harness reads these once (function-local statics) on first use: the int8
# activation track of the MoE (VLLM_ACTQ=1, s16 track off) is the one the GPU path restates.
os.environ.setdefault("VLLM_ACTQ", "1")
os.environ.setdefault("VLLM_ACTQ16", "0")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run on the MI355X box)")
    config.addinivalue_line("markers", "slow: full-size case")


@pytest.fixture(scope="session")
def orc():
    import oracle
    return oracle


@pytest.fixture(scope="session")
def ref(orc):
    if not orc.ref_available():
        pytest.skip("reference harness oracle/_ref/libkref.so not built (needs /root/reference)")
    return orc.ref()


@pytest.fixture(scope="session")
def kq4():
    """libkq4 on the GPU; a GPU test must fail (not skip) if the library or device is missing."""
    import kq4 as k
    k.init(0)
    return k


@pytest.fixture(scope="session")
def kq4_cpu():
    """libkq4 loaded without a device: only calls that touch no GPU (sizes, exports)."""
    import kq4 as k
    k.lib()
    return k


@pytest.fixture(scope="session")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU test needs a ROCm device"
    return torch


def rel_err(got, ref):
    """max|got-ref| / max|ref| (the reference's own verify metric, vllm_safetensors.c:1177-1181)
    and max-abs."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.abs(got - ref).max() if ref.size else 0.0
    m = np.abs(ref).max() if ref.size else 0.0
    return (d / m if m > 0 else d), d


def rn32(q):
    """A rational rounded to binary32, nearest with ties to even (the one rounding of an
    IEEE-754 single-precision instruction)."""
    f = np.float32(float(q))
    c = [f, np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(-np.inf))]
    return min(c, key=lambda v: (abs(Fraction(float(v)) - q),
                                 int(np.array(v, np.float32).view(np.uint32)) & 1))
