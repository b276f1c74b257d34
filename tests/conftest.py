"""Test configuration: package path, the ``gpu`` marker, shared fixtures."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "nano-vllm-practice_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """A GPU device; GPU tests need a visible GPU and the built HIP library."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def ops(gpu):
    """``femtovllm.ops`` on the GPU; raises (fails the test) if the library is missing."""
    import femtovllm.ops

    return femtovllm.ops


@pytest.fixture(params=["split", "one_launch"])
def decode_path(request, gpu):
    """Runs a decode test through both decode routes of the library: the split
    workers + merge kernel, and the one-launch kernel (forced for every
    length through femto_attn_set_decode_single_max_kv)."""
    from femtovllm import _C

    limit = -1 if request.param == "split" else (1 << 30)
    prev = _C._lib.femto_attn_set_decode_single_max_kv(limit)
    yield request.param
    _C._lib.femto_attn_set_decode_single_max_kv(prev)
