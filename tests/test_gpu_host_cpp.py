"""Runs the GPU C++ host-layer tests (tests/cpp/test_gpu_layer.cpp,
tests/cpp/test_host_layer.cpp): device
block tables, BlockPool device pools, and TransformerBlock::forward_into
against a float64 restatement of the decoder layer with the oracle's
attention over the device pool."""
import pytest

from test_host_cpp import _run

pytestmark = pytest.mark.gpu


def test_cpp_gpu_layer(gpu):
    rc, out = _run("test_gpu_layer", timeout=110)
    print(out)
    assert rc == 0, out


def test_cpp_host_layer_on_device(gpu):
    """tests/cpp/test_host_layer.cpp against the HIP library: DeviceBatch's
    incremental uploads over a random append/free/rebind trace, a failed sync
    losing nothing, device block tables, device pool copies, Sampler draws."""
    rc, out = _run("test_host_layer", timeout=110)
    print(out)
    assert rc == 0, out
    assert "all checks passed" in out and "skipped" not in out, out
