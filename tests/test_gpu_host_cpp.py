"""Runs the GPU C++ host-layer test (tests/cpp/test_gpu_layer.cpp): device
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
