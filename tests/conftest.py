import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels through the C ABI")


@pytest.fixture(scope="session")
def ctx():
    """An open C-ABI context on cuda:0 (gpu tests only)."""
    import torch  # noqa: F401  (initialises the HIP runtime for tensor allocation)
    import dyninfer_amd as d

    c = d.Context(0)
    yield c
    c.close()


def _graph_node_types(g):
    """Node types (hipGraphNodeType: 0 kernel, 10 memory allocation, 11 memory
    free, ...) of a captured torch.cuda.CUDAGraph(keep_graph=True), read
    through the process's one HIP runtime (the one torch loaded)."""
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so.7")
    graph = ctypes.c_void_p(g.raw_cuda_graph())
    n = ctypes.c_size_t(0)
    assert hip.hipGraphGetNodes(graph, None, ctypes.byref(n)) == 0
    nodes = (ctypes.c_void_p * n.value)()
    assert hip.hipGraphGetNodes(graph, nodes, ctypes.byref(n)) == 0
    types = []
    for i in range(n.value):
        t = ctypes.c_int(-1)
        assert hip.hipGraphNodeGetType(ctypes.c_void_p(nodes[i]), ctypes.byref(t)) == 0
        types.append(t.value)
    return types


@pytest.fixture
def graph_node_types():
    return _graph_node_types
