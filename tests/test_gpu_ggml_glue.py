"""The ggml glue (kernelcore_amd/ggml/src/ggml-kernelcore/ggml-kernelcore.cpp, built against the
test-only ggml stand-in of tests/ggml_stub) on the GPU, driven through its vtables as ggml's scheduler
drives them: the device as llama.cpp reads it, the weights' and KV caches' buffers
(set / get / memset_tensor, clear, device copies; ggml-kernelcore.cpp:158-246), supports_op, and
graph_compute of whole layer graphs -- every ggml tensor turned into a kcGgmlTensor by the glue
itself -- against kcGgmlGraphCompute on the same graphs, bit for bit, the kept graph included."""
import ctypes as C

import numpy as np
import pytest

import kernelcore_amd as kc
from kernelcore_amd import ggml_graph as gg
from tests import glue, kq
from tests.test_gpu_ggml_backend import Layer

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def runtime():
    kc.init()
    yield
    kc.synchronize()


def test_device_as_llama_cpp_reads_it():
    i = glue.info()
    assert (i["reg"], i["name"], glue.DEVICE_TYPES[i["type"]], i["devices"]) == ("Kernelcore", "Kernelcore", "ACCEL", 1)
    assert i["memory_total"] >= 250 << 30 and 0 < i["memory_free"] <= i["memory_total"]
    assert not i["mmap_support"]  # weights are copied into HBM: llama.cpp reads the file instead of mapping it
    assert "gfx950" in i["description"]
    assert glue.buft(0) == dict(name="Kernelcore", alignment=64, is_host=False, supported=True)
    assert glue.buft(1) == dict(name="Kernelcore_Host", alignment=64, is_host=False, supported=True)
    L = glue.lib()
    assert L.kcgt_supports_mul_mat(12, 3072, 3072, 1, 0) == 1  # a Q4_K weight in the weights' buffers
    assert L.kcgt_supports_mul_mat(14, 3072, 8192, 512, 0) == 1
    assert L.kcgt_supports_mul_mat(12, 3072, 3072, 1, -1) == 0  # not in this backend's buffers
    assert L.kcgt_supports_mul_mat(12, 3072, 3072, 1, 1) == 0  # in the KV buffers
    assert L.kcgt_supports_mul_mat(12, 3000, 3072, 1, 0) == 0  # k not a multiple of 256


@pytest.mark.parametrize("kind,type_,ne0,ne1", [(0, 12, 768, 40), (0, 14, 512, 24), (0, 0, 1000, 3), (1, 1, 1024, 40),
                                                 (1, 0, 96, 5)])
def test_buffers_through_the_vtables(kind, type_, ne0, ne1):
    """set_tensor then get_tensor is the identity (K-quant: repacked into the stream and unpacked);
    memset_tensor sets the range of the ggml bytes; cpy_tensor copies on the device (declined for a
    K-quant weight: its stream is not its ggml bytes); clear sets every byte."""
    if type_ in (12, 14):
        data = kq.random_blocks({12: "q4k", 14: "q6k"}[type_], ne1, ne0, seed=ne0 + ne1)
    else:
        data = np.random.default_rng(ne0).integers(0, 256, ne0 * ne1 * (4 if type_ == 0 else 2), dtype=np.uint8)
    n = data.size
    after_set, after_memset, after_clear, after_cpy = (np.zeros(n, np.uint8) for _ in range(4))
    off, size, value = 7, min(500, n - 7), 0x3C
    rc = glue.lib().kcgt_buffer_ops(kind, type_, ne0, ne1, data.ctypes.data, after_set.ctypes.data, value, off, size,
                                    after_memset.ctypes.data, 0xC3, after_clear.ctypes.data, after_cpy.ctypes.data)
    kq_weight = kind == 0 and type_ in (12, 14)
    assert rc == (-2 if kq_weight else 0)
    assert np.array_equal(after_set, data)
    want = data.copy()
    want[off:off + size] = value
    assert np.array_equal(after_memset, want)
    assert np.array_equal(after_clear, np.full(n, 0xC3, np.uint8))
    if not kq_weight:
        assert np.array_equal(after_cpy, data)


def glue_compute(L, repeat):
    g = L.g
    ts = list(g.keep)
    base = [g.view_of[id(t)][0] if id(t) in g.view_of else None for t in ts]
    tensors = (C.c_void_p * len(ts))(*[C.addressof(t) for t in ts])
    bases = (C.c_void_p * len(ts))(*[C.addressof(b) if b is not None else None for b in base])
    nodes = (C.c_void_p * len(g.nodes))(*[C.addressof(t) for t in g.nodes])
    return glue.lib().kcgt_graph_compute(tensors, bases, len(ts), nodes, len(g.nodes), repeat)


CASES = [
    ("decode", gg.LayerShape(), 1, 40, False),
    ("decode, qwen3 q / k norm", gg.LayerShape(n_embd=1024, n_head=8, n_head_kv=2, head_dim=128, neox=True,
                                              qk_norm=True), 1, 70, False),
    ("decode, shared memory", gg.LayerShape(), 1, 40, True),
    ("batch of 8", gg.LayerShape(), 8, 100, False),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_layer_graph_through_the_glue_equals_the_backend_core(case):
    """The glue builds its own descriptors from ggml tensors (ops, types, shapes, strides, op_params,
    flags, use counts from the graph, buffer kinds through view_src) and calls kcGgmlGraphCompute:
    the layer output and both caches equal the core called on ggml_graph.py's descriptors, bit for
    bit; three calls in a row (the kept graph launched again) leave the same result."""
    name, shape, N, p0, share = case
    got = {}
    for via_glue in (True, False):
        L = Layer(shape, N, p0, seed=2100 + N, share=share)
        if via_glue:
            assert glue_compute(L, repeat=1) == 0
        else:
            be = kc.GgmlBackend()
            be.compute(L.g.nodes)
            be.close()
        kc.synchronize()
        got[via_glue] = [L.get("out", np.float32).view(np.uint32), L.get("k_cache", np.uint16),
                         L.get("v_cache", np.uint16)]
        if via_glue:  # the same step again through a kept graph: the same bits (the cache row rewritten)
            assert glue_compute(L, repeat=3) == 0
            kc.synchronize()
            assert np.array_equal(L.get("out", np.float32).view(np.uint32), got[True][0])
        L.free()
    for a, b, what in zip(got[True], got[False], ("out", "k_cache", "v_cache")):
        assert np.array_equal(a, b), what
