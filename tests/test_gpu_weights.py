"""The weight buffers on the GPU (include/kernelcore/weights.h; the reference backend's
buffer_set_tensor / buffer_get_tensor, integrations/llama.cpp/ggml/src/ggml-kernelcore/
ggml-kernelcore.cpp:175-206): a K-quant weight set whole is read back as the same ggml bytes
(get_tensor o set_tensor = identity, any sub-range), and the matvec over the stream it wrote equals
the oracle's over the ggml blocks, bit for bit; f32 / fp16 tensors are plain copies of byte ranges;
a partial K-quant upload is refused as the reference asserts."""
import numpy as np
import pytest

import kernelcore_amd as kc
import oracle
from tests import kq

pytestmark = pytest.mark.gpu
O = oracle.lib()


@pytest.fixture(scope="module", autouse=True)
def runtime():
    kc.init()
    yield
    kc.synchronize()


@pytest.mark.parametrize("qtype,rows,k", [("q4k", 8, 256), ("q4k", 72, 3072), ("q6k", 16, 768), ("q6k", 136, 1024)])
def test_kquant_round_trip_and_matvec(qtype, rows, k):
    blocks = kq.random_blocks(qtype, rows, k, seed=rows + k)
    dst = kc.Buffer(kc.weight_alloc_size(qtype, rows, k))
    kc.weight_set(qtype, rows, k, dst.ptr, blocks)
    assert np.array_equal(kc.weight_get(qtype, rows, k, dst.ptr, 0, blocks.size), blocks)
    bb = 144 if qtype == "q4k" else 210
    for off, size in ((bb, bb), (3, blocks.size - 10), (blocks.size - 1, 1), (0, 0)):
        assert np.array_equal(kc.weight_get(qtype, rows, k, dst.ptr, off, size), blocks[off:off + size])
    x = kq.randn(k, 7)
    xq, xd = oracle.quantize_q8x4(O, x)
    want = np.zeros(rows, np.float32)
    getattr(O, f"kco_matvec_{qtype}_q8")(blocks, xq, xd, want, rows, k)
    bq, bd, by = kc.Buffer.of(xq), kc.Buffer.of(xd), kc.Buffer(rows * 4)
    kc.launch(f"matvec_{qtype}_q8", kc.MatvecQ4Q8Args(dst.ptr, bq.ptr, bd.ptr, by.ptr, None, rows, k))
    assert np.array_equal(kq.bits(by.download(np.float32)), kq.bits(want))
    with pytest.raises(kc.KcError) as e:
        kc.weight_set(qtype, rows, k, dst.ptr, blocks[: blocks.size - bb])
    assert e.value.name == "InvalidValue" and "whole" in str(e.value)
    for b in (dst, bq, bd, by):
        b.free()


@pytest.mark.parametrize("qtype,rows,k", [("f32", 3, 1000), ("f16", 24, 130)])
def test_plain_tensors_copy_byte_ranges(qtype, rows, k):
    n = kc.weight_alloc_size(qtype, rows, k)
    data = np.random.default_rng(3).integers(0, 256, n, dtype=np.uint8)
    dst = kc.Buffer(n)
    kc.weight_set(qtype, rows, k, dst.ptr, data[:100], offset=0)
    kc.weight_set(qtype, rows, k, dst.ptr, data[100:], offset=100)
    assert np.array_equal(kc.weight_get(qtype, rows, k, dst.ptr, 0, n), data)
    assert np.array_equal(kc.weight_get(qtype, rows, k, dst.ptr, 17, 40), data[17:57])
    dst.free()


@pytest.mark.parametrize("qtype,rows,k", [("q4k", 40, 768), ("q6k", 24, 512), ("f32", 3, 1000)])
def test_memset_tensor_sets_the_ggml_bytes_of_a_range(qtype, rows, k):
    """memset_tensor (buffer_memset_tensor, ggml-kernelcore.cpp:171-173) through kcWeightMemsetTensor:
    get_tensor then reads the value over the range and the earlier bytes everywhere else; a whole
    buffer cleared (buffer_clear, :208-211: kcMemset of the allocation) reads the value everywhere,
    also as a K-quant tensor's ggml bytes (the stream holds exactly the ggml bytes, rearranged)."""
    n = kc.weight_alloc_size(qtype, rows, k)
    if qtype in ("q4k", "q6k"):
        data = kq.random_blocks(qtype, rows, k, seed=rows * k)
    else:
        data = np.random.default_rng(9).integers(0, 256, n, dtype=np.uint8)
    dst = kc.Buffer(n)
    kc.weight_set(qtype, rows, k, dst.ptr, data)
    want = data.copy()
    for off, size, value in ((5, 300, 0x5A), (data.size - 7, 7, 0xFF), (0, 1, 0), (100, 0, 0x11)):
        kc.weight_memset(qtype, rows, k, dst.ptr, value, off, size)
        want[off:off + size] = value
        assert np.array_equal(kc.weight_get(qtype, rows, k, dst.ptr, 0, data.size), want), (off, size)
    with pytest.raises(kc.KcError) as e:
        kc.weight_memset(qtype, rows, k, dst.ptr, 1, data.size - 3, 4)
    assert e.value.name == "InvalidValue"
    kc.call("kcMemset", dst.ptr, 0xA5, n)
    assert np.array_equal(kc.weight_get(qtype, rows, k, dst.ptr, 0, data.size), np.full(data.size, 0xA5, np.uint8))
    dst.free()


def test_device_memory_info():
    """get_memory (the reference returns 0 / 0, ggml-kernelcore.cpp:823-826): hipMemGetInfo's free and
    total HBM bytes; an allocation lowers the free bytes by at least its size."""
    free0, total = kc.device_memory()
    assert total >= 250 << 30 and 0 < free0 <= total  # MI355X: 288 GB of HBM3E
    b = kc.Buffer(1 << 30)
    free1, total1 = kc.device_memory()
    assert total1 == total and free1 <= free0 - (1 << 30) + (64 << 20)
    b.free()
