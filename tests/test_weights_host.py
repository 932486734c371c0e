"""Host-only checks of the weight buffers' sizes and argument rules (include/kernelcore/weights.h;
reference integrations/llama.cpp/ggml/src/ggml-kernelcore/ggml-kernelcore.cpp:103-118, 259-266):
no GPU -- kcWeightAllocSize touches no device, and every refused set / get returns before one."""
import pytest

import kernelcore_amd as kc

DUMMY = 0x1000


@pytest.mark.parametrize("qtype,rows,k", [("q4k", 8, 256), ("q4k", 3072, 3072), ("q6k", 128256, 3072), ("q6k", 16, 8192)])
def test_kquant_alloc_is_the_stream(qtype, rows, k):
    assert kc.weight_alloc_size(qtype, rows, k) == kc.stream_bytes(qtype, rows, k)
    assert kc.weight_alloc_size(qtype, rows, k) >= rows * (k // 256) * (144 if qtype == "q4k" else 210)


def test_plain_alloc_is_ggml_size():
    assert kc.weight_alloc_size("f32", 3, 1000) == 12000
    assert kc.weight_alloc_size("f16", 24, 130) == 24 * 130 * 2


@pytest.mark.parametrize("qtype,rows,k,why", [
    ("q4k", 12, 256, "rows % 8"), ("q6k", 8, 300, "rows % 8"), ("f16", 8, 7, "even k"),
    (13, 8, 256, "qtype"), ("f32", 0, 4, "positive"),
])
def test_refused_shapes(qtype, rows, k, why):
    with pytest.raises(kc.KcError) as e:
        kc.weight_alloc_size(qtype, rows, k)
    assert e.value.name == "InvalidValue" and why in str(e.value), str(e.value)


@pytest.mark.parametrize("fn", ["kcWeightSetTensor", "kcWeightGetTensor"])
def test_refused_ranges(fn):
    whole = 8 * 144
    for qtype, off, size, why in ((12, 0, whole + 1, "beyond"), (12, whole, 1, "beyond"), (0, 8 * 10 * 4, 1, "beyond")):
        with pytest.raises(kc.KcError) as e:
            kc.call(fn, qtype, 8, 256 if qtype == 12 else 10, DUMMY, DUMMY, off, size, None)
        assert why in str(e.value)
    with pytest.raises(kc.KcError) as e:
        kc.call(fn, 12, 8, 256, None, DUMMY, 0, whole, None)
    assert "null" in str(e.value)
