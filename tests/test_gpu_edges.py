"""Edge cases of the by-name kernels on the GPU: empty launches (zero rows or values, accepted by
the reference's validation: llm/llm_kernels.cpp:264-288 in arasheedu/Kernelcore) do nothing and
succeed; the largest k the decode matvec stages (32768, the activation vector in LDS) matches the
oracle bit for bit and one super-block more is refused with InvalidValue; ragged shapes (rows not a
multiple of the 16-row tile, k not a multiple of the 4-super-block group) match the oracle."""
import sys

import numpy as np
import pytest

import kernelcore_amd as kc
import oracle
from tests import kq

pytestmark = pytest.mark.gpu
O = oracle.lib()


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def runtime():
    kc.init()
    yield
    kc.synchronize()


def matvec(qtype, w, x, rows, k):
    nb = k // 32
    stream = kc.upload_weights(qtype, w, rows, k)
    bx, bq, bd, by = kc.Buffer.of(x), kc.Buffer(nb * 32), kc.Buffer(nb * 8), kc.Buffer(max(rows, 8) * 4)
    kc.launch("quantize_q8x4", kc.QuantizeArgs(bx.ptr, bq.ptr, bd.ptr, nb))
    kc.launch(f"matvec_{qtype}_q8", kc.MatvecQ4Q8Args(stream.ptr, bq.ptr, bd.ptr, by.ptr, None, rows, k))
    y = by.download(np.float32)[:rows]
    for b in (stream, bx, bq, bd, by):
        b.free()
    return y


def test_empty_launches_succeed_and_write_nothing():
    k = 256
    w = kq.random_blocks("q4k", 8, k, 1)
    stream = kc.upload_weights("q4k", w, 8, k)
    sentinel = np.full(8, 7.0, np.float32)
    bq, bd, by, bx = kc.Buffer(k), kc.Buffer(64), kc.Buffer.of(sentinel), kc.Buffer.of(np.ones(k, np.float32))
    for q in ("q4k", "q6k"):
        assert kc.launch_status(f"matvec_{q}_q8", kc.MatvecQ4Q8Args(stream.ptr, bq.ptr, bd.ptr, by.ptr, None, 0, k)) == "Success"
    assert kc.launch_status("quantize_q8x4", kc.QuantizeArgs(bx.ptr, bq.ptr, bd.ptr, 0)) == "Success"
    assert kc.launch_status("vector_add", kc.VectorAddArgs(bx.ptr, bx.ptr, by.ptr, 0)) == "Success"
    kc.synchronize()
    assert np.array_equal(by.download(np.float32), sentinel)
    for b in (stream, bq, bd, by, bx):
        b.free()


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
def test_matvec_largest_k(qtype):
    rows, k = 24, 32768
    note(f"matvec {qtype} {rows}x{k}")
    w = kq.random_blocks(qtype, rows, k, 11)
    x = kq.randn(k, 12)
    xq, xd = oracle.quantize_q8x4(O, x)
    want = oracle.matvec(O, qtype, w, xq, xd, rows, k)
    assert np.array_equal(kq.bits(matvec(qtype, w, x, rows, k)), kq.bits(want))
    # one super-block more than the staging holds: refused before any launch
    k2 = k + 256
    nb = k2 // 32
    stream = kc.Buffer(kc.stream_bytes(qtype, rows, k2))
    bq, bd, by = kc.Buffer(nb * 32), kc.Buffer(nb * 8), kc.Buffer(rows * 4)
    st = kc.launch_status(f"matvec_{qtype}_q8", kc.MatvecQ4Q8Args(stream.ptr, bq.ptr, bd.ptr, by.ptr, None, rows, k2))
    assert st == "InvalidValue"
    for b in (stream, bq, bd, by):
        b.free()


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("rows,k", [(8, 256), (24, 1280), (1000, 256 * 7), (4104, 2304)])
def test_matvec_ragged_shapes(qtype, rows, k):
    """rows % 16 != 0 (a half-filled last tile) and k / 256 % 4 != 0 (a padded super-block group)."""
    note(f"matvec ragged {qtype} {rows}x{k}")
    w = kq.random_blocks(qtype, rows, k, rows + k)
    x = kq.uniform(k, 5, -2, 2)
    xq, xd = oracle.quantize_q8x4(O, x)
    want = oracle.matvec(O, qtype, w, xq, xd, rows, k)
    assert np.array_equal(kq.bits(matvec(qtype, w, x, rows, k)), kq.bits(want))
