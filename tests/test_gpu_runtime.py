"""GPU checks of the kc* runtime semantics: memory and its validation, streams, events, graph capture
with concurrent groups, and the capture rules of the reference runtime (src/runtime.cpp:449-455,
882-1038; tests/test_graph.cpp, tests/test_stream.cpp, tests/test_api.cpp)."""
import ctypes as C

import numpy as np
import pytest

import kernelcore_amd as kc
from tests import kq

pytestmark = pytest.mark.gpu
L = None


@pytest.fixture(scope="module", autouse=True)
def runtime():
    global L
    kc.init()
    L = kc.lib()
    yield
    kc.synchronize()


def handle():
    return C.c_void_p()


def test_device_properties():
    p = kc.device_properties()
    print("device:", p.name.decode(), p.worker_count, p.total_memory, flush=True)
    assert p.is_hardware_gpu and p.worker_count > 0 and p.total_memory > 0
    n = C.c_int()
    kc.call("kcGetDeviceCount", C.byref(n))
    assert n.value == 1
    assert kc.status("kcSetDevice", 1) == "InvalidDevice"
    assert kc.status("kcSetDevice", 0) == "Success"


def test_memory_rules():
    b = kc.Buffer(1024)
    assert kc.status("kcFree", C.c_void_p(b.ptr + 16)) == "InvalidPointer"  # not a base
    assert kc.status("kcMemset", C.c_void_p(b.ptr + 1000), 0, 100) == "InvalidPointer"  # past the end
    assert kc.status("kcMemcpy", C.c_void_p(b.ptr), None, 4, kc.HOST_TO_DEVICE) == "InvalidValue"
    assert kc.status("kcMemcpy", C.c_void_p(b.ptr), C.c_void_p(b.ptr), 4, 7) == "InvalidValue"
    p = C.c_void_p()
    assert kc.status("kcMalloc", C.byref(p), 0) == "InvalidValue"
    kc.call("kcMemset", C.c_void_p(b.ptr), 0x5A, 1024)
    assert np.all(b.download(np.uint8) == 0x5A)
    c = kc.Buffer(1024)
    kc.call("kcMemcpy", C.c_void_p(c.ptr), C.c_void_p(b.ptr), 1024, kc.DEVICE_TO_DEVICE)
    assert np.all(c.download(np.uint8) == 0x5A)
    b.free()
    c.free()


def _vec_add_args(n=4096, seed=0):
    a, b = kq.randn(n, seed), kq.randn(n, seed + 1)
    ba, bb, bo = kc.Buffer.of(a), kc.Buffer.of(b), kc.Buffer(n * 4)
    return (a, b), (ba, bb, bo), kc.VectorAddArgs(ba.ptr, bb.ptr, bo.ptr, n)


def test_streams_and_events():
    (a, b), bufs, args = _vec_add_args()
    s, ev, t0, t1 = handle(), handle(), handle(), handle()
    kc.call("kcStreamCreate", C.byref(s))
    kc.call("kcEventCreate", C.byref(ev))
    kc.call("kcEventCreateTimed", C.byref(t0))
    kc.call("kcEventCreateTimed", C.byref(t1))
    kc.call("kcEventRecord", t0, s)
    kc.launch("vector_add", args, s)
    kc.call("kcEventRecord", ev, s)
    kc.call("kcEventRecord", t1, s)
    kc.call("kcEventSynchronize", ev)
    assert kc.status("kcEventQuery", ev) == "Success"
    assert kc.status("kcStreamQuery", s) == "Success"
    ms = C.c_float()
    kc.call("kcEventElapsedTime", C.byref(ms), t0, t1)
    assert ms.value >= 0
    assert np.array_equal(bufs[2].download(np.float32), a + b)
    assert kc.status("kcEventElapsedTime", C.byref(ms), ev, t1) == "InvalidValue"  # untimed event
    for e in (ev, t0, t1):
        kc.call("kcEventDestroy", e)
    kc.call("kcStreamDestroy", s)
    assert kc.status("kcStreamDestroy", s) == "InvalidResourceHandle"
    for x in bufs:
        x.free()


def test_host_func_runs_in_stream_order():
    seen = []
    CB = C.CFUNCTYPE(None, C.c_void_p)
    cb = CB(lambda user: seen.append(user))
    s = handle()
    kc.call("kcStreamCreate", C.byref(s))
    kc.call("kcLaunchHostFunc", s, cb, C.c_void_p(7))
    kc.call("kcStreamSynchronize", s)
    kc.call("kcLaunchHostFunc", None, cb, C.c_void_p(9))  # default stream: synchronous
    assert seen == [7, 9]
    kc.call("kcStreamDestroy", s)


def _matvec_setup(rows=512, k=3072, qtype="q4k", seed=9):
    w = kq.random_blocks(qtype, rows, k, seed)
    x = kq.randn(k, seed + 1)
    stream = kc.upload_weights(qtype, w, rows, k)
    nb = k // 32
    bx, bq, bd, by = kc.Buffer.of(x), kc.Buffer(nb * 32), kc.Buffer(nb * 8), kc.Buffer(rows * 4)
    qa = kc.QuantizeArgs(bx.ptr, bq.ptr, bd.ptr, nb)
    ma = kc.MatvecQ4Q8Args(stream.ptr, bq.ptr, bd.ptr, by.ptr, None, rows, k)
    return (stream, bx, bq, bd, by), qa, ma


def test_graph_capture_replays_match_eager():
    bufs, qa, ma = _matvec_setup()
    kc.launch("quantize_q8x4", qa)
    kc.launch("matvec_q4k_q8", ma)
    eager = bufs[4].download(np.float32)
    kc.call("kcMemset", C.c_void_p(bufs[4].ptr), 0, bufs[4].nbytes)
    s, g = handle(), handle()
    kc.call("kcStreamCreate", C.byref(s))
    kc.call("kcStreamBeginCapture", s)
    kc.launch("quantize_q8x4", qa, s)
    kc.launch("matvec_q4k_q8", ma, s)
    # copies, memsets and syncs are refused while capturing
    assert kc.status("kcMemset", C.c_void_p(bufs[4].ptr), 0, 4) == "UnsupportedOperation"
    assert kc.status("kcDeviceSynchronize") == "UnsupportedOperation"
    assert kc.status("kcStreamSynchronize", s) == "UnsupportedOperation"
    assert kc.status("kcStreamBeginCapture", s) == "InvalidValue"
    kc.call("kcStreamEndCapture", s, C.byref(g))
    assert np.all(bufs[4].download(np.float32) == 0)  # recorded, not run
    for replay in range(3):
        kc.call("kcGraphLaunch", g, s)
        kc.call("kcStreamSynchronize", s)
        assert np.array_equal(bufs[4].download(np.float32), eager), replay
        kc.call("kcMemset", C.c_void_p(bufs[4].ptr), 0, bufs[4].nbytes)
    kc.call("kcGraphLaunch", g, None)  # synchronous on the default stream
    assert np.array_equal(bufs[4].download(np.float32), eager)
    kc.call("kcGraphDestroy", g)
    assert kc.status("kcGraphDestroy", g) == "InvalidResourceHandle"
    kc.call("kcStreamDestroy", s)
    for b in bufs:
        b.free()


def test_concurrent_group_branches():
    (s1, q1, m1), (s2, q2, m2) = [_matvec_setup(rows=256, qtype=t, seed=20 + i) for i, t in enumerate(("q4k", "q6k"))]
    kc.launch("quantize_q8x4", q1)
    kc.launch("quantize_q8x4", q2)
    kc.launch("matvec_q4k_q8", m1)
    kc.launch("matvec_q6k_q8", m2)
    e1, e2 = s1[4].download(np.float32), s2[4].download(np.float32)
    for b in (s1[4], s2[4]):
        kc.call("kcMemset", C.c_void_p(b.ptr), 0, b.nbytes)
    g = handle()
    assert kc.status("kcStreamConcurrentBegin", None) == "InvalidValue"  # not capturing
    kc.call("kcStreamBeginCapture", None)
    kc.call("kcStreamConcurrentBegin", None)
    assert kc.status("kcStreamConcurrentBegin", None) == "InvalidValue"  # already open
    kc.launch("quantize_q8x4", q1)
    kc.launch("quantize_q8x4", q2)
    kc.call("kcStreamConcurrentEnd", None)
    kc.call("kcStreamConcurrentBegin", None)
    kc.launch("matvec_q4k_q8", m1)
    kc.launch("matvec_q6k_q8", m2)
    kc.call("kcStreamConcurrentEnd", None)
    assert kc.status("kcStreamConcurrentEnd", None) == "InvalidValue"
    kc.call("kcStreamEndCapture", None, C.byref(g))
    for replay in range(3):
        kc.call("kcGraphLaunch", g, None)
        assert np.array_equal(s1[4].download(np.float32), e1), replay
        assert np.array_equal(s2[4].download(np.float32), e2), replay
    kc.call("kcGraphDestroy", g)
    for b in s1 + s2:
        b.free()


def test_shutdown_frees_and_reinit():
    b = kc.Buffer(64)
    kc.call("kcShutdown")
    p = C.c_void_p()
    assert kc.status("kcMalloc", C.byref(p), 16) == "NotInitialized"
    kc.init()
    assert kc.status("kcFree", C.c_void_p(b.ptr)) == "InvalidPointer"  # freed by shutdown
    kc.call("kcDeviceReset")
    q = kc.Buffer(16)
    q.free()
