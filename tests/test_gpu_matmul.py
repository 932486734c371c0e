"""GPU parity of the K-quant matmuls (the prefill path) through the C ABI, against the oracle.

Mirrors the reference's tests/test_llm_kernels.cpp:277-340 (per-32 matmuls equal the per-column
matvec, bit-exact, for several ncols and row counts; a dims mismatch is InvalidValue) and :344-420
(per-256 slots equal quantizeQ8K, matmuls equal matvecQ*KQ8K per column, error vs the exact product
below 2% of the largest output and at most 4x the per-32 error). Bar: 1e-3 max relative error;
the column-tiled kernel is also bit-exact and that is asserted where it runs."""
import ctypes as C
import sys

import numpy as np
import pytest

import kernelcore_amd as kc
import oracle
from tests import kq

pytestmark = pytest.mark.gpu
O = oracle.lib()
TOL = 1e-3


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def runtime():
    kc.init()
    yield
    kc.synchronize()


def gpu_slots(x, k, ncols, per256):
    bx = kc.Buffer.of(x)
    ints = ncols * (k // 256 * 85 if per256 else k // 32 * 11)
    bq = kc.Buffer(ints * 4)
    kc.launch("quantize_cols_k" if per256 else "quantize_cols", kc.QuantizeColsArgs(bx.ptr, bq.ptr, None, k, ncols))
    bx.free()
    return bq


def oracle_slots(x, k, ncols, per256):
    q = np.zeros(ncols * (k // 256 * 85 if per256 else k // 32 * 11), np.int32)
    (O.kco_quantize_cols_k if per256 else O.kco_quantize_cols)(x, q, k, ncols)
    return q


def run_matmul(qtype, per256, w, x, rows, k, ncols, name_tile="x8"):
    stream = kc.upload_weights(qtype, w, rows, k)
    bq = gpu_slots(x, k, ncols, per256)
    by = kc.Buffer(rows * ncols * 4)
    name = f"matmul_{qtype}_q8{'k' if per256 else ''}{name_tile}"
    kc.launch(name, kc.MatmulKQ8Args(stream.ptr, bq.ptr, by.ptr, None, rows, k, ncols, 8))
    y = by.download(np.float32).reshape(ncols, rows)
    slots = bq.download(np.int32)
    for b in (stream, bq, by):
        b.free()
    return y, slots


def oracle_matmul(qtype, per256, w, q, rows, k, ncols):
    y = np.zeros(rows * ncols, np.float32)
    getattr(O, f"kco_matmul_{qtype}_q8{'k' if per256 else ''}")(w, q, y, rows, k, ncols)
    return y.reshape(ncols, rows)


CASES = [(8, 256, 1), (8, 256, 3), (40, 768, 4), (40, 768, 7), (64, 3072, 8), (200, 1024, 9), (1000, 512, 13),
         (24, 4096, 5)]


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("per256", [False, True], ids=["q8", "q8k"])
@pytest.mark.parametrize("rows,k,ncols", CASES)
def test_matmul_matches_oracle(qtype, per256, rows, k, ncols):
    note(f"matmul {qtype} per256={per256} {rows}x{k} ncols={ncols}")
    w = kq.random_blocks(qtype, rows, k, seed=rows * 7 + k + ncols)
    x = kq.randn(k * ncols, rows + ncols, 2.0)
    y, slots = run_matmul(qtype, per256, w, x, rows, k, ncols, "x4" if ncols % 2 else "x8")
    q = oracle_slots(x, k, ncols, per256)
    if per256:
        assert np.array_equal(slots, q)
    else:  # the partial-sum tails are not written by quantize_cols
        nb = k // 32
        sl = slots.reshape(ncols, nb * 11)[:, : nb * 10]
        assert np.array_equal(sl, q.reshape(ncols, nb * 11)[:, : nb * 10])
    want = oracle_matmul(qtype, per256, w, q, rows, k, ncols)
    assert kq.rel_diff(y, want) < TOL
    assert np.array_equal(kq.bits(y), kq.bits(want))


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
def test_per32_matmul_equals_per_column_matvec(qtype):
    rows, k, ncols = 1000, 768, 9
    note(f"matmul vs matvec {qtype}")
    w = kq.random_blocks(qtype, rows, k, seed=31)
    x = kq.randn(k * ncols, 32)
    y, _ = run_matmul(qtype, False, w, x, rows, k, ncols)
    for c in range(ncols):
        xq, xd = oracle.quantize_q8x4(O, x[c * k:(c + 1) * k])
        assert np.array_equal(kq.bits(y[c]), kq.bits(oracle.matvec(O, qtype, w, xq, xd, rows, k)))


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
def test_per256_error_bounds(qtype):
    """tests/test_llm_kernels.cpp:396-397: per-256 error < 2% of the largest output, <= 4x per-32."""
    rows, k, ncols = 64, 3072, 4
    note(f"per-256 error bound {qtype}")
    w = kq.random_blocks(qtype, rows, k, seed=41)
    x = kq.randn(k * ncols, 42)
    exact = x.reshape(ncols, k).astype(np.float64) @ oracle.dequant(O, qtype, w, rows, k).astype(np.float64).T
    y8k, _ = run_matmul(qtype, True, w, x, rows, k, ncols)
    y8, _ = run_matmul(qtype, False, w, x, rows, k, ncols)
    e8k = np.abs(y8k - exact).max()
    e8 = np.abs(y8 - exact).max()
    assert e8k < 0.02 * np.abs(exact).max()
    assert e8k <= 4 * e8


def test_matmul_argument_validation():
    rows, k, ncols = 16, 512, 3
    w = kq.random_blocks("q4k", rows, k, seed=5)
    stream = kc.upload_weights("q4k", w, rows, k)
    bq = kc.Buffer(ncols * (k // 256) * 85 * 4)
    by = kc.Buffer(rows * ncols * 4)
    A = kc.MatmulKQ8Args
    ok = A(stream.ptr, bq.ptr, by.ptr, None, rows, k, ncols, 8)
    assert kc.launch_status("matmul_q4k_q8kx8", ok) == "Success"
    assert kc.launch_status("matmul_q4k_q8kx8", A(stream.ptr, bq.ptr, by.ptr, None, rows, k, ncols, 0)) == "InvalidValue"
    assert kc.launch_status("matmul_q4k_q8kx8", A(stream.ptr, bq.ptr, by.ptr, None, rows, k, 0, 8)) == "InvalidValue"
    assert kc.launch_status("matmul_q4k_q8kx8", A(stream.ptr, bq.ptr, by.ptr, None, rows, k, ncols + 1, 8)) == "InvalidPointer"
    assert kc.launch_status("matmul_q4k_q8x8", ok) == "InvalidPointer"  # per-32 slots are larger
    dims = kc.Buffer.of(np.array([rows, k, ncols, 8], np.int32))
    assert kc.launch_status("matmul_q4k_q8kx8", A(stream.ptr, bq.ptr, by.ptr, dims.ptr, rows, k, ncols, 8)) == "Success"
    bad = kc.Buffer.of(np.array([rows, k, ncols, 4], np.int32))
    assert kc.launch_status("matmul_q4k_q8kx8", A(stream.ptr, bq.ptr, by.ptr, bad.ptr, rows, k, ncols, 8)) == "InvalidValue"
    for b in (stream, bq, by, dims, bad):
        b.free()


# ---- the MFMA path (per-256 slots, ncols >= 64 by default) ---------------------------------------------

MFMA_CASES = [(8, 256, 32), (40, 768, 33), (128, 3072, 100), (1000, 1024, 128), (136, 8192, 200), (3072, 3072, 64)]


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("rows,k,ncols", MFMA_CASES)
def test_mfma_matmul_matches_oracle(qtype, rows, k, ncols):
    note(f"mfma {qtype} {rows}x{k} ncols={ncols}")
    w = kq.random_blocks(qtype, rows, k, seed=rows + 3 * k + ncols)
    x = kq.randn(k * ncols, ncols + 5, 1.5)
    kc.set_option("matmul_path", 2)  # Q4_K: the producer-wavefront kernel (kmatmul_mfmaws.hip)
    y, _ = run_matmul(qtype, True, w, x, rows, k, ncols)
    ys = {}
    kc.set_option("matmul_ws", 1)
    for nw in (4, 8):  # workgroups of 4 wavefronts (128 rows) and of 8 (256 rows, staggered loads)
        kc.set_option("matmul_waves", nw)
        ys[nw], _ = run_matmul(qtype, True, w, x, rows, k, ncols)
    kc.set_option("matmul_waves", 0)
    kc.set_option("matmul_ws", 0)
    kc.set_option("matmul_path", 1)
    yc, _ = run_matmul(qtype, True, w, x, rows, k, ncols)
    kc.set_option("matmul_path", 7)  # the wide-tile kernel (kmatmul_mfmaw.hip)
    yw, _ = run_matmul(qtype, True, w, x, rows, k, ncols)
    kc.set_option("matmul_path", 0)
    want = oracle_matmul(qtype, True, w, oracle_slots(x, k, ncols, True), rows, k, ncols)
    assert np.array_equal(kq.bits(yc), kq.bits(want))  # the column-tile path stays bit-exact
    for got in (y, ys[4], ys[8], yw):
        assert kq.rel_diff(got, want) < TOL
        assert kq.rel_diff(got, want) < 1e-5  # exact integers; only the final float combine differs
    # the workgroup shape, and loads issued by wavefronts of their own, change no output's arithmetic
    assert np.array_equal(kq.bits(ys[4]), kq.bits(ys[8]))
    assert np.array_equal(kq.bits(y), kq.bits(ys[8]))


def test_mfma_matmul_config3_shapes():
    """512 tokens through gate/up (8192 x 3072) and down (3072 x 8192), Q4_K."""
    ncols = 512
    for rows, k, seed in ((8192, 3072, 301), (3072, 8192, 302)):
        note(f"mfma cfg3 {rows}x{k}x{ncols}")
        w = kq.random_blocks("q4k", rows, k, seed=seed)
        x = kq.randn(k * ncols, seed + 1)
        want = np.zeros(rows * ncols, np.float32)
        got = {}
        kc.set_option("matmul_ws", 1)  # the 4- and 8-wavefront kernels
        for nw in (4, 8):
            kc.set_option("matmul_waves", nw)
            got[nw], slots = run_matmul("q4k", True, w, x, rows, k, ncols)
        kc.set_option("matmul_waves", 0)
        kc.set_option("matmul_ws", 0)
        got[0], slots = run_matmul("q4k", True, w, x, rows, k, ncols)  # the default: producer wavefronts
        O.kco_matmul_q4k_q8k_mt(w, slots, want, rows, k, ncols, O.kco_max_threads())
        for nw, y in got.items():
            assert kq.rel_diff(y, want.reshape(ncols, rows)) < TOL, nw
        assert np.array_equal(kq.bits(got[4]), kq.bits(got[8]))
        assert np.array_equal(kq.bits(got[0]), kq.bits(got[8]))


def test_captured_matmul_keeps_its_scratch_after_an_eager_growth():
    """The MFMA matmul stages fp16 activations in the runtime's per-stream scratch. A graph captured
    with a 64-column matmul records that buffer; a later eager 512-column matmul on the same stream
    grows the scratch. The graph must still read valid memory on every replay (the buffer a capture
    may hold is retired, not freed), so each replay equals the oracle and the eager result."""
    rows, k = 256, 1024
    w = kq.random_blocks("q4k", rows, k, seed=77)
    stream = kc.upload_weights("q4k", w, rows, k)
    s = C.c_void_p()
    kc.call("kcStreamCreate", C.byref(s))
    bufs = [stream]
    try:
        x64 = kq.randn(64 * k, 78)
        bq64 = gpu_slots(x64, k, 64, True)
        by64 = kc.Buffer(rows * 64 * 4)
        bufs += [bq64, by64]
        want64 = np.zeros(rows * 64, np.float32)
        O.kco_matmul_q4k_q8k(w, oracle_slots(x64, k, 64, True), want64, rows, k, 64)
        note("capture: 64-column matmul")
        kc.call("kcStreamBeginCapture", s)
        kc.launch("matmul_q4k_q8kx8", kc.MatmulKQ8Args(stream.ptr, bq64.ptr, by64.ptr, None, rows, k, 64, 8), s)
        g = C.c_void_p()
        kc.call("kcStreamEndCapture", s, C.byref(g))
        x512 = kq.randn(512 * k, 79)
        bq512 = gpu_slots(x512, k, 512, True)
        by512 = kc.Buffer(rows * 512 * 4)
        bufs += [bq512, by512]
        for rep in range(3):
            kc.call("kcMemset", C.c_void_p(by64.ptr), 0, rows * 64 * 4)
            note(f"eager 512-column matmul, then replay {rep}")
            kc.launch("matmul_q4k_q8kx8", kc.MatmulKQ8Args(stream.ptr, bq512.ptr, by512.ptr, None, rows, k, 512, 8), s)
            kc.call("kcGraphLaunch", g, s)
            kc.call("kcStreamSynchronize", s)
            got = by64.download(np.float32)
            assert kq.rel_diff(got, want64) < TOL
        want512 = np.zeros(rows * 512, np.float32)
        O.kco_matmul_q4k_q8k(w, oracle_slots(x512, k, 512, True), want512, rows, k, 512)
        assert kq.rel_diff(by512.download(np.float32), want512) < TOL
        kc.call("kcGraphDestroy", g)
    finally:
        kc.call("kcStreamSynchronize", s)
        kc.call("kcStreamDestroy", s)
        for b in bufs:
            b.free()
