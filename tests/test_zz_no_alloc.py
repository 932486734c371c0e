"""kcLaunchMatmulNoAlloc against kcLaunchKernel: same name, same arguments, bit-identical outputs.

The no-alloc entry point stages the MFMA matmul's fp16 activations in a fixed device array instead
of the runtime's per-stream scratch; the kernels are the same, so the outputs must be equal bit for
bit. Two calls in a row, the second with a smaller input (the array keeps the first call's
contents), for Q4_K and Q6_K on the MFMA path (per-256 slots, >= 64 columns) and the column path;
then a shape whose staging exceeds the fixed 16 MiB, refused with InvalidValue."""
import ctypes as C
import sys

import numpy as np
import pytest

import kernelcore_amd as kc
from tests import kq

pytestmark = pytest.mark.gpu


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def runtime():
    kc.init()
    yield
    kc.synchronize()


def slots(x, k, ncols):
    bx = kc.Buffer.of(x)
    bq = kc.Buffer(ncols * (k // 256 * 85) * 4)
    kc.launch("quantize_cols_k", kc.QuantizeColsArgs(bx.ptr, bq.ptr, None, k, ncols))
    bx.free()
    return bq


def run_both(qtype, rows, k, ncols, seed):
    note(f"no-alloc matmul {qtype} rows={rows} k={k} ncols={ncols}")
    w = kq.random_blocks(qtype, rows, k, seed)
    stream = kc.upload_weights(qtype, w, rows, k)
    bq = slots(kq.randn(ncols * k, seed + 1), k, ncols)
    ya, yb = kc.Buffer(rows * ncols * 4), kc.Buffer(rows * ncols * 4)
    name = f"matmul_{qtype}_q8kx8"
    kc.launch(name, kc.MatmulKQ8Args(stream.ptr, bq.ptr, ya.ptr, None, rows, k, ncols, 8))
    args = kc.MatmulKQ8Args(stream.ptr, bq.ptr, yb.ptr, None, rows, k, ncols, 8)
    kc.call("kcLaunchMatmulNoAlloc", name.encode(), C.byref(args), None)
    a, b = ya.download(np.float32), yb.download(np.float32)
    for buf in (stream, bq, ya, yb):
        buf.free()
    return a, b


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
def test_no_alloc_matches_launch_kernel_twice(qtype):
    kc.lib().kcLaunchMatmulNoAlloc.argtypes = [C.c_char_p, C.c_void_p, C.c_void_p]
    for rows, k, ncols, seed in ((512, 3072, 256, 1), (256, 2048, 96, 2), (128, 1024, 24, 3)):
        a, b = run_both(qtype, rows, k, ncols, seed)
        assert np.all(np.isfinite(a))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (rows, k, ncols)


def test_no_alloc_refuses_staging_beyond_the_fixed_array():
    kc.lib().kcLaunchMatmulNoAlloc.argtypes = [C.c_char_p, C.c_void_p, C.c_void_p]
    rows, k, ncols = 16, 16384, 512  # 16 MiB of fp16 activations alone, plus mins and scales
    stream = kc.upload_weights("q4k", kq.random_blocks("q4k", rows, k, 9), rows, k)
    bq, by = kc.Buffer(ncols * (k // 256 * 85) * 4), kc.Buffer(rows * ncols * 4)
    try:
        args = kc.MatmulKQ8Args(stream.ptr, bq.ptr, by.ptr, None, rows, k, ncols, 8)
        assert kc.status("kcLaunchMatmulNoAlloc", b"matmul_q4k_q8kx8", C.byref(args), None) == "InvalidValue"
        assert "fixed" in kc.lib().kcGetLastErrorDetail().decode()
        assert kc.status("kcLaunchMatmulNoAlloc", b"matvec_q4k_q8", C.byref(args), None) == "InvalidValue"
    finally:
        for b in (stream, bq, by):
            b.free()
