"""GPU parity of matmul_f16 (fp16 weights x fp32 activations; reference kernels/llm/matmul_f16.cu,
mirror llm/llm_reference.cpp:756-764) through the C ABI, against the oracle (kco_matmul_f16,
pinned bit-exact to the mirror in tests/test_oracle.py).

Every kernel of the launcher is covered: the wavefront-per-row kernel (ncols <= 8, k % 8 == 0),
the MFMA kernel with hi/lo activation operands (ncols > 8, k % 16 == 0), the column launches of 8
(k % 8 == 0 but not % 16) and the one-thread-per-output kernel (k only even), at rows that are not
multiples of the 64-row tile. Bar: 1e-3 max relative error, measured against
the largest output of each column (outputs near zero are sums with cancellation); the kernels
reach ~1e-6. Validation: the reference's rules (rows % 8, k even, ranges, dims)."""
import sys

import numpy as np
import pytest

import kernelcore_amd as kc
import oracle

pytestmark = pytest.mark.gpu
O = oracle.lib()
TOL = 1e-3


@pytest.fixture(scope="module", autouse=True)
def runtime():
    kc.init()
    yield
    kc.synchronize()


def case(rows, k, ncols, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(rows * k) * 0.05).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(ncols * k).astype(np.float32)
    return w, x


def run(w, x, rows, k, ncols, dims=None):
    bw, bx, by = kc.Buffer.of(w), kc.Buffer.of(x), kc.Buffer(rows * ncols * 4)
    kc.launch("matmul_f16", kc.MatmulF16Args(bw.ptr, bx.ptr, by.ptr, dims, rows, k, ncols))
    y = by.download(np.float32).reshape(ncols, rows)
    for b in (bw, bx, by):
        b.free()
    return y


def max_rel(got, want):
    scale = np.maximum(np.abs(want).max(axis=1, keepdims=True), 1e-30)
    return float((np.abs(got.astype(np.float64) - want) / scale).max())


@pytest.mark.parametrize("rows,k,ncols", [
    (8, 256, 1), (1024, 4096, 1), (136, 3072, 2), (72, 512, 3), (1024, 4096, 8),  # wavefront-per-row kernel
    (64, 512, 9), (200, 1024, 64), (1024, 4096, 100), (136, 768, 512),            # MFMA kernel
    (40, 520, 20),                                                                 # k % 16 != 0: launches of 8
    (16, 2, 3), (24, 130, 5),                                                      # k % 8 != 0: one thread each
])
def test_matmul_f16_matches_oracle(rows, k, ncols):
    print(f"matmul_f16 rows {rows} k {k} ncols {ncols}", flush=True)
    sys.stdout.flush()
    w, x = case(rows, k, ncols, rows + k + ncols)
    got = run(w, x, rows, k, ncols)
    want = oracle.matmul_f16(O, w, x, rows, k, ncols).astype(np.float64)
    assert np.all(np.isfinite(got))
    err = max_rel(got, want)
    assert err < TOL, err
    # the kernels keep the activations to within ~2^-22 (hi/lo split): far below the bar
    assert err < 1e-5, err


def test_matmul_f16_validation():
    w, x = case(16, 64, 2, 1)
    bw, bx, by = kc.Buffer.of(w), kc.Buffer.of(x), kc.Buffer(16 * 2 * 4)
    st = lambda a: kc.launch_status("matmul_f16", a)
    assert st(kc.MatmulF16Args(bw.ptr, bx.ptr, by.ptr, None, 16, 64, 2)) == "Success"
    assert st(kc.MatmulF16Args(bw.ptr, bx.ptr, by.ptr, None, 12, 64, 2)) == "InvalidValue"  # rows % 8
    assert st(kc.MatmulF16Args(bw.ptr, bx.ptr, by.ptr, None, 16, 63, 2)) == "InvalidValue"  # k odd
    assert st(kc.MatmulF16Args(bw.ptr, bx.ptr, by.ptr, None, 16, 64, 0)) == "InvalidValue"  # ncols
    assert st(kc.MatmulF16Args(bw.ptr, bx.ptr, by.ptr, None, 16, 64, 3)) != "Success"  # x / y too small
    dims = kc.Buffer.of(np.array([16, 64, 2], np.int32))
    assert st(kc.MatmulF16Args(bw.ptr, bx.ptr, by.ptr, dims.ptr, 16, 64, 2)) == "Success"
    bad = kc.Buffer.of(np.array([16, 64, 3], np.int32))
    assert st(kc.MatmulF16Args(bw.ptr, bx.ptr, by.ptr, bad.ptr, 16, 64, 2)) == "InvalidValue"
    for b in (bw, bx, by, dims, bad):
        b.free()
