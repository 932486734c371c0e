"""GPU weight quantizers (quantize_kquant) bit-for-bit against the CPU restatement of ggml's reference
quantizers (oracle kco_quantize_row_q4k / q6k, pinned by tests/test_quantizer.py), and the synthetic
normal generator (fill_normal_f32): moments, determinism, seeds.

The quantizer is third-party arithmetic (ggml's quantize_row_q4_K_ref / q6_K_ref), absent from the
reference tree, so its parity with a given ggml build is unpinned; what is pinned here is that the
device kernel and the CPU restatement produce the same bytes on the same floats, including zero,
constant, spiked, tiny (subnormal fp16 d) and large blocks."""
import sys

import numpy as np
import pytest

import kernelcore_amd as kc
import oracle

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


def gpu_quantize(qtype, x, rows, k):
    note(f"quantize_kquant {qtype} {rows} x {k}")
    bx = kc.Buffer.of(np.ascontiguousarray(x, np.float32).reshape(-1))
    nbytes = rows * (k // 256) * kc.BLOCK_BYTES[qtype]
    bb = kc.Buffer(max(nbytes, 1))
    kc.launch("quantize_kquant", kc.QuantizeKquantArgs(bx.ptr, bb.ptr, kc.QTYPE[qtype], rows, k))
    out = bb.download(np.uint8, nbytes)
    bx.free()
    bb.free()
    return out


def special_rows(k, seed):
    rng = np.random.default_rng(seed)
    rows = [np.zeros(k), np.full(k, 0.013), np.full(k, -0.02), rng.standard_normal(k) * 0.02,
            rng.standard_normal(k) * 1e-6, rng.standard_normal(k) * 30.0, rng.uniform(0, 0.05, k),
            -rng.uniform(0, 0.05, k)]
    spike = np.zeros(k)
    spike[::97] = 0.5
    rows.append(spike)
    mixed = rng.standard_normal(k) * 0.02
    mixed[: k // 2] = 0.0
    rows.append(mixed)
    return np.array(rows, np.float32)


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("rows,k", [(1, 256), (37, 512), (256, 3072), (64, 8192)])
def test_quantize_bit_exact_on_normal_weights(qtype, rows, k):
    x = (np.random.default_rng(rows + k).standard_normal(rows * k) * 0.02).astype(np.float32)
    want = oracle.quantize_weights(O, qtype, x, rows, k)
    got = gpu_quantize(qtype, x, rows, k)
    assert np.array_equal(got, want), int((got != want).sum())


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
def test_quantize_bit_exact_on_special_rows(qtype):
    k = 1024
    x = special_rows(k, 5)
    want = oracle.quantize_weights(O, qtype, x, x.shape[0], k)
    got = gpu_quantize(qtype, x, x.shape[0], k)
    assert np.array_equal(got, want), np.nonzero(got != want)[0][:10]


def test_quantize_zero_rows_and_validation():
    bx, bb = kc.Buffer(4 * 256), kc.Buffer(144)
    try:
        assert kc.launch_status("quantize_kquant", kc.QuantizeKquantArgs(bx.ptr, bb.ptr, 12, 0, 256)) == "Success"
        assert kc.launch_status("quantize_kquant", kc.QuantizeKquantArgs(bx.ptr, bb.ptr, 13, 1, 256)) == "InvalidValue"
        assert kc.launch_status("quantize_kquant", kc.QuantizeKquantArgs(bx.ptr, bb.ptr, 12, 1, 300)) == "InvalidValue"
        assert kc.launch_status("quantize_kquant", kc.QuantizeKquantArgs(bx.ptr, bb.ptr, 14, 1, 256)) == "InvalidPointer"
    finally:
        bx.free()
        bb.free()


def gpu_normal(n, seed, mean=0.0, std=1.0):
    note(f"fill_normal_f32 n={n} seed={seed}")
    b = kc.Buffer(max(n, 1) * 4)
    kc.launch("fill_normal_f32", kc.FillNormalArgs(b.ptr, n, seed, mean, std))
    y = b.download(np.float32, n)
    b.free()
    return y


def test_fill_normal_moments_and_determinism():
    n = 8_000_001  # odd: the last pair writes one value
    y = gpu_normal(n, 42, 0.0, 0.02)
    assert np.all(np.isfinite(y))
    m, s = float(y.mean()), float(y.std())
    assert abs(m) < 5 * 0.02 / np.sqrt(n) and abs(s / 0.02 - 1) < 2e-3
    z = y / 0.02
    # tail fractions of a standard normal: P(|z| > 1) = 0.3173, P(|z| > 2) = 0.0455, P(|z| > 3) = 0.0027
    for t, p in ((1, 0.3173), (2, 0.0455), (3, 0.0027)):
        assert abs(float(np.mean(np.abs(z) > t)) - p) < 5 * np.sqrt(p / n) + 2e-4
    assert np.array_equal(gpu_normal(1000, 42, 0.0, 0.02), y[:1000])  # a function of (seed, index)
    other = gpu_normal(1000, 43, 0.0, 0.02)
    assert not np.array_equal(other, y[:1000])
    shifted = gpu_normal(1001, 42, 1.5, 2.0)
    assert np.allclose(shifted, 1.5 + 2.0 * (y[:1001] / 0.02), rtol=1e-5, atol=1e-5)
