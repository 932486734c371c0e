"""BASELINE configs 1-3 on the inputs the configs name, and the MFMA matmul at the edge of its exact
integers.

Configs 1-3: weights drawn from N(0, 0.02) and quantized to Q4_K / Q6_K as ggml does
(kernelcore_amd/synth.py: fill_normal_f32 + quantize_kquant on the GPU, the blocks read back to the
host), activations N(0, 1), quantized on the GPU by the reference's quantizers. The activation
slots and the matvecs must equal the oracle's bit for bit; the config-3 matmuls (the MFMA kernel)
sum in another order and are held to 1e-5 (exact integers per super-block; the float combine
differs by ulps). Config 1 also at every matvec launch shape and staging order.

The edge: the MFMA kernels sum each super-block's integer products in f32, exact while the partial
sums stay below 2^24. One super-block of Q4_K reaches sum sc q x = 8 x 63 x 32 x 15 x 127 = 3.07e7
and one of Q6_K 16 x 127 x 16 x 32 x 127 = 1.32e8 in magnitude, with every scale and value at its
largest: blocks and activations drawn near those tops (odd and even products) drive every partial
sum past 2^24, where each f32 addition may round by half its spacing (1 below 2^25, 4 below 2^27). With at most 256 additions per super-block (512 for
Q6_K's two operands) that bounds the error by 256 / |sum| (Q4_K, 1e-5 at the sums drawn) and
512 x 4 / |sum| (Q6_K, 1.8e-5) relative: inside the reference's 1e-3 bar; measured 2.4e-7 and 2.2e-7."""
import sys

import numpy as np
import pytest

import kernelcore_amd as kc
import oracle
from kernelcore_amd import synth
from tests import kq
from tests.test_gpu_kquant import gpu_matvec, gpu_quantize
from tests.test_gpu_matmul import gpu_slots, oracle_slots, run_matmul

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


def test_config1_on_ggml_quantized_weights():
    """Config 1: 3072 x 3072 Q4_K, N(0, 0.02) weights, x ~ N(0, 1): quantize + matvec bit-exact, at
    every launch shape."""
    rows = k = 3072
    w = synth.quantized_matrix("q4k", rows, k, seed=4101)
    x = kq.randn(k, 4102)
    xq, xd = oracle.quantize_q8x4(O, x)
    gq, gd = gpu_quantize(x)
    assert np.array_equal(gq, xq) and np.array_equal(kq.bits(gd), kq.bits(xd))
    want = oracle.matvec(O, "q4k", w, xq, xd, rows, k)
    for waves in (0, 1, 2, 4):
        assert np.array_equal(kq.bits(gpu_matvec("q4k", w, x, rows, k, waves)), kq.bits(want)), waves
    for af in (1, 2):  # the weights' loads first; the activations first
        kc.set_option("matvec_af", af)
        try:
            assert np.array_equal(kq.bits(gpu_matvec("q4k", w, x, rows, k)), kq.bits(want)), af
        finally:
            kc.set_option("matvec_af", 0)


def test_config2_on_ggml_quantized_weights():
    """Config 2: the 128256 x 3072 Q6_K head, N(0, 0.02) weights: bit-exact."""
    rows, k = 128256, 3072
    note("config 2 on ggml-quantized weights")
    w = synth.quantized_matrix("q6k", rows, k, seed=4201)
    x = kq.randn(k, 4202)
    xq, xd = oracle.quantize_q8x4(O, x)
    want = np.zeros(rows, np.float32)
    O.kco_matvec_q6k_q8_mt(w, xq, xd, want, rows, k, O.kco_max_threads())
    assert np.array_equal(kq.bits(gpu_matvec("q6k", w, x, rows, k)), kq.bits(want))


def test_config3_on_ggml_quantized_weights():
    """Config 3: gate / up (8192 x 3072) and down (3072 x 8192) Q4_K at 512 columns, N(0, 0.02)
    weights, x ~ N(0, 1): the per-256 slots bit-exact, the MFMA products within 1e-5."""
    ncols = 512
    for i, (rows, k) in enumerate(((8192, 3072), (3072, 8192))):
        note(f"config 3 on ggml-quantized weights: {rows} x {k}")
        w = synth.quantized_matrix("q4k", rows, k, seed=4301 + i)
        x = kq.randn(k * ncols, 4311 + i)
        slots = oracle_slots(x, k, ncols, True)
        b = gpu_slots(x, k, ncols, True)
        assert np.array_equal(b.download(np.int32), slots)
        b.free()
        y, _ = run_matmul("q4k", True, w, x, rows, k, ncols)
        want = np.zeros(rows * ncols, np.float32)
        O.kco_matmul_q4k_q8k_simd(w, slots, want, rows, k, ncols, O.kco_max_threads())
        r = kq.rel_diff(y, want.reshape(ncols, rows))
        note(f"  max relative difference {r:.2e}")
        assert r < 1e-5


def extreme_q4k(rows, nsb, rng):
    """Q4_K blocks at the top of their ranges: d = 1, dmin = 0, scales 60-63, mins 0, q 13-15 (odd and
    even products, so that partial sums past 2^24 are not multiples of the f32 spacing)."""
    n = rows * nsb
    sc = rng.integers(60, 64, (n, 8))
    b = np.zeros((n, 144), np.uint8)
    b[:, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    # the 12 packed bytes: sc[j] | (sc[j + 4] >> 4) << 6, m[j] | (m[j + 4] >> 4) << 6, and the low
    # nibbles of sc[j + 4] | m[j + 4] << 4 (mins all 0)
    b[:, 4:8] = (sc[:, :4] & 63) | ((sc[:, 4:] >> 4) << 6)
    b[:, 12:16] = sc[:, 4:] & 15
    q = rng.integers(13, 16, (n, 256))
    b[:, 16:] = (q[:, :128] | (q[:, 128:] << 4)).astype(np.uint8)  # (which nibble holds which k is immaterial here)
    return b.reshape(-1)


def extreme_q6k(rows, nsb, rng):
    """Q6_K blocks at the top of their ranges: d = 1, scales 120-127, q 0-3 (q - 32 = -32 .. -29)."""
    n = rows * nsb
    b = np.zeros((n, 210), np.uint8)
    b[:, :128] = rng.integers(0, 4, (n, 128)) | (rng.integers(0, 4, (n, 128)) << 4)
    b[:, 192:208] = rng.integers(120, 128, (n, 16))
    b[:, 208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    return b.reshape(-1)


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
def test_mfma_matmul_past_the_exact_integer_range(qtype):
    """Every super-block's partial sums pass 2^24 (above); the MFMA kernel stays within the bound the
    f32 roundings allow, against the oracle's exact int32 sums."""
    rows, k, ncols = 256, 1024, 64
    nsb = k // 256
    rng = np.random.default_rng(31)
    w = extreme_q4k(rows, nsb, rng) if qtype == "q4k" else extreme_q6k(rows, nsb, rng)
    # integers 100-127 with 127 first in every super-block (the per-256 scale is then 1 and the
    # values quantize to themselves), every other column negative
    x = rng.integers(100, 128, (ncols, k)).astype(np.float32)
    x[:, ::256] = 127.0
    x[1::2] *= -1.0
    x = x.reshape(-1)
    slots = oracle_slots(x, k, ncols, True)
    want = np.zeros(rows * ncols, np.float32)
    getattr(O, f"kco_matmul_{qtype}_q8k")(w, slots, want, rows, k, ncols)
    per_sb = np.abs(want).max() / nsb
    assert per_sb > 2 ** 24  # the edge is driven: each super-block's sum passes 2^24
    y, _ = run_matmul(qtype, True, w, x, rows, k, ncols)
    r = kq.rel_diff(y, want.reshape(ncols, rows))
    # at most 256 (Q4_K) / 512 (Q6_K) additions per super-block, each rounding by at most half the f32
    # spacing of a partial sum below 2^25 (1) / 2^27 (4)
    top, adds, half = (2 ** 25, 256, 1) if qtype == "q4k" else (2 ** 27, 512, 4)
    assert per_sb < top
    bound = adds * half / per_sb
    note(f"{qtype}: |sum| per super-block {per_sb:.3e}, max relative difference {r:.2e} (bound {bound:.1e})")
    assert r <= bound
