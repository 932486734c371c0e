"""GPU parity of the K-quant hot path through the C ABI: weight streams, activation quantizers and
the decode matvecs against the CPU oracle (oracle/kc_oracle.c, bit-identical to the reference's
llm/llm_reference.cpp). The bar is the reference's own: quantized bytes and dequantized values
bit-exact, matvec outputs within 1e-3 max relative error; the kernels are built to be bit-exact
and that is asserted too (tests/test_llm_kernels.cpp:253-256 in the reference holds its kernels to
the same bit-equality against its mirror)."""
import ctypes as C
import sys

import numpy as np
import pytest

import kernelcore_amd as kc
import oracle
from tests import kq

pytestmark = pytest.mark.gpu
O = oracle.lib()
TOL = 1e-3  # max relative error of matvec/matmul outputs


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def runtime():
    kc.init()
    yield
    kc.synchronize()


def q8(x):
    return oracle.quantize_q8x4(O, x)


def gpu_quantize(x):
    nb = x.size // 32
    bx, bq, bd = kc.Buffer.of(x), kc.Buffer(nb * 32), kc.Buffer(nb * 8)
    kc.launch("quantize_q8x4", kc.QuantizeArgs(bx.ptr, bq.ptr, bd.ptr, nb))
    out = bq.download(np.int32), bd.download(np.float32)
    for b in (bx, bq, bd):
        b.free()
    return out


def gpu_matvec(qtype, w, x, rows, k, waves=0):
    kc.set_option("matvec_waves", waves)
    stream = kc.upload_weights(qtype, w, rows, k)
    nb = k // 32
    bx, bq, bd, by = kc.Buffer.of(x), kc.Buffer(nb * 32), kc.Buffer(nb * 8), kc.Buffer(max(rows, 1) * 4)
    kc.launch("quantize_q8x4", kc.QuantizeArgs(bx.ptr, bq.ptr, bd.ptr, nb))
    kc.launch(f"matvec_{qtype}_q8", kc.MatvecQ4Q8Args(stream.ptr, bq.ptr, bd.ptr, by.ptr, None, rows, k))
    y = by.download(np.float32, rows)
    for b in (stream, bx, bq, bd, by):
        b.free()
    kc.set_option("matvec_waves", 0)
    return y


# ---- weight streams -------------------------------------------------------------------------------

def _layout_positions(qtype, rows, k):
    """(stream offset, ggml offset, length) of a few pieces, from the documented layout."""
    nsb = k // 256
    ngroups = (nsb + 3) // 4
    seg = 9216 if qtype == "q4k" else 13440
    bb = kc.BLOCK_BYTES[qtype]
    out = []
    for row, s, c in [(0, 0, 0), (rows - 1, nsb - 1, 1), (min(17, rows - 1), min(5, nsb - 1), 8)]:
        t, r, g, kq_ = row // 16, row % 16, s // 4, s % 4
        lane = kq_ * 16 + r
        out.append(((t * ngroups + g) * seg + c * 1024 + lane * 16, (row * nsb + s) * bb + 16 * c, 16))
        if qtype == "q6k":
            out.append(((t * ngroups + g) * seg + 13 * 1024 + lane * 2, (row * nsb + s) * bb + 208, 2))
    return out


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("rows,k", [(8, 256), (40, 768), (64, 3072), (1000, 4096)])
def test_stream_round_trip_and_layout(qtype, rows, k):
    note(f"stream {qtype} {rows}x{k}")
    w = kq.random_blocks(qtype, rows, k, seed=rows + k)
    raw = kc.Buffer.of(w)
    stream = kc.repack(qtype, raw, rows, k)
    s = stream.download(np.uint8)
    assert s.size == kc.stream_bytes(qtype, rows, k)
    for so, go, n in _layout_positions(qtype, rows, k):
        assert np.array_equal(s[so:so + n], w[go:go + n])
    back = kc.Buffer(w.nbytes)
    kc.launch("unpack_kquant", kc.KquantRepackArgs(stream.ptr, back.ptr, kc.QTYPE[qtype], rows, k))
    assert np.array_equal(back.download(np.uint8), w)
    # the padding (stream bytes beyond the ggml bytes) is zero
    assert (s == 0).sum() >= s.size - w.size
    for b in (raw, stream, back):
        b.free()


# ---- activation quantizers ----------------------------------------------------------------------

def test_quantize_q8x4_bit_exact():
    x = np.concatenate([kq.randn(32 * 300, 1, 3.0), np.zeros(32, np.float32),
                        np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 127.0] + [0.0] * 25, np.float32),
                        kq.randn(32, 2, 1e-30), kq.randn(32, 3, 1e30)]).astype(np.float32)
    note("quantize_q8x4")
    gq, gd = gpu_quantize(x)
    oq, od = q8(x)
    assert np.array_equal(gq, oq)
    assert np.array_equal(kq.bits(gd), kq.bits(od))


@pytest.mark.parametrize("k,ncols", [(256, 1), (3072, 7), (8192, 3)])
def test_quantize_cols_bit_exact(k, ncols):
    note(f"quantize_cols {k}x{ncols}")
    x = kq.randn(k * ncols, k + ncols, 2.0)
    nb, nsb = k // 32, k // 256
    bx = kc.Buffer.of(x)
    bq = kc.Buffer.of(np.full(ncols * nb * 11, -7, np.int32))
    kc.launch("quantize_cols", kc.QuantizeColsArgs(bx.ptr, bq.ptr, None, k, ncols))
    want = np.full(ncols * nb * 11, -7, np.int32)
    O.kco_quantize_cols(x, want, k, ncols)
    assert np.array_equal(bq.download(np.int32), want)  # the partial-sum tail stays untouched
    bk = kc.Buffer(ncols * nsb * 85 * 4)
    kc.launch("quantize_cols_k", kc.QuantizeColsArgs(bx.ptr, bk.ptr, None, k, ncols))
    wk = np.zeros(ncols * nsb * 85, np.int32)
    O.kco_quantize_cols_k(x, wk, k, ncols)
    assert np.array_equal(bk.download(np.int32), wk)
    for b in (bx, bq, bk):
        b.free()


# ---- matvecs --------------------------------------------------------------------------------------

SHAPES = [(8, 256), (16, 256), (24, 512), (40, 768), (64, 3072), (200, 2048), (1000, 4096), (3072, 3072)]


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("rows,k", SHAPES)
def test_matvec_matches_oracle(qtype, rows, k):
    note(f"matvec {qtype} {rows}x{k}")
    w = kq.random_blocks(qtype, rows, k, seed=3 * rows + k + (qtype == "q6k"))
    x = kq.uniform(k, rows, -3, 3)
    xq, xd = q8(x)
    want = oracle.matvec(O, qtype, w, xq, xd, rows, k)
    got = gpu_matvec(qtype, w, x, rows, k)
    assert kq.rel_diff(got, want) < TOL
    assert np.array_equal(kq.bits(got), kq.bits(want))


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("waves", [1, 2, 4])
def test_matvec_launch_shapes_agree(qtype, waves):
    rows, k = 520, 3072
    note(f"matvec {qtype} waves={waves}")
    w = kq.random_blocks(qtype, rows, k, seed=77)
    x = kq.randn(k, 78)
    xq, xd = q8(x)
    want = oracle.matvec(O, qtype, w, xq, xd, rows, k)
    assert np.array_equal(kq.bits(gpu_matvec(qtype, w, x, rows, k, waves)), kq.bits(want))


def test_matvec_q4k_config1_full_size():
    """3072 x 3072 Q4_K, x ~ N(0, 1)."""
    rows = k = 3072
    note("matvec q4k cfg1")
    w = kq.random_blocks("q4k", rows, k, seed=1001)
    x = kq.randn(k, 1002)
    xq, xd = q8(x)
    want = oracle.matvec(O, "q4k", w, xq, xd, rows, k)
    got = gpu_matvec("q4k", w, x, rows, k)
    assert np.array_equal(kq.bits(got), kq.bits(want))
    # the float64 product of the dequantized weights with the quantized activations (exact ints)
    xs = (xq.view(np.int8).reshape(-1, 32).astype(np.float64) * xd[0::2, None]).reshape(-1)
    ref = oracle.dequant(O, "q4k", w[: 64 * 12 * 144], 64, k).astype(np.float64) @ xs
    assert kq.rel_diff(got[:64], ref) < 1e-5


def test_matvec_q6k_config2_full_size():
    """the 128256 x 3072 Q6_K output head."""
    rows, k = 128256, 3072
    note("matvec q6k cfg2")
    w = kq.random_blocks("q6k", rows, k, seed=2001)
    x = kq.randn(k, 2002)
    xq, xd = q8(x)
    want = np.zeros(rows, np.float32)
    O.kco_matvec_q6k_q8_mt(w, xq, xd, want, rows, k, O.kco_max_threads())
    got = gpu_matvec("q6k", w, x, rows, k)
    assert kq.rel_diff(got, want) < TOL
    assert np.array_equal(kq.bits(got), kq.bits(want))


# ---- argument validation (tests/test_llm_kernels.cpp:333-336, 865-889 in the reference) --------------

def test_matvec_argument_validation():
    rows, k = 16, 512
    w = kq.random_blocks("q4k", rows, k, seed=5)
    stream = kc.upload_weights("q4k", w, rows, k)
    nb = k // 32
    bq, bd, by = kc.Buffer(nb * 32), kc.Buffer(nb * 8), kc.Buffer(rows * 4)
    A = kc.MatvecQ4Q8Args
    assert kc.launch_status("matvec_q4k_q8", A(stream.ptr, bq.ptr, bd.ptr, by.ptr, None, 12, k)) == "InvalidValue"
    assert kc.launch_status("matvec_q4k_q8", A(stream.ptr, bq.ptr, bd.ptr, by.ptr, None, rows, 500)) == "InvalidValue"
    assert kc.launch_status("matvec_q4k_q8", A(stream.ptr, bq.ptr, bd.ptr, by.ptr, None, 24, k)) == "InvalidPointer"
    assert kc.launch_status("matvec_q4k_q8", A(stream.ptr, bq.ptr, bd.ptr, by.ptr + 8, None, rows, k)) == "InvalidPointer"
    dims = kc.Buffer.of(np.array([rows, k], np.int32))
    assert kc.launch_status("matvec_q4k_q8", A(stream.ptr, bq.ptr, bd.ptr, by.ptr, dims.ptr, rows, k)) == "Success"
    bad = kc.Buffer.of(np.array([rows, k + 256], np.int32))
    assert kc.launch_status("matvec_q4k_q8", A(stream.ptr, bq.ptr, bd.ptr, by.ptr, bad.ptr, rows, k)) == "InvalidValue"
    assert kc.launch_status("no_such_kernel", A()) == "KernelNotFound"
    L = kc.lib()
    assert kc.ERRORS[L.kcLaunchKernel(b"matvec_q4k_q8", None, None)] == "InvalidValue"
    args = A(stream.ptr, bq.ptr, bd.ptr, by.ptr, None, rows, k)
    assert kc.ERRORS[L.kcLaunchKernelChunked(b"matvec_q4k_q8", C.byref(args), 0, 16, None)] == "InvalidValue"
    assert kc.ERRORS[L.kcLaunchKernelChunked(b"matvec_q4k_q8", C.byref(args), 8, 16, None)] == "Success"
    rp = kc.KquantRepackArgs(0, 0, 12, rows, k)
    assert kc.ERRORS[L.kcLaunchKernelChunked(b"repack_kquant", C.byref(rp), 8, 16, None)] == "UnsupportedOperation"
    for b in (stream, bq, bd, by, dims, bad):
        b.free()
