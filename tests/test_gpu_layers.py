"""GPU parity of the layer kernels around the matmuls, through the C ABI, against the oracle
(reference tests/test_llm_kernels.cpp:423-541 fused norm/SwiGLU bit-exact, :678-707 fp16
conversion known answers, :741-794 flash attention rel < 2e-6). Sums of squares, norms and the
fused quantization are bit-exact; kernels that call exp2f / sinf / cosf are compared with a
tolerance (the GPU's math library differs from the CPU's in the last ulps), and their quantized
output is checked to be exactly the quantization of their own float output."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

import kernelcore_amd as kc
import oracle
from tests import kq

pytestmark = pytest.mark.gpu
O = oracle.lib()
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def runtime():
    kc.init()
    yield
    kc.synchronize()


class Bufs:
    def __init__(self):
        self.all = []

    def of(self, a):
        b = kc.Buffer.of(a)
        self.all.append(b)
        return b

    def new(self, nbytes):
        b = kc.Buffer(nbytes)
        self.all.append(b)
        return b

    def free(self):
        for b in self.all:
            b.free()


def test_add_sumsq_norm_mul_q8_bit_exact():
    n, rows = 3072, 3
    nb = n // 32
    a, b, w = kq.randn(n * rows, 1), kq.randn(n * rows, 2), kq.uniform(n, 3, 0.5, 1.5)
    B = Bufs()
    ba, bb, bw = B.of(a), B.of(b), B.of(w)
    bout, by, bq = B.new(n * rows * 4), B.new(n * rows * 4), B.new(rows * nb * 11 * 4)
    kc.launch("add_sumsq_f", kc.AddSumsqFArgs(ba.ptr, bb.ptr, bout.ptr, bq.ptr, None, n, rows))
    kc.launch("norm_mul_q8_f", kc.NormMulQ8Args(bout.ptr, bw.ptr, by.ptr, bq.ptr, None, n, rows, 1e-5))
    out = np.zeros(n * rows, np.float32)
    q = np.zeros(rows * nb * 11, np.int32)
    O.kco_add_sumsq_f(a, b, out, q, n, rows)
    y = np.zeros(n * rows, np.float32)
    O.kco_norm_mul_q8(out, w, y, q, n, rows, 1e-5)
    assert np.array_equal(kq.bits(bout.download(np.float32)), kq.bits(out))
    assert np.array_equal(kq.bits(by.download(np.float32)), kq.bits(y))
    assert np.array_equal(bq.download(np.int32), q)
    # sumsq_part + norm_mul_q8k_f (per-256 slots, partial sums after the rows' slots)
    nsb = n // 256
    bk = B.new(rows * (nsb * 85 + nb * 11) * 4)
    kc.launch("sumsq_part", kc.SumsqPartArgs(bout.ptr, bk.at(rows * nsb * 85 * 4), None, n, rows))
    by2 = B.new(n * rows * 4)
    kc.launch("norm_mul_q8k_f", kc.NormMulQ8Args(bout.ptr, bw.ptr, by2.ptr, bk.ptr, None, n, rows, 1e-5))
    sq = np.zeros(rows * nb * 11, np.int32)
    O.kco_sumsq_part(out, sq, n, rows)
    qk = np.zeros(rows * nsb * 85, np.int32)
    y2 = np.zeros(n * rows, np.float32)
    O.kco_norm_mul_q8k(out, w, y2, qk, sq, n, rows, 1e-5)
    got = bk.download(np.int32)
    assert np.array_equal(got[: rows * nsb * 85], qk)
    assert np.array_equal(kq.bits(by2.download(np.float32)), kq.bits(y2))
    B.free()


@pytest.mark.parametrize("n,rows", [(256, 1), (3072, 1), (3072, 3), (4096, 2), (8192, 1), (5120, 2)])
@pytest.mark.parametrize("mode", ["add", "in_place", "norm_only"])
def test_add_norm_q8_one_launch_bit_exact(n, rows, mode):
    """add_norm_q8_f: add_sumsq_f (or sumsq_part) + norm_mul_q8_f in one launch -- x, y and every
    slot word (codes, scale / sum pairs, the per-32 sums of squares in the tails) as the oracle's
    two steps; in place: x is a's buffer (the residual stream)."""
    note(f"add_norm_q8_f n={n} rows={rows} {mode}")
    nb = n // 32
    a, b, w = kq.randn(n * rows, n + rows), kq.randn(n * rows, n + 7), kq.uniform(n, 3, 0.5, 1.5)
    B = Bufs()
    ba, bb, bw = B.of(a), B.of(b), B.of(w)
    bx = ba if mode == "in_place" else B.of(a if mode == "norm_only" else np.zeros(n * rows, np.float32))
    by, bq = B.new(n * rows * 4), B.new(rows * nb * 11 * 4)
    has_add = mode != "norm_only"
    kc.launch("add_norm_q8_f", kc.AddNormQ8FArgs(ba.ptr if has_add else None, bb.ptr if has_add else None, bx.ptr,
                                                 bw.ptr, by.ptr, bq.ptr, None, n, rows, 1e-5))
    x = np.zeros(n * rows, np.float32)
    q = np.zeros(rows * nb * 11, np.int32)
    if has_add:
        O.kco_add_sumsq_f(a, b, x, q, n, rows)
    else:
        x = a.copy()
        O.kco_sumsq_part(x, q, n, rows)
    y = np.zeros(n * rows, np.float32)
    O.kco_norm_mul_q8(x, w, y, q, n, rows, 1e-5)
    assert np.array_equal(kq.bits(bx.download(np.float32)), kq.bits(x))
    assert np.array_equal(kq.bits(by.download(np.float32)), kq.bits(y))
    assert np.array_equal(bq.download(np.int32), q)
    B.free()


def test_add_norm_q8_refuses_what_it_does_not_cover():
    B = Bufs()
    big = B.new(8448 * 4 * 2)
    q = B.new(8448 // 32 * 11 * 4 * 2)
    A = kc.AddNormQ8FArgs
    assert kc.launch_status("add_norm_q8_f", A(None, None, big.ptr, big.ptr, big.ptr, q.ptr, None, 8448, 1, 1e-5)) \
        == "InvalidValue"  # rows past 8192 values: the two kernels
    assert kc.launch_status("add_norm_q8_f", A(big.ptr, None, big.ptr, big.ptr, big.ptr, q.ptr, None, 256, 1, 1e-5)) \
        == "InvalidValue"  # a without b
    assert kc.launch_status("add_norm_q8_f", A(None, None, big.ptr, big.ptr, big.ptr, q.ptr, None, 300, 1, 1e-5)) \
        == "InvalidValue"
    B.free()


def test_norm_golden_fixture():
    g = np.load(os.path.join(GOLDEN, "norm_mul_q8.npz"))
    n, rows = int(g["n"]), int(g["rows"])
    B = Bufs()
    ba, bb, bw = B.of(g["a"]), B.of(g["b"]), B.of(g["w"])
    bout, by, bq = B.new(n * rows * 4), B.new(n * rows * 4), B.new(rows * (n // 32) * 11 * 4)
    kc.launch("add_sumsq_f", kc.AddSumsqFArgs(ba.ptr, bb.ptr, bout.ptr, bq.ptr, None, n, rows))
    kc.launch("norm_mul_q8_f", kc.NormMulQ8Args(bout.ptr, bw.ptr, by.ptr, bq.ptr, None, n, rows, 1e-5))
    assert np.array_equal(bq.download(np.int32), g["q"])
    assert np.array_equal(kq.bits(by.download(np.float32)), kq.bits(g["y"]))
    # the same in one add_norm_q8_f launch
    bx2, by2, bq2 = B.new(n * rows * 4), B.new(n * rows * 4), B.new(rows * (n // 32) * 11 * 4)
    kc.launch("add_norm_q8_f", kc.AddNormQ8FArgs(ba.ptr, bb.ptr, bx2.ptr, bw.ptr, by2.ptr, bq2.ptr, None, n, rows, 1e-5))
    assert np.array_equal(bq2.download(np.int32), g["q"])
    assert np.array_equal(kq.bits(by2.download(np.float32)), kq.bits(g["y"]))
    B.free()


@pytest.mark.parametrize("per256,n", [(False, 8192), (True, 8192), (True, 12288), (True, 256), (True, 1280)])
def test_silu_mul_q8(per256, n):
    cols = 3
    g, u = kq.randn(n * cols, 4, 3.0), kq.randn(n * cols, 5)
    B = Bufs()
    bg, bu, by = B.of(g), B.of(u), B.new(n * cols * 4)
    slot = n // 256 * 85 if per256 else n // 32 * 11
    bq = B.new(cols * slot * 4)
    kc.launch("silu_mul_q8kf" if per256 else "silu_mul_q8x4f", kc.SiluMulQ8FArgs(bg.ptr, bu.ptr, by.ptr, bq.ptr, None, n, cols))
    y = by.download(np.float32)
    want = np.zeros(n * cols, np.float32)
    O.kco_silu_mul(g, u, want, n * cols)
    assert np.allclose(y, want, rtol=2e-6, atol=1e-30)
    q = bq.download(np.int32).reshape(cols, slot)
    for c in range(cols):  # exactly the quantization of the GPU's own y
        yc = y[c * n:(c + 1) * n]
        if per256:
            assert np.array_equal(q[c], oracle.quantize_q8k(O, yc))
        else:
            xq, xd = oracle.quantize_q8x4(O, yc)
            assert np.array_equal(q[c, : n // 32 * 8], xq)
            assert np.array_equal(kq.bits(q[c, n // 32 * 8: n // 32 * 10].view(np.float32)), kq.bits(xd))
    B.free()


@pytest.mark.parametrize("n,rows", [(128, 40), (128, 4133), (64, 70), (8, 3), (100, 3), (130, 5), (4096, 2),
                                    (20000, 2)])
def test_rms_norm_rows_bit_exact(n, rows):
    """rms_norm with one lane per row (rows of up to 128 values, a multiple of 4: a Qwen3 layer's per-head
    q / k norms; 4133 rows end inside a workgroup), one workgroup per row (up to 16384 values), past that
    one thread per row: all the reference's sequential sums, bit for bit; also in place."""
    note(f"rms_norm n={n} rows={rows}")
    x, w = kq.randn(n * rows, 60 + rows), kq.uniform(n, 61, 0.5, 1.5)
    B = Bufs()
    bx, bw, by = B.of(x), B.of(w), B.new(n * rows * 4)
    want = np.zeros_like(x)
    O.kco_rms_norm(x, w, want, n, rows, 1e-6)
    kc.launch("rms_norm", kc.RmsNormArgs(bx.ptr, bw.ptr, by.ptr, n, rows, 1e-6))
    assert np.array_equal(kq.bits(by.download(np.float32)), kq.bits(want))
    kc.launch("rms_norm", kc.RmsNormArgs(bx.ptr, bw.ptr, bx.ptr, n, rows, 1e-6))  # y = x
    assert np.array_equal(kq.bits(bx.download(np.float32)), kq.bits(want))
    B.free()


def test_elementwise_ops():
    n, rows = 256, 5
    x, w, u = kq.randn(n * rows, 6), kq.uniform(n, 7, 0.5, 1.5), kq.randn(n * rows, 8)
    B = Bufs()
    bx, bw, bu, by = B.of(x), B.of(w), B.of(u), B.new(n * rows * 4)
    kc.launch("rms_norm", kc.RmsNormArgs(bx.ptr, bw.ptr, by.ptr, n, rows, 1e-6))
    want = np.zeros_like(x)
    O.kco_rms_norm(x, w, want, n, rows, 1e-6)
    assert np.array_equal(kq.bits(by.download(np.float32)), kq.bits(want))
    kc.launch("mul_rows", kc.MulRowsArgs(bx.ptr, bw.ptr, by.ptr, n, n * rows))
    O.kco_mul_rows(x, w, want, n, n * rows)
    assert np.array_equal(kq.bits(by.download(np.float32)), kq.bits(want))
    kc.launch("vector_add", kc.VectorAddArgs(bx.ptr, bu.ptr, by.ptr, n * rows))
    assert np.array_equal(kq.bits(by.download(np.float32)), kq.bits(x + u))
    kc.launch("silu_mul", kc.SiluMulArgs(bx.ptr, bu.ptr, by.ptr, n * rows))
    O.kco_silu_mul(x, u, want, n * rows)
    assert np.allclose(by.download(np.float32), want, rtol=2e-6, atol=1e-30)
    B.free()


@pytest.mark.parametrize("neox", [False, True])
def test_rope_ggml(neox):
    hd, nh, nt = 128, 8, 5
    x = kq.randn(hd * nh * nt, 9)
    pos = np.array([0, 1, 77, 511, 1300], np.int32)
    ff = kq.uniform(hd // 2, 10, 1.0, 4.0)
    B = Bufs()
    bx, by, bp, bf = B.of(x), B.new(x.nbytes), B.of(pos), B.of(ff)
    kc.launch("rope_ggml", kc.RopeGgmlArgs(bx.ptr, by.ptr, bp.ptr, bf.ptr, None, hd, nh, nt, np.log2(500000.0), neox))
    want = np.zeros_like(x)
    O.kco_rope_ggml(x, want, pos, ff, hd, nh, nt, np.log2(500000.0), int(neox))
    got = by.download(np.float32)
    assert np.abs(got - want).max() < 2e-5
    assert np.array_equal(got.reshape(nt, -1)[0], x.reshape(nt, -1)[0])  # position 0 is the identity
    B.free()


def test_set_rows_f16_known_answers():
    pairs, rows, src_row, dst_row, dst_rows = 16, 5, 40, 20, 6
    src = np.concatenate([kq.randn(4 * src_row, 11, 300.0), np.zeros(src_row, np.float32)])
    special = np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, -70000.0, 1e-8, -1e-8, 6.1e-5, 2.98e-8, 1.0 + 2 ** -11,
                        1.0 + 3 * 2 ** -11, -2.5, 1e30, 5.96e-8, 3.0], np.float32)
    src[4 * src_row: 4 * src_row + 16] = special
    idx = np.array([2, -1, 0, 9, 5], np.int64)
    B = Bufs()
    bs, bi = B.of(src), B.of(idx)
    bd = B.of(np.full(dst_rows * dst_row, 0x11111111, np.int32))
    kc.launch("set_rows_f16", kc.SetRowsF16Args(bs.ptr, bi.ptr, bd.ptr, None, pairs, rows, src_row, dst_row, dst_rows))
    want = np.full(dst_rows * dst_row * 2, 0x1111, np.uint16)
    O.kco_set_rows_f16(src, idx, want, pairs, rows, src_row, dst_row, dst_rows)
    assert np.array_equal(bd.download(np.uint16), want)
    B.free()


def _fa_case(seed, H=8, H_kv=2, T=300, D=128, N=3, mask=True):
    rng = np.random.default_rng(seed)
    tp = (T + 7) // 8 * 8
    q = rng.standard_normal(N * H * D).astype(np.float32)
    k = rng.standard_normal(T * H_kv * D).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(T * H_kv * D).astype(np.float16).view(np.uint16)
    m = np.zeros(N * tp, np.float16)
    if mask:
        m[:] = -np.inf
        for i in range(N):
            m[i * tp:i * tp + T - N + 1 + i] = 0.0
    d = kc.FaDims(H=H, T=T, D=D, group=H // H_kv, tp=tp, k_row=H_kv * D // 2, k_head=D // 2, v_row=H_kv * D // 2,
                  v_head=D // 2, N=N, q_tok=H * D, q_head=D, m_row=tp // 2, has_mask=int(mask), H_kv=H_kv)
    od = oracle.FaDims(*[getattr(d, f) for f, _ in kc.FaDims._fields_])
    return q, k, v, m.view(np.uint16), d, od


@pytest.mark.parametrize("mask", [True, False])
@pytest.mark.parametrize("shape", [dict(), dict(H=24, H_kv=8, T=640, N=1), dict(H=32, H_kv=8, T=1300, N=2)])
def test_flash_attention(mask, shape):
    note(f"attention {shape} mask={mask}")
    q, k, v, m, d, od = _fa_case(12, mask=mask, **shape)
    want = np.zeros(d.N * d.H * d.D, np.float32)
    O.kco_flash_attn_f16(q, k, v, m, want, C.byref(od), 0.0883883)
    B = Bufs()
    bq, bk, bv, bm = B.of(q), B.of(k), B.of(v), B.of(m if mask else np.zeros(8, np.uint16))
    bs, bmx, bo = B.new(d.H * d.N * d.tp * 4), B.new(d.H * d.N * 4), B.new(want.nbytes)
    kc.launch("fa_scores", kc.FaScoresArgs(bq.ptr, bk.ptr, bm.ptr, bs.ptr, None, d, 0.0883883))
    kc.launch("fa_max", kc.FaMaxArgs(bs.ptr, bmx.ptr, None, d))
    kc.launch("fa_exp", kc.FaExpArgs(bs.ptr, bmx.ptr, None, d))
    kc.launch("fa_values", kc.FaValuesArgs(bs.ptr, bv.ptr, bo.ptr, None, d))
    four = bo.download(np.float32)
    assert kq.rel_diff(four, want) < 2e-6
    bo2 = B.new(want.nbytes)
    kc.launch("flash_attn_f16", kc.FlashAttnArgs(bq.ptr, bk.ptr, bv.ptr, bm.ptr, bo2.ptr, None, d, 0.0883883))
    assert kq.rel_diff(bo2.download(np.float32), want) < 2e-6
    B.free()


def test_flash_attention_golden_fixture():
    g = np.load(os.path.join(GOLDEN, "flash_attn_f16.npz"))
    d = kc.FaDims(*[int(x) for x in g["dims"]])
    B = Bufs()
    bq, bk, bv, bm, bo = B.of(g["q"]), B.of(g["k"]), B.of(g["v"]), B.of(g["m"]), B.new(g["out"].nbytes)
    kc.launch("flash_attn_f16", kc.FlashAttnArgs(bq.ptr, bk.ptr, bv.ptr, bm.ptr, bo.ptr, None, d, float(g["scale"])))
    assert kq.rel_diff(bo.download(np.float32), g["out"]) < 2e-6
    B.free()


def test_layer_argument_validation():
    B = Bufs()
    x = B.new(4096)
    q = B.new(4096)
    assert kc.launch_status("add_sumsq_f", kc.AddSumsqFArgs(x.ptr, x.ptr, x.ptr, q.ptr, None, 100, 1)) == "InvalidValue"
    assert kc.launch_status("sumsq_part", kc.SumsqPartArgs(x.ptr, q.ptr, None, 256, 4)) == "Success"
    assert kc.launch_status("sumsq_part", kc.SumsqPartArgs(x.ptr, q.ptr, None, 256, 5)) == "InvalidPointer"
    assert kc.launch_status("rope_ggml", kc.RopeGgmlArgs(x.ptr, x.ptr, q.ptr, q.ptr, None, 24, 1, 1, 1.0, False)) == "InvalidValue"
    d = kc.FaDims(H=3, T=8, D=8, group=2, tp=8, k_row=4, k_head=4, v_row=4, v_head=4, N=1, q_tok=24, q_head=8,
                  m_row=4, has_mask=0, H_kv=2)  # H != H_kv * group
    assert kc.launch_status("fa_max", kc.FaMaxArgs(x.ptr, q.ptr, None, d)) == "InvalidValue"
    B.free()


@pytest.mark.parametrize("mask", ["causal", "none", "holes"])
@pytest.mark.parametrize("shape", [dict(), dict(H=24, H_kv=8, T=700, N=1), dict(H=32, H_kv=8, T=1300, N=2),
                                   dict(H=8, H_kv=8, T=65, D=64, N=8), dict(H=16, H_kv=2, T=1, D=64, N=1),
                                   dict(H=16, H_kv=2, T=64, D=128, N=5), dict(H=8, H_kv=1, T=200, D=64, N=4)])
def test_flash_decode_split_context(mask, shape):
    """flash_decode_f16 (the context split over 64-position chunks, merged in chunk order) against the
    oracle's FLASH_ATTN_EXT: every group size the kernels take shapes of 1-8, D 64 and 128, one to
    eight query tokens, contexts of one position, one chunk, one more position than a chunk and
    1300; masks causal, absent, or with every position of the second chunk masked (a chunk that
    contributes nothing) and random holes."""
    note(f"flash_decode {shape} mask={mask}")
    q, k, v, m, d, od = _fa_case(14, mask=mask != "none", **shape)
    if mask == "holes":
        mm = m.view(np.float16).reshape(d.N, d.tp)
        rng = np.random.default_rng(3)
        mm[:, 64:128] = -np.inf
        mm[rng.random(mm.shape) < 0.2] = -np.inf
        mm[:, 0] = 0.0  # every query keeps one position
        m = mm.reshape(-1).view(np.uint16)
    want = np.zeros(d.N * d.H * d.D, np.float32)
    O.kco_flash_attn_f16(q, k, v, m, want, C.byref(od), 0.0883883)
    B = Bufs()
    bq, bk, bv, bm = B.of(q), B.of(k), B.of(v), B.of(m if mask != "none" else np.zeros(8, np.uint16))
    nch = (d.T + 63) // 64
    bp, bo = B.new(d.N * d.H * nch * (d.D + 2) * 4), B.new(want.nbytes)
    kc.launch("flash_decode_f16", kc.FlashDecodeArgs(bq.ptr, bk.ptr, bv.ptr, bm.ptr, bo.ptr, bp.ptr, None, d, 0.0883883))
    got = bo.download(np.float32)
    assert np.all(np.isfinite(got))
    assert kq.rel_diff(got, want) < 2e-6, kq.rel_diff(got, want)
    # a part buffer one float short is refused before any launch
    small = B.new(d.N * d.H * nch * (d.D + 2) * 4 - 4)
    with pytest.raises(kc.KcError):
        kc.launch("flash_decode_f16", kc.FlashDecodeArgs(bq.ptr, bk.ptr, bv.ptr, bm.ptr, bo.ptr, small.ptr, None, d,
                                                         0.0883883))
    B.free()
