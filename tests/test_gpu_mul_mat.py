"""The MUL_MAT dispatcher (kcMulMat, include/kernelcore/mul_mat.h) on the GPU: every branch of the
reference backend's mul_mat_impl / quantized_input / batch_k256
(integrations/llama.cpp/ggml/src/ggml-kernelcore/ggml-kernelcore.cpp:424,471-497,555-589) checked
twice -- the launches it recorded (its plan: the quantizer, the product kernel, the launch count,
the input reuse) and its output against the oracle on the same inputs:
  - ncols == 1: quantize_q8x4 + matvec_{q4k,q6k}_q8, bit-exact (the matvec's own bar);
  - a batch, defaults: quantize_cols_k + matmul_*_q8kx8 (x4 up to 4 columns) against the oracle's
    per-256 matmul -- bit-exact on the column-tiled kernel (under 64 columns), 1e-3 on the MFMA one;
  - GGML_KERNELCORE_Q8K=0: quantize_cols + matmul_*_q8x{4,8} on per-32 slots, each column
    bit-identical to the per-column matvec (the reference's own equality, tests/test_llm_kernels.cpp:277-340);
  - GGML_KERNELCORE_TILE=4: the x4 names;
  - GGML_KERNELCORE_MATVEC_COLS=1: one matvec per column;
  - strided input columns (no per-256 slots): one quantize_q8x4 per column, then the per-32 matmul;
  - F16 weights: matmul_f16 on the f32 columns (the oracle's matmul_f16, 1e-3);
  - two matrices reading one input quantize it once per recording; a reset or a scratch growth
    makes the next one quantize again;
  - the fused producers (fused_norm :502-530, fused_swiglu :533-545): [ADD +] RMS_NORM + MUL and
    SWIGLU write their f32 output (the norm bit-exact against the oracle's fused restatement, SwiGLU
    within 2e-6: exp2 ulps) and its 8-bit slots, which the MUL_MAT reading that output then takes
    without a quantizer -- its result bit-exact against the oracle on the same f32 values."""
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


class Case:
    """A weight matrix (ggml blocks and the GPU stream) and ncols input columns, stride in floats."""

    def __init__(self, qtype, rows, k, ncols, seed, stride=None):
        self.qtype, self.rows, self.k, self.ncols = qtype, rows, k, ncols
        self.stride = stride or k
        self.blocks = kq.random_blocks(qtype, rows, k, seed)
        self.w = kc.upload_weights(qtype, self.blocks, rows, k)
        x = np.zeros(self.stride * ncols, np.float32)
        xs = kq.randn(k * ncols, seed + 1, 1.5).reshape(ncols, k)
        x.reshape(ncols, self.stride)[:, :k] = xs
        self.cols = xs
        self.bx = kc.Buffer.of(x)
        self.by = kc.Buffer(rows * ncols * 4)

    def run(self, rec):
        plan = rec.mul_mat(self.qtype, self.w.ptr, self.rows, self.k, self.bx.ptr, self.ncols, self.by.ptr,
                           x_col_bytes=4 * self.stride)
        note(f"  {self.qtype} {self.rows}x{self.k} ncols={self.ncols} stride={self.stride}: {plan}")
        return plan

    def y(self):
        kc.synchronize()
        return self.by.download(np.float32).reshape(self.ncols, self.rows)

    def matvec_oracle(self):
        out = np.zeros((self.ncols, self.rows), np.float32)
        for c in range(self.ncols):
            xq, xd = oracle.quantize_q8x4(O, self.cols[c])
            getattr(O, f"kco_matvec_{self.qtype}_q8")(self.blocks, xq, xd, out[c], self.rows, self.k)
        return out

    def matmul_k_oracle(self):
        q = np.zeros(self.ncols * (self.k // 256 * 85), np.int32)
        O.kco_quantize_cols_k(np.ascontiguousarray(self.cols).reshape(-1), q, self.k, self.ncols)
        y = np.zeros(self.rows * self.ncols, np.float32)
        getattr(O, f"kco_matmul_{self.qtype}_q8k")(self.blocks, q, y, self.rows, self.k, self.ncols)
        return y.reshape(self.ncols, self.rows)

    def free(self):
        for b in (self.w, self.bx, self.by):
            b.free()


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
def test_single_column_is_quantize_then_matvec(qtype):
    c = Case(qtype, 72, 768, 1, 11)
    rec = kc.MulMatRecording()
    plan = c.run(rec)
    assert plan == {"quantizer": "quantize_q8x4", "input_reused": False, "kernel": f"matvec_{qtype}_q8",
                    "launches": 2, "k256": False}
    assert np.array_equal(kq.bits(c.y()), kq.bits(c.matvec_oracle()))
    rec.close()
    c.free()


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("ncols,name", [(3, "x4"), (4, "x4"), (7, "x8"), (64, "x8")])
def test_batch_defaults_take_per256_slots(qtype, ncols, name):
    c = Case(qtype, 136, 1024, ncols, 20 + ncols)
    rec = kc.MulMatRecording()
    plan = c.run(rec)
    assert plan == {"quantizer": "quantize_cols_k", "input_reused": False, "kernel": f"matmul_{qtype}_q8k{name}",
                    "launches": 2, "k256": True}
    want = c.matmul_k_oracle()
    if ncols < 64:  # the column-tiled kernel: bit-exact
        assert np.array_equal(kq.bits(c.y()), kq.bits(want))
    else:  # the MFMA kernel: exact integers, the final float combine in another order
        assert kq.rel_diff(c.y(), want) < TOL
    rec.close()
    c.free()


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("ncols,tile,name", [(3, 8, "x4"), (6, 8, "x8"), (6, 4, "x4")])
def test_q8k_off_takes_per32_slots_equal_to_the_matvec(qtype, ncols, tile, name):
    c = Case(qtype, 40, 512, ncols, 30 + ncols)
    rec = kc.MulMatRecording(q8k=0, tile=tile)
    plan = c.run(rec)
    assert plan == {"quantizer": "quantize_cols", "input_reused": False, "kernel": f"matmul_{qtype}_q8{name}",
                    "launches": 2, "k256": False}
    assert np.array_equal(kq.bits(c.y()), kq.bits(c.matvec_oracle()))
    rec.close()
    c.free()


def test_tile4_batch_names_x4():
    c = Case("q4k", 64, 512, 9, 41)
    rec = kc.MulMatRecording(tile=4)
    assert c.run(rec)["kernel"] == "matmul_q4k_q8kx4"
    assert np.array_equal(kq.bits(c.y()), kq.bits(c.matmul_k_oracle()))
    rec.close()
    c.free()


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
def test_matvec_cols_runs_one_matvec_per_column(qtype):
    c = Case(qtype, 48, 768, 5, 50)
    rec = kc.MulMatRecording(matvec_cols=1)
    plan = c.run(rec)
    assert plan == {"quantizer": "quantize_cols", "input_reused": False, "kernel": f"matvec_{qtype}_q8",
                    "launches": 1 + 5, "k256": False}
    assert np.array_equal(kq.bits(c.y()), kq.bits(c.matvec_oracle()))
    rec.close()
    c.free()


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
def test_strided_columns_quantize_per_column(qtype):
    c = Case(qtype, 32, 512, 5, 60, stride=512 + 16)
    rec = kc.MulMatRecording()
    plan = c.run(rec)
    assert plan == {"quantizer": "quantize_q8x4", "input_reused": False, "kernel": f"matmul_{qtype}_q8x8",
                    "launches": 5 + 1, "k256": False}
    assert np.array_equal(kq.bits(c.y()), kq.bits(c.matvec_oracle()))
    rec.close()
    c.free()


@pytest.mark.parametrize("ncols", [1, 6])
def test_f16_weights_take_matmul_f16(ncols):
    rows, k = 64, 320
    rng = np.random.default_rng(70 + ncols)
    w = (rng.standard_normal(rows * k) * 0.05).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(ncols * k).astype(np.float32)
    bw, bx, by = kc.Buffer.of(w), kc.Buffer.of(x), kc.Buffer(rows * ncols * 4)
    rec = kc.MulMatRecording()
    plan = rec.mul_mat("f16", bw.ptr, rows, k, bx.ptr, ncols, by.ptr)
    assert plan == {"quantizer": "", "input_reused": False, "kernel": "matmul_f16", "launches": 1, "k256": False}
    kc.synchronize()
    got = by.download(np.float32).reshape(ncols, rows)
    assert kq.rel_diff(got, oracle.matmul_f16(O, w, x, rows, k, ncols)) < TOL
    rec.close()
    for b in (bw, bx, by):
        b.free()


def test_one_input_is_quantized_once_per_recording():
    """q, k, v read one input: the second and third nodes reuse its slots (quantized_input's
    cache); a reset starts a recording that quantizes it again."""
    k, ncols = 768, 6
    x = kq.randn(k * ncols, 80, 1.5)
    bx = kc.Buffer.of(x)
    mats = [Case(qt, rows, k, ncols, 81 + i) for i, (qt, rows) in enumerate((("q4k", 96), ("q4k", 32), ("q6k", 32)))]
    rec = kc.MulMatRecording()
    plans = []
    for m in mats:
        m.bx.free()
        m.bx, m.cols = bx, x.reshape(ncols, k)
        plans.append(m.run(rec))
    assert [p["input_reused"] for p in plans] == [False, True, True]
    assert [p["quantizer"] for p in plans] == ["quantize_cols_k", "", ""]
    assert [p["launches"] for p in plans] == [2, 1, 1]
    for m in mats:
        assert np.array_equal(kq.bits(m.y()), kq.bits(m.matmul_k_oracle()))
    rec.reset()
    assert mats[0].run(rec)["input_reused"] is False
    # another column count or slot kind is another input
    assert mats[0].run(rec)["input_reused"] is True
    rec2 = kc.MulMatRecording(q8k=0)
    assert mats[1].run(rec2)["quantizer"] == "quantize_cols"
    rec.close()
    rec2.close()
    for m in mats:
        m.bx = kc.Buffer(4)
        m.free()
    bx.free()


def test_scratch_growth_drops_the_cached_inputs():
    small = Case("q4k", 32, 256, 2, 90)
    big = Case("q4k", 64, 8192, 40, 91)
    rec = kc.MulMatRecording()
    assert small.run(rec)["input_reused"] is False
    assert big.run(rec)["input_reused"] is False  # grows the scratch past the first size
    assert small.run(rec)["input_reused"] is False  # its slots were in the old scratch
    assert np.array_equal(kq.bits(small.y()), kq.bits(small.matmul_k_oracle()))
    assert np.array_equal(kq.bits(big.y()), kq.bits(big.matmul_k_oracle()))
    rec.close()
    small.free()
    big.free()


@pytest.mark.parametrize("rows", [1, 6])
@pytest.mark.parametrize("with_add", [False, True])
def test_fused_norm_feeds_the_next_mul_mat(rows, with_add):
    """[ADD +] RMS_NORM + MUL: per 256 values for a batch, one launch of the partial sums and one of
    the norm; per 32 for one row, both in one add_norm_q8_f launch. The q / k / v MUL_MATs after it
    reuse its slots."""
    n = 1024
    nb, nsb = n // 32, n // 256
    a, b, w = kq.randn(n * rows, 101), kq.randn(n * rows, 102), kq.uniform(n, 103, 0.5, 1.5)
    x0 = kq.randn(n * rows, 104)
    ba, bb, bw = kc.Buffer.of(a), kc.Buffer.of(b), kc.Buffer.of(w)
    bx = kc.Buffer.of(np.zeros(n * rows, np.float32) if with_add else x0)
    by = kc.Buffer(n * rows * 4)
    rec = kc.MulMatRecording()
    plan = rec.fused_norm(bx.ptr, bw.ptr, by.ptr, n, rows, 1e-5, a=ba.ptr if with_add else None,
                          b=bb.ptr if with_add else None)
    k256 = rows > 1
    if k256:
        assert plan == {"quantizer": "add_sumsq_f" if with_add else "sumsq_part", "input_reused": False,
                        "kernel": "norm_mul_q8k_f", "launches": 2, "k256": True}
    else:
        assert plan == {"quantizer": "", "input_reused": False, "kernel": "add_norm_q8_f", "launches": 1,
                        "k256": False}
    # the oracle's fused restatement of the same two steps
    x = np.zeros(n * rows, np.float32)
    sq = np.zeros(rows * nb * 11, np.int32)
    if with_add:
        O.kco_add_sumsq_f(a, b, x, sq, n, rows)
    else:
        x = x0.copy()
        O.kco_sumsq_part(x, sq, n, rows)
    y = np.zeros(n * rows, np.float32)
    if k256:
        qk = np.zeros(rows * nsb * 85, np.int32)
        O.kco_norm_mul_q8k(x, w, y, qk, sq, n, rows, 1e-5)
    else:
        O.kco_norm_mul_q8(x, w, y, sq, n, rows, 1e-5)
    kc.synchronize()
    assert np.array_equal(kq.bits(bx.download(np.float32)), kq.bits(x))
    assert np.array_equal(kq.bits(by.download(np.float32)), kq.bits(y))
    # q (Q4_K 96 rows) and v (Q6_K 32 rows) read y: no quantizer, the norm's slots
    for qt, r in (("q4k", 96), ("q6k", 32)):
        c = Case(qt, r, n, rows, 110 + r)
        c.bx.free()
        c.bx, c.cols = by, y.reshape(rows, n)
        p = c.run(rec)
        assert p["input_reused"] is True and p["quantizer"] == "" and p["launches"] == (1 if k256 else rows)
        want = c.matmul_k_oracle() if k256 else c.matvec_oracle()
        assert np.array_equal(kq.bits(c.y()), kq.bits(want))
        c.bx = kc.Buffer(4)
        c.free()
    rec.close()
    for buf in (ba, bb, bw, bx, by):
        buf.free()


@pytest.mark.parametrize("cols", [1, 5])
def test_fused_swiglu_feeds_the_down_projection(cols):
    n = 2048
    g, u = kq.randn(n * cols, 120, 3.0), kq.randn(n * cols, 121)
    bg, bu, by = kc.Buffer.of(g), kc.Buffer.of(u), kc.Buffer(n * cols * 4)
    rec = kc.MulMatRecording()
    plan = rec.fused_swiglu(bg.ptr, bu.ptr, by.ptr, n, cols)
    k256 = cols > 1
    assert plan == {"quantizer": "", "input_reused": False, "kernel": "silu_mul_q8kf" if k256 else "silu_mul_q8x4f",
                    "launches": 1, "k256": k256}
    want_y = np.zeros(n * cols, np.float32)
    O.kco_silu_mul(g, u, want_y, n * cols)
    kc.synchronize()
    y = by.download(np.float32)
    # silu's exp2 on the GPU and on the host differ in the last ulps (the layer tests' bar); the down
    # projection below reads the GPU's own y, so its check stays bit-exact
    assert np.allclose(y, want_y, rtol=2e-6, atol=1e-30)
    c = Case("q6k", 64, n, cols, 130)  # down (Q6_K) reads y
    c.bx.free()
    c.bx, c.cols = by, y.reshape(cols, n)
    p = c.run(rec)
    assert p["input_reused"] is True and p["quantizer"] == ""
    want = c.matmul_k_oracle() if k256 else c.matvec_oracle()
    assert np.array_equal(kq.bits(c.y()), kq.bits(want))
    c.bx = kc.Buffer(4)
    c.free()
    rec.close()
    for buf in (bg, bu, by):
        buf.free()
