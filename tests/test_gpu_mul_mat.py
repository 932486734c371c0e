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
    makes the next one quantize again."""
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
