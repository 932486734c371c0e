"""GPU block dequantization (get_rows_kquant) bit-for-bit against the reference's formula.

The north star requires block dequantization to be bit-exact. The kernel decodes rows of the
device weight stream with ggml's dequantize_row_q4_K / q6_K in the reference's float order
(llm/llm_reference.cpp:342-383: d1 = d*sc, m1 = dmin*m, y = d1*q - m1; y = (d*sc)*q). It is compared
with:
  * the oracle's restatement (oracle/kc_oracle.c, itself bit-exact to the reference's
    llm_reference.cpp in tests/test_oracle.py), on random blocks, ragged shapes and repeated /
    permuted row ids;
  * the committed `deq` arrays of tests/golden/matvec_*.npz, written from the reference's own
    library by tests/golden/make_golden.py;
  * blocks whose fp16 d / dmin are the edge patterns of binary16: zero, -0, the smallest and largest
    subnormal, the largest finite value (both signs), infinity and NaN (NaN outputs must sit where
    the reference's do; their payloads are not compared).
Row ids outside [0, rows) give rows of zeros (the ids are device data no host check sees)."""
import glob
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


def gpu_rows(qtype, w, rows, k, ids):
    note(f"get_rows_kquant {qtype} rows={rows} k={k} n={len(ids)}")
    stream = kc.upload_weights(qtype, w, rows, k)
    ids = np.ascontiguousarray(ids, np.int32)
    bi = kc.Buffer.of(ids if ids.size else np.zeros(1, np.int32))
    by = kc.Buffer(max(ids.size, 1) * k * 4)
    kc.launch("get_rows_kquant", kc.GetRowsKquantArgs(stream.ptr, bi.ptr, by.ptr, kc.QTYPE[qtype], rows, k, ids.size))
    y = by.download(np.float32, ids.size * k).reshape(ids.size, k)
    for b in (stream, bi, by):
        b.free()
    return y


def same_bits(a, b):
    """Bit-identical, except that NaN payloads are not compared (only their positions)."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(kq.bits(a[~na]), kq.bits(b[~nb]))


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("rows,k", [(16, 256), (40, 768), (33, 1280), (7, 3072), (128, 4096)])
def test_get_rows_bit_exact_random_blocks(qtype, rows, k):
    w = kq.random_blocks(qtype, rows, k, seed=rows * 7 + k)
    want = oracle.dequant(O, qtype, w, rows, k)
    ids = np.arange(rows)
    got = gpu_rows(qtype, w, rows, k, ids)
    assert same_bits(got, want)
    # repeated and permuted ids
    perm = np.random.default_rng(rows).permutation(np.concatenate([ids, ids[: rows // 2]]))
    got = gpu_rows(qtype, w, rows, k, perm)
    assert same_bits(got, want[perm])


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "matvec_*.npz"))))
def test_get_rows_matches_golden_dequant(path):
    z = np.load(path)
    qtype, rows, k = str(z["qtype"]), int(z["rows"]), int(z["k"])
    got = gpu_rows(qtype, z["w"], rows, k, np.arange(rows))
    assert same_bits(got.reshape(-1), z["deq"])


EDGE_HALVES = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0xFBFF, 0x3C00, 0x7C00, 0x7E00]


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
def test_get_rows_fp16_scale_edge_patterns(qtype):
    rows, k = 16 * len(EDGE_HALVES), 512
    w = kq.random_blocks(qtype, rows, k, seed=91).reshape(rows * 2, -1).copy()
    n = len(EDGE_HALVES)
    for i in range(rows * 2):
        d = EDGE_HALVES[i % n]
        if qtype == "q4k":
            w[i, 0:2] = np.array([d], np.uint16).view(np.uint8)
            w[i, 2:4] = np.array([EDGE_HALVES[(i // n + i) % n]], np.uint16).view(np.uint8)
        else:
            w[i, 208:210] = np.array([d], np.uint16).view(np.uint8)
    w = w.reshape(-1)
    want = oracle.dequant(O, qtype, w, rows, k)
    got = gpu_rows(qtype, w, rows, k, np.arange(rows))
    assert np.isnan(want).any() and np.isinf(want).any()  # the patterns reach NaN and infinity
    assert same_bits(got, want)


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
def test_get_rows_out_of_range_ids_give_zeros(qtype):
    rows, k = 24, 512
    w = kq.random_blocks(qtype, rows, k, seed=5)
    want = oracle.dequant(O, qtype, w, rows, k)
    ids = np.array([3, -1, rows, 2**31 - 1, 23, -2**31], np.int32)
    got = gpu_rows(qtype, w, rows, k, ids)
    assert same_bits(got[0], want[3]) and same_bits(got[4], want[23])
    assert not got[[1, 2, 3, 5]].any()


def test_get_rows_validation():
    w = kq.random_blocks("q4k", 16, 256, seed=1)
    stream = kc.upload_weights("q4k", w, 16, 256)
    bi, by = kc.Buffer.of(np.zeros(4, np.int32)), kc.Buffer(4 * 256 * 4)
    try:
        bad = [kc.GetRowsKquantArgs(stream.ptr, bi.ptr, by.ptr, 13, 16, 256, 4),       # qtype
               kc.GetRowsKquantArgs(stream.ptr, bi.ptr, by.ptr, 12, 16, 300, 4),       # k % 256
               kc.GetRowsKquantArgs(stream.ptr, bi.ptr, by.ptr, 12, 16, 256, 5),       # ids / y too short
               kc.GetRowsKquantArgs(stream.ptr, bi.ptr, by.ptr, 12, 64, 256, 4)]       # stream too short
        for a in bad:
            assert kc.launch_status("get_rows_kquant", a) in ("InvalidValue", "InvalidPointer")
        assert kc.launch_status("get_rows_kquant", kc.GetRowsKquantArgs(stream.ptr, bi.ptr, by.ptr, 12, 16, 256, 0)) == "Success"
    finally:
        for b in (stream, bi, by):
            b.free()
