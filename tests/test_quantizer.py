"""The restated ggml weight quantizers (oracle kco_quantize_row_q4k / q6k): f32 -> block_q4_K /
block_q6_K. The reference ships no quantizer and no quantized fixture (its weights come from GGUF
files ggml wrote; its tests fabricate random blocks, tests/test_llm_kernels.cpp:209-219), so bit
parity with a given ggml build is unpinned. What the format and the method fix is checked here, so
that a dropped term, a wrong index or a transposed nibble fails:

  * the bytes decode (with the oracle's dequantization, itself bit-exact to the reference) to
    values within the format's error on N(0, 0.02) weights: Q4_K 8%, Q6_K 2% relative RMS;
  * the last step is a nearest-grid-point rounding: every value lies within half a grid step of its
    decoded value unless it is clamped at the grid's end (beyond it, on the clamped side);
  * the searches earn their keep: lower error than naive min/max (Q4_K) and max-abs (Q6_K)
    quantizers of the same block layout, written here in numpy;
  * exact symmetries of the method: scaling x by 2^e only scales the fp16 d (and dmin) by 2^e
    (while d stays a normal fp16 number);
    negating x only flips the sign of Q6_K's d;
  * special inputs: all-zero blocks, constant blocks, one spike in a block of zeros."""
import numpy as np
import pytest

import oracle
from tests.model64 import dequant_q4k, dequant_q6k

L = oracle.lib()
BB = {"q4k": 144, "q6k": 210}


def quant(qtype, x):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    return oracle.quantize_weights(L, qtype, x, 1, x.size, threads=1)


def deq(qtype, b, k):
    return oracle.dequant(L, qtype, b, 1, k).reshape(-1).astype(np.float64)


def normal(n, seed, std=0.02):
    return (np.random.default_rng(seed).standard_normal(n) * std).astype(np.float32)


def rel_rms(a, b):
    return float(np.sqrt(np.mean((np.asarray(a, np.float64) - b) ** 2)) / np.sqrt(np.mean(np.asarray(b, np.float64) ** 2)))


@pytest.mark.parametrize("qtype,bound", [("q4k", 0.08), ("q6k", 0.02)])
def test_round_trip_error_within_format(qtype, bound):
    x = normal(256 * 400, 1)
    b = quant(qtype, x)
    assert b.size == 400 * BB[qtype]
    assert rel_rms(deq(qtype, b, x.size), x) < bound


def test_q4k_last_step_is_nearest_grid_point():
    x = normal(256 * 300, 2).astype(np.float64)
    b = quant("q4k", x).reshape(-1, 144)
    y = dequant_q4k(b).reshape(-1)
    blocks = b.astype(np.int64)
    xs = x.reshape(-1, 8, 32)
    ys = y.reshape(-1, 8, 32)
    d = np.ascontiguousarray(b[:, 0:2]).view(np.float16).astype(np.float64).reshape(-1)
    sc = blocks[:, 4:16]
    checked = 0
    for j in range(8):
        s = sc[:, j] & 63 if j < 4 else (sc[:, j + 4] & 0xF) | ((sc[:, j - 4] >> 6) << 4)
        step = d * s  # the grid spacing of sub-block j
        err = np.abs(xs[:, j, :] - ys[:, j, :])
        half = step[:, None] / 2 * (1 + 1e-5) + 1e-9
        q = (b[:, 16 + 32 * (j // 2):16 + 32 * (j // 2) + 32] >> (4 * (j % 2))) & 0xF
        inside = (q > 0) & (q < 15) & (step[:, None] > 0)
        assert np.all(err[inside] <= np.broadcast_to(half, err.shape)[inside])
        lo, hi = (q == 0) & (step[:, None] > 0), (q == 15) & (step[:, None] > 0)
        assert np.all((xs[:, j, :] <= ys[:, j, :] + np.broadcast_to(half, err.shape))[lo])
        assert np.all((xs[:, j, :] >= ys[:, j, :] - np.broadcast_to(half, err.shape))[hi])
        checked += inside.sum()
    assert checked > 0.8 * x.size


def test_q6k_last_step_is_nearest_grid_point():
    x = normal(256 * 300, 3).astype(np.float64)
    b = quant("q6k", x).reshape(-1, 210)
    y = dequant_q6k(b).reshape(-1)
    d = np.ascontiguousarray(b[:, 208:210]).view(np.float16).astype(np.float64).reshape(-1)
    sc = b[:, 192:208].view(np.int8).astype(np.float64)
    step = np.abs(d[:, None] * sc)  # per sub-block of 16
    xs, ys = x.reshape(-1, 16, 16), y.reshape(-1, 16, 16)
    q = np.rint(ys / np.where(step[..., None] > 0, d[:, None, None] * sc[..., None], 1.0))  # q - 32
    err = np.abs(xs - ys)
    half = step[..., None] / 2 * (1 + 1e-5) + 1e-9
    inside = (q > -32) & (q < 31) & (step[..., None] > 0)
    assert np.all(err[inside] <= np.broadcast_to(half, err.shape)[inside])
    assert inside.sum() > 0.95 * x.size


def _naive_q4k(x):
    """min/max per sub-block of 32, 6-bit scales and mins, fp16 d and dmin: the same layout."""
    xs = x.reshape(-1, 8, 32).astype(np.float64)
    mn = np.minimum(xs.min(axis=2), 0.0)
    mx = xs.max(axis=2)
    scale = (mx - mn) / 15
    d = (scale.max(axis=1) / 63).astype(np.float16).astype(np.float64)
    dmin = ((-mn).max(axis=1) / 63).astype(np.float16).astype(np.float64)
    ls = np.clip(np.rint(scale / np.where(d > 0, d, 1)[:, None]), 0, 63)
    lm = np.clip(np.rint(-mn / np.where(dmin > 0, dmin, 1)[:, None]), 0, 63)
    step, off = d[:, None] * ls, dmin[:, None] * lm
    q = np.clip(np.rint((xs + off[..., None]) / np.where(step > 0, step, 1)[..., None]), 0, 15)
    return (step[..., None] * q - off[..., None]).reshape(-1)


def _naive_q6k(x):
    xs = x.reshape(-1, 16, 16).astype(np.float64)
    scale = np.abs(xs).max(axis=2) / 31
    d = (scale.max(axis=1) / 127).astype(np.float16).astype(np.float64)
    sc = np.clip(np.rint(scale / np.where(d > 0, d, 1)[:, None]), -128, 127)
    step = d[:, None] * sc
    q = np.clip(np.rint(xs / np.where(step > 0, step, 1)[..., None]), -32, 31)
    return (step[..., None] * q).reshape(-1)


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
def test_search_beats_naive_quantizer(qtype):
    x = normal(256 * 400, 4)
    ours = rel_rms(deq(qtype, quant(qtype, x), x.size), x)
    naive = rel_rms(_naive_q4k(x) if qtype == "q4k" else _naive_q6k(x), x)
    assert ours < 0.95 * naive, (ours, naive)


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("e", [1, 3, 6])
def test_power_of_two_scaling_only_scales_d(qtype, e):
    """Exact while d stays a normal fp16 value (at 6.1e-5 and below, a subnormal d loses bits and the
    last rounding step may move): the base draw is N(0, 0.16), which puts d near 1e-4 (Q6_K) and
    1e-3 (Q4_K)."""
    x = normal(256 * 50, 5, std=0.16)
    a = quant(qtype, x).reshape(-1, BB[qtype])
    b = quant(qtype, x * np.float32(2.0 ** e)).reshape(-1, BB[qtype])
    dcols = [0, 1, 2, 3] if qtype == "q4k" else [208, 209]
    rest = [c for c in range(BB[qtype]) if c not in dcols]
    assert np.array_equal(a[:, rest], b[:, rest])
    for c0 in dcols[::2]:
        da = np.ascontiguousarray(a[:, c0:c0 + 2]).view(np.float16).astype(np.float64)
        db = np.ascontiguousarray(b[:, c0:c0 + 2]).view(np.float16).astype(np.float64)
        assert np.array_equal(db, da * 2.0 ** e)


def test_q6k_negation_flips_only_the_sign_of_d():
    x = normal(256 * 50, 6)
    a = quant("q6k", x).reshape(-1, 210)
    b = quant("q6k", -x).reshape(-1, 210)
    assert np.array_equal(a[:, :209], b[:, :209])
    assert np.array_equal(a[:, 209] ^ 0x80, b[:, 209])


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
def test_special_blocks(qtype):
    z = quant(qtype, np.zeros(512, np.float32))
    assert not z.any()  # all-zero input: an all-zero block (d = dmin = 0)
    for c in (0.013, -0.02):
        x = np.full(256, c, np.float32)
        y = deq(qtype, quant(qtype, x), 256)
        assert np.abs(y - c).max() <= 0.02 * abs(c) + 1e-6
    x = np.zeros(256, np.float32)
    x[77] = 0.5  # one spike: it must survive, everything else stays near 0
    y = deq(qtype, quant(qtype, x), 256)
    assert abs(y[77] - 0.5) < 0.02 and np.abs(np.delete(y, 77)).max() < 0.02


def test_threads_do_not_change_bytes():
    x = normal(3072 * 64, 7)
    for qt in ("q4k", "q6k"):
        a = oracle.quantize_weights(L, qt, x, 64, 3072, threads=1)
        b = oracle.quantize_weights(L, qt, x, 64, 3072, threads=8)
        assert np.array_equal(a, b)
