"""Pins the CPU oracle (oracle/kc_oracle.c) before anything is checked against it.

Three kinds of checks, so that a dropped term, a wrong index or a swapped operand fails one:
  * bit-exact agreement with the reference's own llm/llm_reference.cpp (oracle/_ref), on random
    inputs, where that library was built (it is built here and travels with the tree);
  * the committed fixtures in tests/golden/ (made by tests/golden/make_golden.py from oracle/_ref);
  * closed forms that do not go through either: IEEE binary16 over all 65536 patterns, the
    textbook K-quant formulas evaluated in float64 from the parsed block fields, quantizer
    invariants, and dequantized float64 dot products (3e-2 of the largest output, the
    reference's own bound, tests/test_llm_kernels.cpp:232-242).
"""
import ctypes as C
import glob
import os

import numpy as np
import pytest

import oracle
from tests import kq

L = oracle.lib()


@pytest.fixture(scope="module")
def R():
    """The reference's own llm_reference.cpp built into oracle/_ref: loaded only by the tests that
    compare against it, and only in the container that holds the reference tree (the build never
    travels to the GPU box)."""
    r = oracle.ref()
    if r is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    return r

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---- fp16 ----------------------------------------------------------------------------------

def test_f16_to_f32_exhaustive_ieee():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = np.array([L.kco_f16_to_f32(int(v)) for v in h], np.float32)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_to_f32_matches_reference_bits(R):
    for v in range(0, 65536, 7):
        a, b = L.kco_f16_to_f32(v), R.kcref_f16_to_f32(v)
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32) or (np.isnan(a) and np.isnan(b))


def test_f32_to_f16_round_nearest_even_with_saturation():
    x = np.concatenate([kq.randn(20000, 1, 100.0), kq.randn(20000, 2, 1e-5), kq.uniform(5000, 3, -7e4, 7e4),
                        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, -65520.0, 1e30, -1e30, 6.1e-5, 5.96e-8,
                                  2.98e-8, 2.99e-8, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11], np.float32)])
    got = np.array([L.kco_f32_to_f16(float(v)) for v in x], np.uint16)
    want = x.astype(np.float16).view(np.uint16).copy()  # numpy: IEEE round to nearest even
    big = np.abs(x) >= 65520.0
    want[big] = np.where(x[big] < 0, 0xFBFF, 0x7BFF)  # saturate to the largest finite value
    want[(x == 0)] = 0  # -0 gives +0
    assert np.array_equal(got, want)


def test_f32_to_f16_matches_reference(R):
    x = np.concatenate([kq.randn(20000, 4, 300.0), kq.randn(5000, 5, 1e-6)])
    for v in x:
        assert L.kco_f32_to_f16(float(v)) == R.kcref_f32_to_f16(float(v))


# ---- dequantization ---------------------------------------------------------------------------

def _q4k_textbook(block):
    """dequantize_row_q4_K from the block fields in float64 (ggml's formula, not the oracle's code)."""
    d = float(block[0:2].view(np.float16)[0])
    dmin = float(block[2:4].view(np.float16)[0])
    sc = block[4:16].astype(np.int64)
    qs = block[16:144]
    out = np.zeros(256)
    for j in range(8):
        if j < 4:
            s, m = sc[j] & 63, sc[j + 4] & 63
        else:
            s = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4)
            m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4)
        q = (qs[32 * (j // 2):32 * (j // 2) + 32] >> (4 * (j % 2))) & 0xF
        out[32 * j:32 * j + 32] = d * s * q - dmin * m
    return out


def _q6k_textbook(block):
    ql, qh = block[0:128].astype(np.int64), block[128:192].astype(np.int64)
    sc = block[192:208].view(np.int8).astype(np.int64)
    d = float(block[208:210].view(np.float16)[0])
    out = np.zeros(256)
    for i in range(256):
        n, r = divmod(i, 128)
        quad, l = divmod(r, 32)
        byte = ql[64 * n + l + (32 if quad in (1, 3) else 0)]
        lo = (byte >> 4) if quad >= 2 else (byte & 0xF)
        hi = (qh[32 * n + l] >> (2 * quad)) & 3
        out[i] = d * sc[8 * n + l // 16 + 2 * quad] * ((lo | (hi << 4)) - 32)
    return out


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
def test_dequant_textbook(qtype):
    w = kq.random_blocks(qtype, 4, 512, seed=11)
    got = oracle.dequant(L, qtype, w, 4, 512)
    bb = kq.BLOCK_BYTES[qtype]
    blocks = w.reshape(-1, bb)
    want = np.concatenate([(_q4k_textbook if qtype == "q4k" else _q6k_textbook)(b) for b in blocks]).reshape(4, 512)
    # two float32 roundings per value (d*sc, then *q - m)
    assert np.allclose(got, want, rtol=3e-7, atol=3e-7 * np.abs(want).max())


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
def test_dequant_matches_reference_bits(qtype, R):
    w = kq.random_blocks(qtype, 16, 1024, seed=12)
    assert np.array_equal(kq.bits(oracle.dequant(L, qtype, w, 16, 1024)), kq.bits(oracle.dequant(R, qtype, w, 16, 1024)))


# ---- activation quantizers ---------------------------------------------------------------------

def _unpack_q8(xq):
    return xq.view(np.int8).astype(np.int64)


def test_quantize_q8x4_invariants():
    x = np.concatenate([kq.randn(32 * 64, 21), np.zeros(32, np.float32),
                        np.full(32, 127.0, np.float32) * np.tile([1, -1], 16).astype(np.float32)])
    xq, xd = oracle.quantize_q8x4(L, x)
    q = _unpack_q8(xq).reshape(-1, 32)
    d, sums = xd[0::2], xd[1::2]
    xb = x.reshape(-1, 32)
    assert np.all(np.abs(q) <= 127)
    assert np.array_equal(sums, q.sum(1).astype(np.float32))  # sum is exact
    assert np.array_equal(d, (np.abs(xb).max(1) / np.float32(127)).astype(np.float32))
    assert np.all(q[-2] == 0) and d[-2] == 0  # all-zero block
    nz = d > 0
    err = np.abs(q[nz] * d[nz, None].astype(np.float64) - xb[nz])
    assert np.all(err <= 0.5 * d[nz, None] * (1 + 1e-6))  # round to nearest
    # ties go away from zero: x = (k + 0.5) * d exactly representable
    t = np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5] + [127.0] + [0.0] * 25, np.float32)
    tq, td = oracle.quantize_q8x4(L, t)
    assert td[0] == 1.0
    assert list(_unpack_q8(tq)[:7]) == [1, -1, 2, -2, 3, -3, 127]


def test_quantize_q8k_invariants():
    x = kq.randn(256 * 6, 22, 3.0)
    q = oracle.quantize_q8k(L, x)
    nsb = 6
    vals = _unpack_q8(q[:nsb * 64]).reshape(nsb, 256)
    d = q[nsb * 64:nsb * 65].view(np.float32)
    s16 = q[nsb * 65:nsb * 81].reshape(nsb, 16)
    packed = q[nsb * 81:nsb * 85].reshape(nsb, 4).view(np.uint8).reshape(nsb, 16)
    assert np.array_equal(d, (np.abs(x.reshape(nsb, 256)).max(1) / np.float32(127)).astype(np.float32))
    assert np.array_equal(s16, vals.reshape(nsb, 16, 16).sum(2))
    b32 = vals.reshape(nsb, 8, 32).sum(2)
    hi = packed[:, :8].view(np.int8).astype(np.int64)
    lo = packed[:, 8:].astype(np.int64)
    assert np.array_equal(hi * 64 + lo, b32)  # B == (B >> 6) * 64 + (B & 63)
    assert np.all(lo < 64)


def test_quantizers_match_reference_bits(R):
    x = kq.randn(256 * 12, 23, 2.0)
    a = oracle.quantize_q8x4(L, x)
    b = oracle.quantize_q8x4(R, x)
    assert np.array_equal(a[0], b[0]) and np.array_equal(kq.bits(a[1]), kq.bits(b[1]))
    assert np.array_equal(oracle.quantize_q8k(L, x), oracle.quantize_q8k(R, x))


def test_quantize_cols_equal_per_column():
    k, ncols = 512, 5
    x = kq.randn(k * ncols, 24)
    nb = k // 32
    q = np.full(ncols * nb * 11, -1, np.int32)
    L.kco_quantize_cols(x, q, k, ncols)
    for c in range(ncols):
        xq, xd = oracle.quantize_q8x4(L, x[c * k:(c + 1) * k])
        slot = q[c * nb * 11:(c + 1) * nb * 11]
        assert np.array_equal(slot[:nb * 8], xq) and np.array_equal(slot[nb * 8:nb * 10].view(np.float32), xd)
        assert np.all(slot[nb * 10:] == -1)  # partial-sum tail untouched
    qk = np.zeros(ncols * 2 * 85, np.int32)
    L.kco_quantize_cols_k(x, qk, k, ncols)
    for c in range(ncols):
        assert np.array_equal(qk[c * 170:(c + 1) * 170], oracle.quantize_q8k(L, x[c * k:(c + 1) * k]))


# ---- matvecs ---------------------------------------------------------------------------------------

SHAPES = [(8, 256), (40, 768), (64, 3072)]


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("rows,k", SHAPES)
def test_matvec_close_to_dequantized_float64(qtype, rows, k):
    w = kq.random_blocks(qtype, rows, k, seed=rows * 31 + k)
    x = kq.uniform(k, 61, -3, 3)
    xq, xd = oracle.quantize_q8x4(L, x)
    y = oracle.matvec(L, qtype, w, xq, xd, rows, k)
    flt = oracle.dequant(L, qtype, w, rows, k).astype(np.float64) @ x.astype(np.float64)
    assert kq.rel_diff(y, flt) < 3e-2
    # the integer part is exact: against the dequantized weights times the *quantized* activations
    xs = (_unpack_q8(xq).reshape(-1, 32) * xd[0::2, None].astype(np.float64)).reshape(-1)
    exact = oracle.dequant(L, qtype, w, rows, k).astype(np.float64) @ xs
    assert kq.rel_diff(y, exact) < 1e-5


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("rows,k", SHAPES)
def test_matvec_matches_reference_bits(qtype, rows, k, R):
    w = kq.random_blocks(qtype, rows, k, seed=rows + k + (qtype == "q6k"))
    x = kq.uniform(k, 62, -3, 3)
    xq, xd = oracle.quantize_q8x4(L, x)
    assert np.array_equal(kq.bits(oracle.matvec(L, qtype, w, xq, xd, rows, k)),
                          kq.bits(oracle.matvec(R, qtype, w, xq, xd, rows, k)))
    slot = oracle.quantize_q8k(L, x)
    a = oracle.matvec_q8k(L, qtype, w, slot, rows, k)
    assert np.array_equal(kq.bits(a), kq.bits(oracle.matvec_q8k(R, qtype, w, slot, rows, k)))
    # per-256 activations: close to the exact product (tests/test_llm_kernels.cpp:396-397)
    flt = oracle.dequant(L, qtype, w, rows, k).astype(np.float64) @ x.astype(np.float64)
    assert kq.rel_diff(a, flt) < 2e-2


# ---- layer ops ------------------------------------------------------------------------------------

def test_layer_ops_match_reference_bits(R):
    n, rows = 512, 3
    nb = n // 32
    a, b, w = kq.randn(n * rows, 31), kq.randn(n * rows, 32), kq.uniform(n, 33, 0.5, 1.5)

    def both(name, *shapes_and_args):
        outs = []
        for lib, pre in ((L, "kco_"), (R, "kcref_")):
            bufs = [np.zeros(s, dt) for s, dt in shapes_and_args[0]]
            getattr(lib, pre + name)(*shapes_and_args[1](bufs))
            outs.append(bufs)
        for u, v in zip(*outs):
            assert np.array_equal(u.view(np.uint8), v.view(np.uint8)), name
        return outs[0]

    both("rms_norm", [((n * rows,), np.float32)], lambda o: (a, w, o[0], n, rows, 1e-5))
    both("mul_rows", [((n * rows,), np.float32)], lambda o: (a, w, o[0], n, n * rows))
    both("silu_mul", [((n * rows,), np.float32)], lambda o: (a, b, o[0], n * rows))
    out, q = both("add_sumsq_f", [((n * rows,), np.float32), ((rows * nb * 11,), np.int32)],
                  lambda o: (a, b, o[0], o[1], n, rows))
    both("sumsq_part", [((rows * nb * 11,), np.int32)], lambda o: (a, o[0], n, rows))

    def nm(o):
        o[1][:] = q
        return (out, w, o[0], o[1], n, rows, 1e-5)
    both("norm_mul_q8", [((n * rows,), np.float32), ((rows * nb * 11,), np.int32)], nm)
    both("norm_mul_q8k", [((n * rows,), np.float32), ((rows * (n // 256) * 85,), np.int32)],
         lambda o: (out, w, o[0], o[1], q, n, rows, 1e-5))
    both("silu_mul_q8f", [((n * rows,), np.float32), ((rows * nb * 11,), np.int32)],
         lambda o: (a, b, o[0], o[1], n, rows))
    both("silu_mul_q8k", [((n * rows,), np.float32), ((rows * (n // 256) * 85,), np.int32)],
         lambda o: (a, b, o[0], o[1], n, rows))
    idx = np.array([2, -1, 0, 7], np.int64)
    src = kq.randn(4 * 32, 34, 50.0)
    both("set_rows_f16", [((5 * 40,), np.uint16)], lambda o: (src, idx, o[0], 16, 4, 32, 20, 5))


def test_norm_mul_q8_closed_form():
    n, rows = 768, 2
    x, w = kq.randn(n * rows, 35), kq.uniform(n, 36, 0.5, 1.5)
    q = np.zeros(rows * (n // 32) * 11, np.int32)
    L.kco_sumsq_part(x, q, n, rows)
    y = np.zeros(n * rows, np.float32)
    L.kco_norm_mul_q8(x, w, y, q, n, rows, 1e-5)
    xr = x.reshape(rows, n).astype(np.float64)
    want = xr / np.sqrt((xr ** 2).mean(1, keepdims=True) + 1e-5) * w
    assert np.allclose(y.reshape(rows, n), want, rtol=2e-6, atol=1e-6)
    for r in range(rows):  # the slot holds exactly quantize_q8x4 of y
        slot = q[r * (n // 32) * 11:(r + 1) * (n // 32) * 11]
        xq, xd = oracle.quantize_q8x4(L, y[r * n:(r + 1) * n])
        assert np.array_equal(slot[:n // 32 * 8], xq) and np.array_equal(slot[n // 32 * 8:n // 32 * 10].view(np.float32), xd)


@pytest.mark.parametrize("neox", [0, 1])
def test_rope_rotation_closed_form(neox):
    hd, nh, nt = 128, 3, 4
    x = kq.randn(hd * nh * nt, 37)
    pos = np.array([0, 5, 77, 1000], np.int32)
    ff = kq.uniform(hd // 2, 38, 1.0, 4.0)
    y = np.zeros_like(x)
    L.kco_rope_ggml(x, y, pos, ff, hd, nh, nt, np.log2(500000.0), neox)
    X = x.reshape(nt, nh, hd).astype(np.float64)
    i = np.arange(hd // 2)
    th = pos[:, None] * (500000.0 ** (-i / (hd // 2))) / ff
    if neox:
        a, b = X[..., :hd // 2], X[..., hd // 2:]
    else:
        a, b = X[..., 0::2], X[..., 1::2]
    c, s = np.cos(th)[:, None, :], np.sin(th)[:, None, :]
    Y = y.reshape(nt, nh, hd)
    ya, yb = (Y[..., :hd // 2], Y[..., hd // 2:]) if neox else (Y[..., 0::2], Y[..., 1::2])
    # theta is a float32 product: its rounding (|theta| <= 1000) bounds the angle error
    assert np.abs(ya - (a * c - b * s)).max() < 2e-4 and np.abs(yb - (a * s + b * c)).max() < 2e-4
    assert np.array_equal(y.reshape(nt, nh, hd)[0], x.reshape(nt, nh, hd)[0])  # position 0: identity


def test_rope_turns_variant_matches_reference_bits(R):
    hd, nh, nt = 128, 2, 3
    x = kq.randn(hd * nh * nt, 39)
    pos = np.array([1, 300, 640], np.int32)
    ff = np.ones(hd // 2, np.float32)
    for neox in (0, 1):
        y1, y2 = np.zeros_like(x), np.zeros_like(x)
        L.kco_rope_ggml_turns(x, y1, pos, ff, hd, nh, nt, np.log2(500000.0), neox)
        R.kcref_rope_ggml(x, y2, pos, ff, hd, nh, nt, np.log2(500000.0), neox)
        assert np.array_equal(kq.bits(y1), kq.bits(y2))


def _fa_case(seed, H=8, H_kv=2, T=37, D=64, N=2, mask=True):
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
    d = oracle.FaDims(H=H, T=T, D=D, group=H // H_kv, tp=tp, k_row=H_kv * D // 2, k_head=D // 2,
                      v_row=H_kv * D // 2, v_head=D // 2, N=N, q_tok=H * D, q_head=D, m_row=tp // 2,
                      has_mask=int(mask), H_kv=H_kv)
    return q, k, v, m.view(np.uint16), d


def test_flash_attn_closed_form():
    q, k, v, m, d = _fa_case(41)
    out = np.zeros(d.N * d.H * d.D, np.float32)
    L.kco_flash_attn_f16(q, k, v, m, out, C.byref(d), 0.125)
    Q = q.reshape(d.N, d.H, d.D).astype(np.float64)
    K = k.view(np.float16).reshape(d.T, d.H_kv, d.D).astype(np.float64)
    V = v.view(np.float16).reshape(d.T, d.H_kv, d.D).astype(np.float64)
    M = m.view(np.float16).reshape(d.N, d.tp)[:, :d.T].astype(np.float64)
    want = np.zeros((d.N, d.H, d.D))
    for i in range(d.N):
        for h in range(d.H):
            s = K[:, h // d.group] @ Q[i, h] * 0.125 + M[i]
            p = np.exp(s - s.max())
            want[i, h] = p @ V[:, h // d.group] / p.sum()
    assert np.abs(out.reshape(want.shape) - want).max() < 1e-5


def test_flash_attn_matches_reference_bits(R):
    q, k, v, m, d = _fa_case(42)
    a = np.zeros(d.N * d.H * d.D, np.float32)
    b = np.zeros_like(a)
    L.kco_flash_attn_f16(q, k, v, m, a, C.byref(d), 0.1)
    dims = np.array([getattr(d, f) for f, _ in oracle.FaDims._fields_], np.int32)
    R.kcref_flash_attn_f16(q, k, v, m, b, dims, 0.1)
    assert np.array_equal(kq.bits(a), kq.bits(b))


# ---- fp16 weights (matmul_f16) ----------------------------------------------------------------

F16_SHAPES = [(8, 2, 1), (16, 64, 3), (24, 130, 5), (64, 512, 8)]


def _f16_case(rows, k, nc, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(rows * k) * 0.05).astype(np.float16).view(np.uint16)
    x = rng.standard_normal(nc * k).astype(np.float32)
    return w, x


@pytest.mark.parametrize("rows,k,nc", F16_SHAPES)
def test_matmul_f16_close_to_float64(rows, k, nc):
    """Against the float64 product of the same fp16 values (numpy's own binary16 decoding): an f32
    running sum of k terms stays within k * 2^-24 of the sum of absolute products."""
    w, x = _f16_case(rows, k, nc, 40 + k)
    got = oracle.matmul_f16(L, w, x, rows, k, nc).astype(np.float64)
    wd = w.view(np.float16).astype(np.float64).reshape(rows, k)
    xd = x.astype(np.float64).reshape(nc, k)
    want = xd @ wd.T
    bound = (np.abs(xd) @ np.abs(wd).T) * (k * 2.0 ** -24) + 1e-30
    assert np.all(np.abs(got - want) <= bound)
    # a transposed operand or a dropped odd term fails by far more than the bound
    assert not np.allclose(got, xd @ (wd * (np.arange(k) % 2 == 0)).T, rtol=1e-3)


@pytest.mark.parametrize("rows,k,nc", F16_SHAPES)
def test_matmul_f16_matches_reference_bits(rows, k, nc, R):
    w, x = _f16_case(rows, k, nc, 50 + rows)
    a = oracle.matmul_f16(L, w, x, rows, k, nc)
    b = oracle.matmul_f16(R, w, x, rows, k, nc)
    assert np.array_equal(kq.bits(a), kq.bits(b))


# ---- committed fixtures (made by tests/golden/make_golden.py from oracle/_ref) --------------------

def _golden_files():
    return sorted(glob.glob(os.path.join(GOLDEN, "*.npz")))


def test_golden_fixtures_present():
    assert len(_golden_files()) >= 4


@pytest.mark.parametrize("path", _golden_files(), ids=os.path.basename)
def test_oracle_matches_golden(path):
    g = np.load(path)
    kind = str(g["kind"])
    if kind == "matvec":
        qt, rows, k = str(g["qtype"]), int(g["rows"]), int(g["k"])
        xq, xd = oracle.quantize_q8x4(L, g["x"])
        assert np.array_equal(xq, g["xq"]) and np.array_equal(kq.bits(xd), kq.bits(g["xd"]))
        assert np.array_equal(kq.bits(oracle.matvec(L, qt, g["w"], xq, xd, rows, k)), kq.bits(g["y"]))
        slot = oracle.quantize_q8k(L, g["x"])
        assert np.array_equal(slot, g["slot"])
        assert np.array_equal(kq.bits(oracle.matvec_q8k(L, qt, g["w"], slot, rows, k)), kq.bits(g["yk"]))
        assert np.array_equal(kq.bits(oracle.dequant(L, qt, g["w"], rows, k).reshape(-1)), kq.bits(g["deq"]))
    elif kind == "f16":
        got = np.array([L.kco_f32_to_f16(float(v)) for v in g["x"]], np.uint16)
        assert np.array_equal(got, g["h"])
    elif kind == "attn":
        d = oracle.FaDims(*[int(v) for v in g["dims"]])
        out = np.zeros(d.N * d.H * d.D, np.float32)
        L.kco_flash_attn_f16(g["q"], g["k"], g["v"], g["m"], out, C.byref(d), float(g["scale"]))
        assert np.array_equal(kq.bits(out), kq.bits(g["out"]))
    elif kind == "norm":
        n, rows = int(g["n"]), int(g["rows"])
        q = np.zeros(rows * (n // 32) * 11, np.int32)
        out = np.zeros(n * rows, np.float32)
        L.kco_add_sumsq_f(g["a"], g["b"], out, q, n, rows)
        y = np.zeros(n * rows, np.float32)
        L.kco_norm_mul_q8(out, g["w"], y, q, n, rows, 1e-5)
        assert np.array_equal(q, g["q"]) and np.array_equal(kq.bits(y), kq.bits(g["y"]))
    elif kind == "matmul_f16":
        rows, k, nc = int(g["rows"]), int(g["k"]), int(g["ncols"])
        assert np.array_equal(kq.bits(oracle.matmul_f16(L, g["w"], g["x"], rows, k, nc)), kq.bits(g["y"]))
    else:
        pytest.fail(f"unknown fixture kind {kind}")
