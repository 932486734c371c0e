"""The vectorised, threaded oracle forms (oracle/kc_oracle_simd.c) are bit-identical to the scalar
restatement (oracle/kc_oracle.c, itself bit-exact to the reference's llm_reference.cpp) at every
level the CPU offers: scalar, AVX2 (vpmaddubsw/vpmaddwd) and AVX-512 VNNI (vpdpbusd). Only the
integer dot products are vectorised; these tests would catch a lane mapped to the wrong sub-block,
a dropped lane or a signed/unsigned mix-up (the weight blocks are random bytes, the activations
span the full int8 range)."""
import ctypes as C

import numpy as np
import pytest

import oracle
from oracle import FaDims
from tests import kq

L = oracle.lib()
LEVELS = [lv for lv in (0, 1, 2) if lv <= L.kco_simd_level()]


@pytest.fixture(params=LEVELS, ids=["scalar", "avx2", "avx512vnni"][: len(LEVELS)])
def level(request):
    got = L.kco_simd_cap(request.param)
    assert got == request.param
    yield got
    L.kco_simd_cap(2)


def slots_k(x, k, ncols):
    q = np.zeros(ncols * (k // 256 * 85), np.int32)
    L.kco_quantize_cols_k(x, q, k, ncols)
    return q


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("rows,k,ncols", [(8, 256, 1), (40, 768, 5), (24, 3072, 17)])
def test_matmul_q8k_simd_bit_exact(level, qtype, rows, k, ncols):
    w = kq.random_blocks(qtype, rows, k, seed=rows + k)
    x = kq.uniform(ncols * k, 3, -4, 4)
    q = slots_k(x, k, ncols)
    want = np.zeros(rows * ncols, np.float32)
    getattr(L, f"kco_matmul_{qtype}_q8k")(w, q, want, rows, k, ncols)
    for threads in (1, 3):
        got = np.zeros(rows * ncols, np.float32)
        getattr(L, f"kco_matmul_{qtype}_q8k_simd")(w, q, got, rows, k, ncols, threads)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("qtype", ["q4k", "q6k"])
@pytest.mark.parametrize("rows,k", [(8, 256), (40, 768), (64, 4096)])
def test_matvec_q8_simd_bit_exact(level, qtype, rows, k):
    w = kq.random_blocks(qtype, rows, k, seed=rows * 3 + k)
    x = kq.uniform(k, 4, -5, 5)
    x[::37] = 0.0
    xq, xd = oracle.quantize_q8x4(L, x)
    want = oracle.matvec(L, qtype, w, xq, xd, rows, k)
    got = np.zeros(rows, np.float32)
    getattr(L, f"kco_matvec_{qtype}_q8_simd")(w, xq, xd, got, rows, k, 2)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_flash_attn_mt_bit_exact():
    rng = np.random.default_rng(5)
    H, Hkv, D, T, N = 8, 2, 64, 45, 5
    q = rng.standard_normal(N * H * D).astype(np.float32)
    k = rng.standard_normal(T * Hkv * D).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(T * Hkv * D).astype(np.float16).view(np.uint16)
    tp = (T + 7) // 8 * 8
    mask = np.zeros(N * tp, np.float16)
    for i in range(N):
        mask[i * tp + T - N + i + 1:(i + 1) * tp] = -np.inf
    d = FaDims(H=H, T=T, D=D, group=H // Hkv, tp=tp, k_row=Hkv * D // 2, k_head=D // 2, v_row=Hkv * D // 2,
               v_head=D // 2, N=N, q_tok=H * D, q_head=D, m_row=tp // 2, has_mask=1, H_kv=Hkv)
    want = np.zeros(N * H * D, np.float32)
    L.kco_flash_attn_f16(q, k, v, mask.view(np.uint16), want, C.byref(d), np.float32(0.125))
    for threads in (1, 4):
        got = np.zeros_like(want)
        L.kco_flash_attn_f16_mt(q, k, v, mask.view(np.uint16), got, C.byref(d), np.float32(0.125), threads)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
