"""ctypes bindings for the CPU oracle (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package: it is
the checker, never the thing measured or shipped. ``lib()`` is the from-scratch C restatement
(oracle/kc_oracle.c); ``ref()`` is the reference's own llm/llm_reference.cpp built into
oracle/_ref (None when it was not built).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i = C.c_int
_f = C.c_float


class FaDims(C.Structure):
    """FaDims field order of llm/llm_kernels.hpp:316-332."""
    _fields_ = [(n, C.c_int) for n in (
        "H", "T", "D", "group", "tp", "k_row", "k_head", "v_row", "v_head", "N", "q_tok", "q_head", "m_row",
        "has_mask", "H_kv")]


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _sig(lib, prefix):
    def s(name, res, *args):
        fn = getattr(lib, prefix + name)
        fn.restype = res
        fn.argtypes = list(args)
    s("f16_to_f32", _f, C.c_uint16)
    s("f32_to_f16", C.c_uint16, _f)
    s("dequant_row_q4k", None, _u8p, _i, _f32p)
    s("dequant_row_q6k", None, _u8p, _i, _f32p)
    s("quantize_q8x4", None, _f32p, _i32p, _f32p, _i)
    s("quantize_q8k", None, _f32p, _i32p, _i)
    for q in ("q4k", "q6k"):
        s(f"matvec_{q}_q8", None, _u8p, _i32p, _f32p, _f32p, _i, _i)
        s(f"matvec_{q}_q8k", None, _u8p, _i32p, _f32p, _i, _i)
    s("rms_norm", None, _f32p, _f32p, _f32p, _i, _i, _f)
    s("mul_rows", None, _f32p, _f32p, _f32p, _i, _i)
    s("silu_mul", None, _f32p, _f32p, _f32p, _i)
    s("rope_ggml", None, _f32p, _f32p, _i32p, _f32p, _i, _i, _i, _f, _i)
    s("add_sumsq_f", None, _f32p, _f32p, _f32p, _i32p, _i, _i)
    s("sumsq_part", None, _f32p, _i32p, _i, _i)
    s("norm_mul_q8", None, _f32p, _f32p, _f32p, _i32p, _i, _i, _f)
    s("norm_mul_q8k", None, _f32p, _f32p, _f32p, _i32p, _i32p, _i, _i, _f)
    s("silu_mul_q8f", None, _f32p, _f32p, _f32p, _i32p, _i, _i)
    s("silu_mul_q8k", None, _f32p, _f32p, _f32p, _i32p, _i, _i)
    s("set_rows_f16", None, _f32p, _i64p, _u16p, _i, _i, _i, _i, _i)
    s("matmul_f16", None, _u16p, _f32p, _f32p, _i, _i, _i)


def lib():
    """The C restatement (oracle/liboracle.so), built on first use if missing."""
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = C.CDLL(path)
        _sig(L, "kco_")
        L.kco_rope_ggml_turns.restype = None
        L.kco_rope_ggml_turns.argtypes = [_f32p, _f32p, _i32p, _f32p, _i, _i, _i, _f, _i]
        L.kco_quantize_cols.argtypes = [_f32p, _i32p, _i, _i]
        L.kco_quantize_cols_k.argtypes = [_f32p, _i32p, _i, _i]
        for q in ("q4k", "q6k"):
            for a in ("q8", "q8k"):
                getattr(L, f"kco_matmul_{q}_{a}").argtypes = [_u8p, _i32p, _f32p, _i, _i, _i]
        L.kco_flash_attn_f16.argtypes = [_f32p, _u16p, _u16p, _u16p, _f32p, C.POINTER(FaDims), _f]
        L.kco_add.argtypes = [_f32p, _f32p, _f32p, _i]
        for q in ("q4k", "q6k"):
            getattr(L, f"kco_matvec_{q}_q8_mt").argtypes = [_u8p, _i32p, _f32p, _f32p, _i, _i, _i]
        L.kco_matmul_q4k_q8k_mt.argtypes = [_u8p, _i32p, _f32p, _i, _i, _i, _i]
        L.kco_max_threads.restype = _i
        L.kco_simd_level.restype = _i
        L.kco_simd_cap.restype = _i
        L.kco_simd_cap.argtypes = [_i]
        for q in ("q4k", "q6k"):
            getattr(L, f"kco_matmul_{q}_q8k_simd").argtypes = [_u8p, _i32p, _f32p, _i, _i, _i, _i]
            getattr(L, f"kco_matvec_{q}_q8_simd").argtypes = [_u8p, _i32p, _f32p, _f32p, _i, _i, _i]
        L.kco_flash_attn_f16_mt.argtypes = [_f32p, _u16p, _u16p, _u16p, _f32p, C.POINTER(FaDims), _f, _i]
        L.kco_f32_to_f16_rne.restype = C.c_uint16
        L.kco_f32_to_f16_rne.argtypes = [_f]
        for q in ("q4k", "q6k"):
            getattr(L, f"kco_quantize_row_{q}").argtypes = [_f32p, _u8p, _i]
            getattr(L, f"kco_quantize_{q}_mt").argtypes = [_f32p, _u8p, _i, _i, _i]
        _LIB = L
    return _LIB


def ref():
    """The reference's own llm_reference.cpp (oracle/_ref/libkcref.so), or None if not built."""
    global _REF
    if _REF is None:
        path = os.path.join(HERE, "_ref", "libkcref.so")
        if not os.path.exists(path):
            return None
        R = C.CDLL(path)
        _sig(R, "kcref_")
        R.kcref_repack_q4k.argtypes = [_u8p, _i, _i, _i32p]
        R.kcref_repack_q6k.argtypes = [_u8p, _i, _i, _i32p]
        R.kcref_flash_attn_f16.argtypes = [_f32p, _u16p, _u16p, _u16p, _f32p, _i32p, _f]
        _REF = R
    return _REF


# ---- numpy conveniences over either library (prefix "kco_" or "kcref_") -----------------

def _fn(L, name):
    return getattr(L, ("kco_" if L is _LIB else "kcref_") + name)


def quantize_q8x4(L, x):
    x = np.ascontiguousarray(x, np.float32)
    nb = x.size // 32
    xq = np.zeros(nb * 8, np.int32)
    xd = np.zeros(nb * 2, np.float32)
    _fn(L, "quantize_q8x4")(x, xq, xd, nb)
    return xq, xd


def quantize_q8k(L, x):
    x = np.ascontiguousarray(x, np.float32)
    nsb = x.size // 256
    q = np.zeros(nsb * 85, np.int32)
    _fn(L, "quantize_q8k")(x, q, nsb)
    return q


def matvec(L, qtype, w, xq, xd, rows, k):
    y = np.zeros(rows, np.float32)
    _fn(L, f"matvec_{qtype}_q8")(np.ascontiguousarray(w, np.uint8), xq, xd, y, rows, k)
    return y


def matvec_q8k(L, qtype, w, slot, rows, k):
    y = np.zeros(rows, np.float32)
    _fn(L, f"matvec_{qtype}_q8k")(np.ascontiguousarray(w, np.uint8), slot, y, rows, k)
    return y


def dequant(L, qtype, w, rows, k):
    bb = 144 if qtype == "q4k" else 210
    w = np.ascontiguousarray(w, np.uint8).reshape(rows, k // 256 * bb)
    out = np.zeros((rows, k), np.float32)
    for r in range(rows):
        row = np.zeros(k, np.float32)
        _fn(L, f"dequant_row_{qtype}")(np.ascontiguousarray(w[r]), k, row)
        out[r] = row
    return out


def quantize_weights(L, qtype, x, rows, k, threads=0):
    """rows x k floats -> ggml blocks (uint8, rows * k/256 * 144 or 210 bytes) with the restated
    ggml reference quantizer."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.zeros(rows * (k // 256) * (144 if qtype == "q4k" else 210), np.uint8)
    getattr(L, f"kco_quantize_{qtype}_mt")(x, out, rows, k, threads or L.kco_max_threads())
    return out


def matmul_f16(L, w, x, rows, k, ncols):
    """Y [ncols][rows] = W X for row-major fp16 weights (uint16 bits) and ncols columns of k floats."""
    y = np.zeros(rows * ncols, np.float32)
    _fn(L, "matmul_f16")(np.ascontiguousarray(w, np.uint16).reshape(-1), np.ascontiguousarray(x, np.float32).reshape(-1),
                         y, rows, k, ncols)
    return y.reshape(ncols, rows)
