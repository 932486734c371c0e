"""Writes the golden fixtures in tests/golden/ from the reference's own C++ mirror.

Run in the build container, where oracle/_ref/libkcref.so is compiled from
/root/reference/llm/llm_reference.cpp (oracle/Makefile): `python tests/golden/make_golden.py`.
Every output below is computed by the reference's code (kcref_*); the inputs are seeded.
The fixtures are data only (inputs and expected outputs), a few tens of KB in total.
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from tests import kq  # noqa: E402


def matvec_case(R, qtype, rows, k, seed):
    w = kq.random_blocks(qtype, rows, k, seed)
    x = kq.uniform(k, seed + 1, -3, 3)
    xq, xd = oracle.quantize_q8x4(R, x)
    slot = oracle.quantize_q8k(R, x)
    np.savez_compressed(
        os.path.join(HERE, f"matvec_{qtype}_{rows}x{k}.npz"), kind="matvec", qtype=qtype, rows=rows, k=k, w=w, x=x,
        xq=xq, xd=xd, y=oracle.matvec(R, qtype, w, xq, xd, rows, k), slot=slot,
        yk=oracle.matvec_q8k(R, qtype, w, slot, rows, k), deq=oracle.dequant(R, qtype, w, rows, k).reshape(-1))


def main():
    R = oracle.ref()
    if R is None:
        sys.exit("oracle/_ref/libkcref.so is not built: run make -C oracle in the build container")
    matvec_case(R, "q4k", 8, 256, 100)
    matvec_case(R, "q4k", 40, 768, 101)
    matvec_case(R, "q6k", 8, 256, 102)
    matvec_case(R, "q6k", 40, 768, 103)
    x = np.concatenate([kq.randn(2000, 104, 1000.0), kq.randn(500, 105, 1e-6),
                        np.array([0.0, -0.0, 65519.0, 65520.0, -7e4, 6.1e-5], np.float32)])
    np.savez_compressed(os.path.join(HERE, "f32_to_f16.npz"), kind="f16", x=x,
                        h=np.array([R.kcref_f32_to_f16(float(v)) for v in x], np.uint16))
    # attention over an fp16 cache with a causal mask
    rng = np.random.default_rng(106)
    H, H_kv, T, D, N = 8, 2, 29, 64, 2
    tp = (T + 7) // 8 * 8
    q = rng.standard_normal(N * H * D).astype(np.float32)
    k = rng.standard_normal(T * H_kv * D).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(T * H_kv * D).astype(np.float16).view(np.uint16)
    m = np.full(N * tp, -np.inf, np.float16)
    for i in range(N):
        m[i * tp:i * tp + T - N + 1 + i] = 0
    m = m.view(np.uint16)
    dims = np.array([H, T, D, H // H_kv, tp, H_kv * D // 2, D // 2, H_kv * D // 2, D // 2, N, H * D, D, tp // 2, 1,
                     H_kv], np.int32)
    out = np.zeros(N * H * D, np.float32)
    R.kcref_flash_attn_f16(q, k, v, m, out, dims, 0.125)
    np.savez_compressed(os.path.join(HERE, "flash_attn_f16.npz"), kind="attn", q=q, k=k, v=v, m=m, dims=dims,
                        scale=np.float32(0.125), out=out)
    # residual add + RMS norm + per-32 quantization
    n, rows = 512, 2
    a, b, w = kq.randn(n * rows, 107), kq.randn(n * rows, 108), kq.uniform(n, 109, 0.5, 1.5)
    qs = np.zeros(rows * (n // 32) * 11, np.int32)
    s = np.zeros(n * rows, np.float32)
    R.kcref_add_sumsq_f(a, b, s, qs, n, rows)
    y = np.zeros(n * rows, np.float32)
    R.kcref_norm_mul_q8(s, w, y, qs, n, rows, np.float32(1e-5))
    np.savez_compressed(os.path.join(HERE, "norm_mul_q8.npz"), kind="norm", n=n, rows=rows, a=a, b=b, w=w, q=qs, y=y)
    # fp16 weights x fp32 activations (matmul_f16), 24 rows x 96 values x 3 columns
    rows, k, nc = 24, 96, 3
    wf = (kq.randn(rows * k, 110) * np.float32(0.05)).astype(np.float16).view(np.uint16)
    xf = kq.randn(nc * k, 111)
    np.savez_compressed(os.path.join(HERE, "matmul_f16.npz"), kind="matmul_f16", rows=rows, k=k, ncols=nc, w=wf, x=xf,
                        y=oracle.matmul_f16(R, wf, xf, rows, k, nc))
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
