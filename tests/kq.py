"""Input generators shared by the tests: random K-quant blocks and activations.

Blocks follow the reference tests (tests/test_llm_kernels.cpp:205-219): random bytes, with every
fp16 scale replaced by a positive value in [2^-9, 2^-6) so that outputs stay finite.
"""
import numpy as np

QK = 256
BLOCK_BYTES = {"q4k": 144, "q6k": 210}


def _half(rng, n):
    return (0x1800 + rng.integers(0, 0x0C00, size=n)).astype(np.uint16)


def random_blocks(qtype, rows, k, seed):
    rng = np.random.default_rng(seed)
    bb = BLOCK_BYTES[qtype]
    nblk = rows * (k // QK)
    b = rng.integers(0, 256, size=(nblk, bb), dtype=np.uint8)
    if qtype == "q4k":
        b[:, 0:2] = _half(rng, nblk).view(np.uint8).reshape(nblk, 2)
        b[:, 2:4] = _half(rng, nblk).view(np.uint8).reshape(nblk, 2)
    else:
        b[:, 208:210] = _half(rng, nblk).view(np.uint8).reshape(nblk, 2)
    return b.reshape(-1)


def randn(n, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(n) * scale).astype(np.float32)


def uniform(n, seed, lo=-1.0, hi=1.0):
    return np.random.default_rng(seed).uniform(lo, hi, n).astype(np.float32)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def rel_diff(a, b):
    """max |a - b| / max |b| (tests/test_llm_kernels.cpp:53-63)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    if not np.all(np.isfinite(a)):
        return np.inf
    scale = np.abs(b).max()
    m = np.abs(a - b).max()
    return m / scale if scale > 0 else m
