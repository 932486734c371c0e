"""Random-init model weights shared by the model tests and the bench: ggml K-quant blocks with
bounded fp16 scales (the reference tests' generator, tests/test_llm_kernels.cpp:205-219) and norm
weights near 1. Returns {(tensor_id, layer): array} in the layout kcModelSetTensor expects."""
import numpy as np

from oracle.model import F16, F32, Q6K, shapes


def random_weights(cfg, seed, types=None):
    """types[(id, layer)] = Q4K / Q6K / F16 overrides a matrix's default type (F16: row-major
    halves ~ N(0, 0.02), as uint8 bytes)."""
    rng = np.random.default_rng(seed)
    out = {}
    table = shapes(cfg)
    types = types or {}
    ids_global = [0, 1, 2]
    ids_layer = [3, 4, 5, 6, 7, 8, 9, 10, 11] + ([12, 13] if cfg["qk_norm"] else [])
    keys = [(t, -1) for t in ids_global] + [(t, l) for l in range(cfg["n_layer"]) for t in ids_layer]
    for tid, layer in keys:
        qt, rows, k = table[tid]
        qt = types.get((tid, layer), qt)
        if qt == F32:
            out[(tid, layer)] = rng.uniform(0.8, 1.2, k).astype(np.float32)
            continue
        if qt == F16:
            out[(tid, layer)] = (rng.standard_normal(rows * k) * 0.02).astype(np.float16).view(np.uint8)
            continue
        bb = 210 if qt == Q6K else 144
        n = rows * (k // 256)
        b = rng.integers(0, 256, size=(n, bb), dtype=np.uint8)
        half = lambda: (0x1800 + rng.integers(0, 0x0C00, size=n)).astype(np.uint16).view(np.uint8).reshape(n, 2)
        if qt == Q6K:
            b[:, 208:210] = half()
        else:
            b[:, 0:2] = half()
            b[:, 2:4] = half()
        out[(tid, layer)] = b.reshape(-1)
    return out


def quantized_weights(cfg, seed, types=None, std=0.02):
    """The configs' workload: every matrix drawn from N(0, std) and quantized to its ggml type
    with the restated ggml reference quantizer (oracle.quantize_weights); norm weights
    1 + 0.1 * U(-1, 1); F16 overrides keep the N(0, std) values as halves."""
    import oracle

    L = oracle.lib()
    rng = np.random.default_rng(seed)
    out = {}
    table = shapes(cfg)
    types = types or {}
    ids_global = [0, 1, 2]
    ids_layer = [3, 4, 5, 6, 7, 8, 9, 10, 11] + ([12, 13] if cfg["qk_norm"] else [])
    keys = [(t, -1) for t in ids_global] + [(t, l) for l in range(cfg["n_layer"]) for t in ids_layer]
    for tid, layer in keys:
        qt, rows, k = table[tid]
        qt = types.get((tid, layer), qt)
        if qt == F32:
            out[(tid, layer)] = (1.0 + 0.1 * rng.uniform(-1.0, 1.0, k)).astype(np.float32)
            continue
        x = (rng.standard_normal(rows * k, dtype=np.float32) * std).astype(np.float32)
        if qt == F16:
            out[(tid, layer)] = x.astype(np.float16).view(np.uint8)
            continue
        out[(tid, layer)] = oracle.quantize_weights(L, "q6k" if qt == Q6K else "q4k", x, rows, k)
    return out
