"""Synthetic model weights of the BASELINE configurations, made on the device.

Every matrix is drawn from N(0, std) by the fill_normal_f32 kernel (a function of the seed, the
tensor and the index only) and quantized to its ggml type by quantize_kquant (ggml's reference
Q4_K / Q6_K quantizers, as the GGUF files the reference reads were made); norm weights are
1 + 0.1 * U(-1, 1) from numpy. The bytes come back to the host, where the model upload
(kcModelSetTensor) and any CPU check can read the same values. A 3B-shape model takes about a
second.
"""
from __future__ import annotations

import numpy as np

from . import (QTYPE, Buffer, FillNormalArgs, QuantizeKquantArgs, launch, repack, synchronize)

Q4K, Q6K, F32, F16 = 12, 14, 0, 1


def shapes(cfg):
    """tensor id -> (default qtype, rows, k): the table of kcModelTensorInfo."""
    E, Q, KV, F, V, hd = (cfg["n_embd"], cfg["n_head"] * cfg["head_dim"], cfg["n_head_kv"] * cfg["head_dim"],
                          cfg["n_ff"], cfg["n_vocab"], cfg["head_dim"])
    return {0: (Q4K, V, E), 1: (F32, 1, E), 2: (Q6K, V, E), 3: (F32, 1, E), 4: (Q4K, Q, E), 5: (Q4K, KV, E),
            6: (Q6K, KV, E), 7: (Q4K, E, Q), 8: (F32, 1, E), 9: (Q4K, F, E), 10: (Q4K, F, E), 11: (Q6K, E, F),
            12: (F32, 1, hd), 13: (F32, 1, hd)}


def tensor_keys(cfg):
    per_layer = [3, 4, 5, 6, 7, 8, 9, 10, 11] + ([12, 13] if cfg["qk_norm"] else [])
    return [(t, -1) for t in (0, 1, 2)] + [(t, l) for l in range(cfg["n_layer"]) for t in per_layer]


def _seed(seed, tid, layer):
    return (seed * 1_000_003 + tid * 10_007 + (layer + 1) * 101) & 0x7FFF_FFFF_FFFF_FFFF


def quantized_matrix(qtype, rows, k, seed, std=0.02, f32=None, blocks=None):
    """rows x k weights ~ N(0, std) quantized to qtype ("q4k" / "q6k") on the device: host uint8 blocks.
    f32 / blocks: optional device Buffers large enough to reuse."""
    n = rows * k
    nbytes = rows * (k // 256) * (144 if qtype == "q4k" else 210)
    own_f, own_b = f32 is None, blocks is None
    f32 = f32 or Buffer(n * 4)
    blocks = blocks or Buffer(nbytes)
    try:
        launch("fill_normal_f32", FillNormalArgs(f32.ptr, n, seed, 0.0, std))
        launch("quantize_kquant", QuantizeKquantArgs(f32.ptr, blocks.ptr, QTYPE[qtype], rows, k))
        synchronize()
        return blocks.download(np.uint8, nbytes)
    finally:
        if own_f:
            f32.free()
        if own_b:
            blocks.free()


def quantized_stream(qtype, rows, k, seed, std=0.02, f32=None, blocks=None):
    """The same matrix as quantized_matrix, left on the device as the repacked weight stream the
    kernels read (a new Buffer); nothing crosses to the host. f32 / blocks: optional device Buffers
    large enough to reuse."""
    n = rows * k
    own_f, own_b = f32 is None, blocks is None
    f32 = f32 or Buffer(n * 4)
    blocks = blocks or Buffer(rows * (k // 256) * (144 if qtype == "q4k" else 210))
    try:
        launch("fill_normal_f32", FillNormalArgs(f32.ptr, n, seed, 0.0, std))
        launch("quantize_kquant", QuantizeKquantArgs(f32.ptr, blocks.ptr, QTYPE[qtype], rows, k))
        return repack(qtype, blocks, rows, k)
    finally:
        synchronize()
        if own_f:
            f32.free()
        if own_b:
            blocks.free()


def model_weights(cfg, seed, std=0.02, types=None):
    """{(tensor id, layer): host array} for every tensor of cfg (layer -1 for the global ones), in
    the layout kcModelSetTensor takes: ggml blocks for the matrices, float32 for the norms.
    types[(id, layer)] may override a matrix's K-quant type (Q4K / Q6K)."""
    table = shapes(cfg)
    types = types or {}
    keys = tensor_keys(cfg)
    big = max(table[t][1] * table[t][2] for t, _ in keys if table[t][0] != F32)
    f32, blocks = Buffer(big * 4), Buffer(big // 256 * 210)
    rng = np.random.default_rng(seed)
    out = {}
    try:
        for tid, layer in keys:
            qt, rows, k = table[tid]
            qt = types.get((tid, layer), qt)
            if qt == F32:
                out[(tid, layer)] = (1.0 + 0.1 * rng.uniform(-1.0, 1.0, k)).astype(np.float32)
                continue
            out[(tid, layer)] = quantized_matrix("q6k" if qt == Q6K else "q4k", rows, k, _seed(seed, tid, layer), std,
                                                 f32, blocks)
    finally:
        f32.free()
        blocks.free()
    return out
